"""GPU parity of the RMSNorm kernel (tg_hip_rms_norm_dev; tg_rms_norm,
csrc/libtinygiant.c:680-698): y = (x * (1/sqrt(mean(x^2) + eps))) * w per
row.  The GPU sums x^2 in its own order, so the bar is <= 2e-6 of max|y|
(the decode step's RMSNorm stage bar); widths cover one partial 256-block,
widths that are not multiples of 4, the model widths and the 16384 limit,
which is also the largest width accepted."""

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _run(tg, x, w, eps):
    lib = tg.lib()
    rows, n = x.shape
    xd, yd = tg.DeviceArray(x.nbytes), tg.DeviceArray(x.nbytes)
    xd.upload(x)
    wd = None
    if w is not None:
        wd = tg.DeviceArray(w.nbytes)
        wd.upload(w)
    lib.tg_hip_rms_norm_dev(xd.ptr, wd.ptr if wd else None, yd.ptr, rows, n, eps, None)
    lib.tg_hip_synchronize()
    return yd.download(np.float32, rows * n).reshape(rows, n)


@pytest.mark.parametrize("n,rows,weighted", [(100, 3, True), (257, 2, False), (2048, 4, True), (2880, 2, True),
                                             (4099, 1, True), (16384, 2, True)])
def test_rms_norm_dev_vs_oracle(tg, orc, n, rows, weighted):
    say("rms_norm", n, rows, weighted)
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
    x[0, : n // 3] = 0
    w = rng.uniform(0.5, 1.5, n).astype(np.float32) if weighted else None
    got = _run(tg, x, w, 1e-6)
    for r in range(rows):
        ref = orc.rms_norm(x[r], w if weighted else np.ones(n, np.float32), 1e-6)
        assert np.abs(got[r] - ref).max() <= 2e-6 * np.abs(ref).max(), r


def test_rms_norm_dev_rejects_wider_rows(tg):
    lib = tg.lib()
    lib.tg_hip_clear_error()
    lib.tg_hip_rms_norm_dev(None, None, None, 1, 16385, 1e-6, None)
    assert "16384" in tg.last_error()
