"""GPU check of tg_hip_matmul_dev_noalloc, the entry point that allocates
nothing (its q8 scratch is the library's fixed device array), against
tg_hip_matmul_dev with a caller workspace: two calls in a row, the second
with a smaller input, must give the same bits (the same kernels run on the
same inputs; only the scratch address differs).  Also: shapes past the fixed
scratch are refused with an error and leave the outputs untouched."""

import ctypes
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _case(tg, fmt, nrows, ncols, k, seed):
    import tinygiant_amd.synth as S
    lib = tg.lib()
    rng = np.random.default_rng(seed)
    nbytes = nrows * lib.tg_row_bytes(fmt, ncols)
    mat = tg.DeviceArray(nbytes)
    if fmt == 1:   # F16 rows: finite values (random bytes would include inf and NaN patterns)
        mat.upload((rng.standard_normal(nrows * ncols) * 0.05).astype(np.float16))
    else:
        lib.tg_hip_synth_fill(fmt, S.tensor_seed(seed, 0, 0, 0), mat.ptr, nbytes, None)
    bias = tg.DeviceArray(nrows * 4)
    bias.upload(rng.standard_normal(nrows).astype(np.float32))
    x = tg.DeviceArray(k * ncols * 4)
    x.upload(rng.standard_normal((k, ncols)).astype(np.float32))
    return mat, bias, x


@pytest.mark.parametrize("fmt,ncols", [(0, 2048), (2, 768), (3, 2880), (4, 2880), (1, 1024)])
def test_noalloc_matches_workspace_entry(tg, fmt, ncols):
    lib = tg.lib()
    lib.tg_hip_init()
    nrows = 300
    for k, seed in ((6, 11), (2, 12)):   # the second call is smaller
        say(f"noalloc fmt={fmt} ncols={ncols} k={k}")
        mat, bias, x = _case(tg, fmt, nrows, ncols, k, seed + fmt)
        ref = tg.DeviceArray(k * nrows * 4)
        got = tg.DeviceArray(k * nrows * 4)
        ws = tg.DeviceArray(lib.tg_hip_matmul_scratch_bytes(k, ncols))
        lib.tg_hip_matmul_dev(fmt, mat.ptr, bias.ptr, x.ptr, ref.ptr, nrows, ncols, k, ws.ptr, None)
        lib.tg_hip_matmul_dev_noalloc(fmt, mat.ptr, bias.ptr, x.ptr, got.ptr, nrows, ncols, k, None)
        lib.tg_hip_synchronize()
        assert not lib.tg_hip_last_error(), tg.last_error()
        a = ref.download(np.float32, k * nrows)
        b = got.download(np.float32, k * nrows)
        assert np.all(np.isfinite(a))
        assert a.tobytes() == b.tobytes()
        for arr in (mat, bias, x, ref, got, ws):
            arr.free()


def test_noalloc_refuses_oversize(tg):
    lib = tg.lib()
    lib.tg_hip_init()
    cap = lib.tg_hip_matmul_noalloc_max_bytes()
    ncols = 4096
    per_row = lib.tg_hip_matmul_scratch_bytes(1, ncols)
    k = cap // per_row + 1
    assert lib.tg_hip_matmul_scratch_bytes(k, ncols) > cap
    say(f"noalloc oversize k={k}")
    mat, bias, x = _case(tg, 0, 8, ncols, k, 5)
    out = tg.DeviceArray(k * 8 * 4)
    sentinel = np.full(k * 8, 7.0, np.float32)
    out.upload(sentinel)
    lib.tg_hip_clear_error()
    lib.tg_hip_matmul_dev_noalloc(0, mat.ptr, bias.ptr, x.ptr, out.ptr, 8, ncols, k, None)
    lib.tg_hip_synchronize()
    assert b"scratch" in (lib.tg_hip_last_error() or b"")
    lib.tg_hip_clear_error()
    assert np.array_equal(out.download(np.float32, k * 8), sentinel)
    for arr in (mat, bias, x, out):
        arr.free()
