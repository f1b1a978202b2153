"""GPU parity of the device router (tg_hip_route_dev) against the oracle's
restatement of Router.logits/_topk/_weights (tinygiant/router.py:29-42).

Bars: the selected experts and their order equal the oracle's unless two
logits at the selection boundary (or adjacent in the order) are closer than
1e-5 of the logit scale (f32 summation order differs); weights within 2e-6
absolute (exp and the sum are float32, the sum grouped as numpy groups it).
"""

import ctypes
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _route(tg, router, bias, x, top_k, resident=None):
    lib = tg.lib()
    k, dim = x.shape
    n_exp = router.shape[0]
    arrs = []

    def dev(a):
        d = tg.DeviceArray(a.nbytes)
        d.upload(np.ascontiguousarray(a))
        arrs.append(d)
        return d

    rd, xd = dev(router), dev(x)
    bd = dev(bias) if bias is not None else None
    idx = tg.DeviceArray(k * top_k * 4)
    w = tg.DeviceArray(k * top_k * 4)
    sc = tg.DeviceArray(lib.tg_hip_route_scratch_bytes(k, n_exp))
    lib.tg_hip_clear_error()
    if resident is None:
        lib.tg_hip_route_dev(rd.ptr, bd.ptr if bd else None, xd.ptr, k, n_exp, dim, top_k, idx.ptr, w.ptr, sc.ptr,
                             None)
    else:
        md = dev(np.asarray(resident, np.uint8))
        lib.tg_hip_route_restricted_dev(rd.ptr, bd.ptr if bd else None, xd.ptr, k, n_exp, dim, top_k, md.ptr, idx.ptr,
                                        w.ptr, sc.ptr, None)
    lib.tg_hip_synchronize()
    assert tg.last_error() == "", tg.last_error()
    gi = idx.download(np.int32, k * top_k).reshape(k, top_k)
    gw = w.download(np.float32, k * top_k).reshape(k, top_k)
    for a in arrs + [idx, w, sc]:
        a.free()
    return gi, gw


@pytest.mark.parametrize("n_exp,dim,top_k,k", [(128, 2048, 8, 1), (128, 2048, 8, 9), (128, 2880, 4, 5),
                                              (64, 512, 16, 3), (200, 256, 6, 2)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_route_matches_oracle(tg, orc, n_exp, dim, top_k, k, with_bias):
    say(f"route n={n_exp} dim={dim} top_k={top_k} k={k} bias={with_bias}")
    rng = np.random.default_rng(n_exp + dim + k)
    router = (rng.standard_normal((n_exp, dim)) * 0.05).astype(np.float32)
    bias = (rng.standard_normal(n_exp) * 0.1).astype(np.float32) if with_bias else None
    x = rng.standard_normal((k, dim)).astype(np.float32)
    gi, gw = _route(tg, router, bias, x, top_k)
    for j in range(k):
        logits, idx, w = orc.route(router, bias, x[j], top_k)
        tol = 1e-5 * np.abs(logits).max()
        if list(gi[j]) != list(idx):
            order = np.sort(logits)[::-1]
            gaps = np.abs(np.diff(order[:top_k + 1]))
            assert gaps.min() <= tol, (j, list(gi[j]), list(idx))
            continue
        assert np.abs(gw[j] - w).max() <= 2e-6, (j, gw[j], w)
        assert abs(float(gw[j].sum()) - 1.0) <= 1e-6


@pytest.mark.parametrize("n_res", [64, 9, 8, 3])
def test_route_restricted_matches_oracle(tg, orc, n_res):
    """A draft pass's routing (Router.select(restrict=True),
    tinygiant/router.py:46-54) over 128 experts of which n_res are resident:
    the same bars as above, against the oracle's restricted selection (3
    resident experts: fewer than top_k, the unrestricted selection)."""
    n_exp, dim, top_k, k = 128, 2048, 8, 5
    say(f"route restricted n_res={n_res}")
    rng = np.random.default_rng(700 + n_res)
    router = (rng.standard_normal((n_exp, dim)) * 0.05).astype(np.float32)
    bias = (rng.standard_normal(n_exp) * 0.1).astype(np.float32)
    resident = np.zeros(n_exp, bool)
    resident[rng.choice(n_exp, n_res, replace=False)] = True
    x = rng.standard_normal((k, dim)).astype(np.float32)
    gi, gw = _route(tg, router, bias, x, top_k, resident=resident)
    for j in range(k):
        logits, idx, w = orc.route(router, bias, x[j], top_k, resident=resident)
        if n_res >= top_k:
            assert all(resident[e] for e in gi[j]), (j, list(gi[j]))
        tol = 1e-5 * np.abs(logits).max()
        if list(gi[j]) != list(idx):
            pool = logits[resident] if n_res >= top_k else logits
            order = np.sort(pool)[::-1]
            gaps = np.abs(np.diff(order[:top_k + 1]))
            assert gaps.min() <= tol, (j, list(gi[j]), list(idx))
            continue
        assert np.abs(gw[j] - w).max() <= 2e-6, (j, gw[j], w)
