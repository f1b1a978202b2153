"""GPU parity of the MXFP4 scale byte's edge cases (e8m0_to_fp32_half,
csrc/libtinygiant.c:516-519: e < 2 takes the denormal branch
0x00200000 << e, i.e. 2^-128 and 2^-127; otherwise 2^(e-128), so 254 gives
2^126 and 255 gives 2^127).

Every synthetic MXFP4 tensor elsewhere draws e from 118-130, so these cases
build rows by hand:
  * matmul (k_gemv, the v_dot4 path): rows whose every block has e in {0, 1}
    (outputs near 1e-34: a path that flushed the denormal scale, or read
    e = 0 as 2^-127, is off by 100%), and rows with one block at e = 254 or
    255 holding a single unit code against x = 1 (outputs 2^126, 2^127);
    x is integer-valued with amax 127 so every q8 scale is 1 and each block
    term is an exact f32 product;
  * the MoE phases -- per-pair, expert-major and the block-scaled MFMA
    phases: one expert whose gate and up rows are all e in {0, 1}, so its
    hidden rows are of order 1e-34 and the per-row bars pin the branch;
  * e = 255 where the block-scaled MFMA phases would run: the OCP MX format
    reads that byte as NaN, and the hardware does, so a layer whose active
    MXFP4 matrices hold one runs the v_dot4 phases instead (the library scans
    the scale bytes: per call for staged weights, once per registered range
    or plan); the results equal the oracle's 2^127 arithmetic on the host
    call and on a plan, and the persistent gpt-oss step, which has no v_dot4
    form, refuses such a layer.
"""

import sys

import numpy as np
import pytest

import oracle as O
from tests.test_gpu_parity import close

pytestmark = pytest.mark.gpu
RB = 17


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _mx_rows(rng, nrows, ncols, e_choices):
    m = rng.integers(0, 256, nrows * ncols // 32 * RB, dtype=np.uint8).reshape(nrows, ncols // 32, RB)
    m[:, :, 0] = rng.choice(e_choices, (nrows, ncols // 32))
    return m


def _int_x(rng, ncols):
    x = rng.integers(-40, 41, ncols).astype(np.float32)
    x[::256] = 127.0           # amax 127 in every q8 block: scale 1, q == x
    return x


def test_matmul_e8m0_denormal_and_top_exponents(tg, orc):
    rng = np.random.default_rng(255)
    ncols = 2880
    nb = ncols // 32
    x = _int_x(rng, ncols)
    x[1] = 1.0                 # the unit operand of the single-code blocks below
    rows = []
    # rows 0-31: every block e in {0, 1}
    rows.append(_mx_rows(rng, 32, ncols, [0, 1]))
    # rows 32-47: e in {0, 1, 2, 3} mixed with normal exponents
    rows.append(_mx_rows(rng, 16, ncols, [0, 1, 2, 3, 120, 127, 128]))
    # rows 48-55: block 0 at e = 254 (rows 48-51) or 255 (rows 52-55) holding one
    # code 1 (kvalue 1) in value slot 1, i.e. times x[1] = 1; other blocks e = 0
    big = _mx_rows(rng, 8, ncols, [0])
    big[:, 0, 1:] = 0           # code bytes of block 0: every value kvalue[0] = 0 ...
    big[:, 0, 2] = 0x01         # ... but value 1 (low nibble of code byte 1): kvalue[1] = 1
    big[:4, 0, 0] = 254
    big[4:, 0, 0] = 255
    rows.append(big)
    mat = np.concatenate(rows).reshape(-1)
    nrows = 56
    got = tg.matmul(O.FMT_MXFP4, mat, None, x, nrows, ncols)
    ref = orc.matmul(O.FMT_MXFP4, mat, None, x, nrows, ncols)
    assert np.all(np.isfinite(ref)) and np.all(np.isfinite(got)), (got[48:], ref[48:])
    # exact expectations for the top exponents: 2^126 (resp. 2^127) * x[1] + the e = 0 rest
    assert abs(ref[48] / 2.0 ** 126 - 1) < 1e-6 and abs(ref[52] / 2.0 ** 127 - 1) < 1e-6
    for lo, hi in ((0, 32), (32, 48), (48, 56)):
        for r in range(lo, hi):
            ok = abs(float(got[r]) - float(ref[r])) <= 1e-5 * max(abs(float(ref[r])), 1e-37)
            assert ok, (r, got[r], ref[r])
    # the all-denormal-scale rows are of order 1e-34, not flushed
    assert np.all(np.abs(ref[:32]) > 1e-38) and np.all(np.abs(got[:32]) > 1e-38)
    say(f"  e in {{0,1}} rows: |out| ~ {np.abs(ref[:32]).mean():.2e}; e=254/255 rows {ref[48]:.3e} {ref[52]:.3e}")


def _moe_case(rng, n, D, I, k):
    """MXFP4 experts of D x I: every block of expert 0's gate rows and of
    expert 1's up rows has e in {0, 1} (so their hidden values, silu(g) * u,
    are of order 1e-34); all other exponents are normal.  Experts 0 and 1
    serve every row."""
    normal = list(range(118, 131))
    g, u, d = [], [], []
    for e in range(n):
        g.append(_mx_rows(rng, I, D, [0, 1] if e == 0 else normal).reshape(-1))
        u.append(_mx_rows(rng, I, D, [0, 1] if e == 1 else normal).reshape(-1))
        d.append(_mx_rows(rng, D, I, normal).reshape(-1))
    rw = np.zeros((n, k), np.float32)
    rw[0] = 0.5
    rw[1] = 0.3
    for r in range(k):
        rw[2 + r % (n - 2), r] = 0.2
    x = rng.uniform(-1, 1, (k, D)).astype(np.float32)
    return g, u, d, rw, x


@pytest.mark.parametrize("path", ["per-pair", "expert-major", "mfma"])
def test_moe_e8m0_denormal_expert(tg, orc, path):
    rng = np.random.default_rng(7 + len(path))
    n, D, I = 4, 1024, 1024
    k = 12 if path == "mfma" else 3
    g, u, d, rw, x = _moe_case(rng, n, D, I, k)
    fm = [O.FMT_MXFP4] * n
    lib = tg.lib()
    P = int(np.count_nonzero(rw))
    if path == "mfma":
        assert int(np.count_nonzero(rw, axis=1).max()) >= 4
    prev_g = lib.tg_hip_set_moe_grouped_min_rows(1 if path == "mfma" else 0)
    prev_e = lib.tg_hip_set_moe_expert_major(0 if path == "per-pair" else 1)
    try:
        h_gpu = np.zeros((P, I), np.float32)
        got = tg.moe_forward_rows_v2(g, u, d, O.FMT_MXFP4, fm, None, None, None, O.ACT_SILU, rw, x,
                                     np.zeros((k, D), np.float32), I, hidden_out=h_gpu)
    finally:
        lib.tg_hip_set_moe_grouped_min_rows(prev_g)
        lib.tg_hip_set_moe_expert_major(prev_e)
    h_ref = np.zeros((P, I), np.float32)
    orc.moe_v2(g, u, d, O.FMT_MXFP4, fm, None, None, None, O.ACT_SILU, rw, x, np.zeros((k, D), np.float32), I,
               hidden_out=h_ref)
    tiny = np.abs(h_ref[:2 * k]).max(axis=1)   # pairs of experts 0 and 1 come first
    say(f"  {path}: experts 0-1 hidden |max| {tiny.min():.2e} .. {tiny.max():.2e}, pairs {P}")
    assert np.all(tiny > 0) and np.all(tiny < 1e-30)
    for p in range(P):
        ok, rel = close(h_gpu[p], h_ref[p], tol=1e-4)
        assert ok, (path, "hidden", p, rel)
    ref_b = orc.moe_v2(g, u, d, O.FMT_MXFP4, fm, None, None, None, O.ACT_SILU, rw, x, np.zeros((k, D), np.float32),
                       I, hidden_in=h_gpu)
    ok, rel = close(got, ref_b)
    assert ok, (path, "down+combine", rel)


def _e255_case(rng, n=2, D=1024, I=1024):
    g, u, d = [], [], []
    for e in range(n):
        g.append(_mx_rows(rng, I, D, list(range(118, 131))).reshape(I, D // 32, RB))
        u.append(_mx_rows(rng, I, D, list(range(118, 131))).reshape(-1))
        d.append(_mx_rows(rng, D, I, list(range(118, 131))).reshape(-1))
    g[0][5, 3, 0] = 255          # gate row 5 of expert 0, block 3
    return [a.reshape(-1) for a in g], u, d


@pytest.mark.parametrize("registered", [False, True])
def test_moe_e8m0_255_takes_the_exact_phases(tg, orc, registered):
    """With the MFMA phases forced on (threshold 1 pair), a layer holding an
    e = 255 block gives the oracle's 2^127 results, finite where the
    reference's are, both with staged (host) weights and with weights made
    resident by tg_mlock (scanned once, then remembered)."""
    rng = np.random.default_rng(2551)
    n, D, I, k = 2, 1024, 1024, 8
    g, u, d = _e255_case(rng, n, D, I)
    rw = np.full((n, k), 0.5, np.float32)
    x = rng.uniform(-1e-3, 1e-3, (k, D)).astype(np.float32)
    fm = [O.FMT_MXFP4] * n
    lib = tg.lib()
    if registered:
        for m in g + u + d:
            assert lib.tg_mlock(m.ctypes.data, m.nbytes) == 0
    h_ref = np.zeros((n * k, I), np.float32)
    ref = orc.moe_v2(g, u, d, O.FMT_MXFP4, fm, None, None, None, O.ACT_SILU, rw, x, np.zeros((k, D), np.float32), I,
                     hidden_out=h_ref)
    assert np.all(np.isfinite(h_ref[:k, 5])) and np.all(np.isfinite(ref))
    prev = lib.tg_hip_set_moe_grouped_min_rows(1)
    try:
        for rep in range(2):   # the second call of a registered layer takes the remembered result
            h = np.zeros((n * k, I), np.float32)
            got = tg.moe_forward_rows_v2(g, u, d, O.FMT_MXFP4, fm, None, None, None, O.ACT_SILU, rw, x,
                                         np.zeros((k, D), np.float32), I, hidden_out=h)
            assert np.all(np.isfinite(h)) and np.all(np.isfinite(got)), rep
            for p in range(n * k):
                ok, rel = close(h[p], h_ref[p], tol=1e-4)
                assert ok, (rep, p, rel)
            ref_b = orc.moe_v2(g, u, d, O.FMT_MXFP4, fm, None, None, None, O.ACT_SILU, rw, x,
                               np.zeros((k, D), np.float32), I, hidden_in=h)
            ok, rel = close(got, ref_b)
            assert ok, (rep, rel)
    finally:
        lib.tg_hip_set_moe_grouped_min_rows(prev)
        if registered:
            for m in g + u + d:
                lib.tg_hip_unregister(m.ctypes.data)


def test_moe_e8m0_255_on_a_plan(tg, orc):
    """A device-resident plan with an e = 255 block (scanned when the plan is
    made), run with the MFMA phases forced on, equals the oracle."""
    import ctypes
    rng = np.random.default_rng(2552)
    n, D, I, k = 2, 1024, 1024, 8
    g, u, d = _e255_case(rng, n, D, I)
    rw = np.full((n, k), 0.5, np.float32)
    x = rng.uniform(-1e-3, 1e-3, (k, D)).astype(np.float32)
    lib = tg.lib()
    bufs = []

    def put(a):
        b = tg.DeviceArray(a.nbytes)
        b.upload(a)
        bufs.append(b)
        return b.ptr
    try:
        gp = (ctypes.c_void_p * n)(*[put(a) for a in g])
        up = (ctypes.c_void_p * n)(*[put(a) for a in u])
        dp = (ctypes.c_void_p * n)(*[put(a) for a in d])
        fm = np.full(n, O.FMT_MXFP4, np.int32)
        plan = lib.tg_hip_moe_plan_create(ctypes.addressof(gp), ctypes.addressof(up), ctypes.addressof(dp),
                                          O.FMT_MXFP4, fm.ctypes.data, None, None, None, O.ACT_SILU, n,
                                          rw.ctypes.data, k, D, I)
        assert plan, tg.last_error()
        xd = tg.DeviceArray(x.nbytes)
        xd.upload(x)
        yd = tg.DeviceArray(x.nbytes)
        yd.upload(np.zeros_like(x))
        bufs += [xd, yd]
        prev = lib.tg_hip_set_moe_grouped_min_rows(1)
        try:
            lib.tg_hip_moe_plan_run(plan, xd.ptr, yd.ptr, None)
            lib.tg_hip_synchronize()
        finally:
            lib.tg_hip_set_moe_grouped_min_rows(prev)
            lib.tg_hip_moe_plan_destroy(plan)
        got = yd.download(np.float32, k * D).reshape(k, D)
        ref = orc.moe_v2(g, u, d, O.FMT_MXFP4, list(fm), None, None, None, O.ACT_SILU, rw, x,
                         np.zeros((k, D), np.float32), I)
        assert np.all(np.isfinite(got))
        ok, rel = close(got, ref, tol=1e-4)
        assert ok, rel
    finally:
        for b in bufs:
            b.free()


def test_decode_mx_step_refuses_e8m0_255(tg):
    """The persistent gpt-oss step (block-scaled MFMA, no v_dot4 form) is not
    created over a layer holding an e = 255 block: NULL and an error naming
    the byte, while modes 0 and 1 (per-layer kernels) accept it."""
    import ctypes
    import tinygiant_amd.synth as S
    lib = tg.lib()
    D = I = 2880
    n = 4
    rb = lib.tg_row_bytes(O.FMT_MXFP4, D)
    bufs = []

    def mat(seed, nrows, poke=False):
        b = tg.DeviceArray(nrows * rb)
        lib.tg_hip_synth_fill(3, seed, b.ptr, nrows * rb, None)
        if poke:
            b.upload(np.array([255], np.uint8), offset=7 * rb + 17 * 11)   # row 7, block 11: its scale byte
        bufs.append(b)
        return b.ptr
    try:
        gp = (ctypes.c_void_p * n)(*[mat(S.tensor_seed(91, 0, e, 0), I, poke=e == 2) for e in range(n)])
        up = (ctypes.c_void_p * n)(*[mat(S.tensor_seed(91, 0, e, 1), I) for e in range(n)])
        dp = (ctypes.c_void_p * n)(*[mat(S.tensor_seed(91, 0, e, 2), D) for e in range(n)])
        biases = []
        for nrows in (I, I, D):
            arr = []
            for e in range(n):
                b = tg.DeviceArray(nrows * 4)
                b.upload(np.zeros(nrows, np.float32))
                bufs.append(b)
                arr.append(b.ptr)
            biases.append((ctypes.c_void_p * n)(*arr))
        fm = np.full(n, O.FMT_MXFP4, np.int32)
        rw = np.full((n, 1), 0.25, np.float32)
        plan = lib.tg_hip_moe_plan_create(ctypes.addressof(gp), ctypes.addressof(up), ctypes.addressof(dp),
                                          O.FMT_MXFP4, fm.ctypes.data, *[ctypes.addressof(b) for b in biases],
                                          O.ACT_GPTOSS, n, rw.ctypes.data, 1, D, I)
        assert plan, tg.last_error()
        h = tg.DeviceArray(D * 4)
        h.upload(np.zeros(D, np.float32))
        bufs.append(h)
        arr = (ctypes.c_void_p * 1)(plan)
        try:
            for mode, ok in ((3, False), (2, False), (0, True), (1, True)):
                lib.tg_hip_clear_error()
                st = lib.tg_hip_decode_create(ctypes.addressof(arr), 1, None, ctypes.c_float(1e-5), h.ptr, mode)
                if ok:
                    assert st, (mode, tg.last_error())
                    lib.tg_hip_decode_destroy(st)
                else:
                    assert not st, mode
                    assert "255" in tg.last_error(), tg.last_error()
        finally:
            lib.tg_hip_moe_plan_destroy(plan)
    finally:
        for b in bufs:
            b.free()
