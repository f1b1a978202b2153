"""GPU parity of the output head with fused argmax (tg_hip_head_argmax_dev):
the reference's per-row tg_rms_norm + tg_matmul over the head
(tinygiant/engine.py:347-354) followed by numpy.argmax of each row
(tinygiant/specdec.py:77,90).

Bars:
  logits (no RMSNorm weight)   <= 1e-5 of max|logit| against the oracle's
                               tg_matmul of the same rows (the q8 of the
                               input is computed from identical f32 values)
  logits (with RMSNorm)        <= 1e-4 of max: the GPU's normalized rows may
                               differ from the oracle's by an ulp, which can
                               flip one q8 rounding (same bound as the MoE
                               hidden stage)
  argmax                       equal to numpy.argmax of the oracle logits,
                               unless the oracle's top two logits are closer
                               than the logit tolerance (a near tie)
  ties                         first index, as numpy.argmax
"""

import ctypes
import sys

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu
Q4K, Q6K = 0, 2


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _head(tg, fmt, mat, x, nrows, ncols, norm=None, eps=1e-6, want_logits=True):
    lib = tg.lib()
    k = x.shape[0]
    md = tg.DeviceArray(mat.nbytes)
    md.upload(mat)
    xd = tg.DeviceArray(x.nbytes)
    xd.upload(np.ascontiguousarray(x, np.float32))
    nd = None
    if norm is not None:
        nd = tg.DeviceArray(norm.nbytes)
        nd.upload(norm)
    ld = tg.DeviceArray(k * nrows * 4) if want_logits else None
    ad = tg.DeviceArray(k * 4)
    vd = tg.DeviceArray(k * 4)
    sb = lib.tg_hip_head_scratch_bytes(k, nrows, ncols)
    sd = tg.DeviceArray(sb)
    lib.tg_hip_clear_error()
    lib.tg_hip_head_argmax_dev(fmt, md.ptr, xd.ptr, nd.ptr if nd else None, ctypes.c_float(eps), k, nrows, ncols,
                               ld.ptr if ld else None, ad.ptr, vd.ptr, sd.ptr, None)
    lib.tg_hip_synchronize()
    assert tg.last_error() == "", tg.last_error()
    logits = ld.download(np.float32, k * nrows).reshape(k, nrows) if ld else None
    am = ad.download(np.int32, k)
    mv = vd.download(np.float32, k)
    for a in (md, xd, nd, ld, ad, vd, sd):
        if a is not None:
            a.free()
    return logits, am, mv


def _oracle(orc, fmt, mat, x, nrows, ncols, norm=None, eps=1e-6):
    rows = []
    for r in range(x.shape[0]):
        xr = orc.rms_norm(x[r], norm, eps) if norm is not None else x[r]
        rows.append(orc.matmul(fmt, mat, None, xr, nrows, ncols))
    return np.stack(rows)


def _check(ref, logits, am, mv, tol):
    scale = np.abs(ref).max()
    if logits is not None:
        err = np.abs(logits - ref).max() / scale
        assert err <= tol, err
    for j in range(ref.shape[0]):
        want = int(np.argmax(ref[j]))
        top2 = np.sort(ref[j])[-2:]
        if am[j] != want:
            # only a near tie may flip the winner
            assert top2[1] - top2[0] <= 2 * tol * scale, (j, am[j], want, top2)
            assert abs(ref[j][am[j]] - top2[1]) <= 2 * tol * scale
        if logits is not None:
            assert am[j] == int(np.argmax(logits[j])), j
            assert mv[j] == logits[j][am[j]]


@pytest.mark.parametrize("k", [1, 5, 9, 16])
def test_head_q6k_fused_matches_oracle(tg, orc, k):
    """Q6_K head of 2048 columns: the fused single-pass kernel."""
    import tinygiant_amd.synth as S
    nrows, ncols = 3001, 2048   # not a multiple of the 4 rows a wave covers
    say(f"head q6k fused k={k}")
    mat = S.matrix_host(Q6K, S.tensor_seed(11, 0, 0, 3), nrows, ncols)
    x = np.random.default_rng(k).standard_normal((k, ncols)).astype(np.float32)
    logits, am, mv = _head(tg, Q6K, mat, x, nrows, ncols)
    ref = _oracle(orc, Q6K, mat, x, nrows, ncols)
    _check(ref, logits, am, mv, 1e-5)


def test_head_q6k_fused_argmax_without_logits(tg, orc):
    """The argmax does not depend on the logits buffer being requested."""
    import tinygiant_amd.synth as S
    nrows, ncols, k = 2053, 2048, 3
    mat = S.matrix_host(Q6K, S.tensor_seed(12, 0, 0, 3), nrows, ncols)
    x = np.random.default_rng(7).standard_normal((k, ncols)).astype(np.float32)
    l1, a1, v1 = _head(tg, Q6K, mat, x, nrows, ncols)
    _, a2, v2 = _head(tg, Q6K, mat, x, nrows, ncols, want_logits=False)
    assert np.array_equal(a1, a2) and np.array_equal(v1, v2)


def test_head_q6k_with_rmsnorm(tg, orc):
    """x_j = RMSNorm(h_j) * output_norm then the head, as engine.py:350-353."""
    import tinygiant_amd.synth as S
    nrows, ncols, k = 1500, 2048, 5
    mat = S.matrix_host(Q6K, S.tensor_seed(13, 0, 0, 3), nrows, ncols)
    rng = np.random.default_rng(9)
    x = (3.0 * rng.standard_normal((k, ncols))).astype(np.float32)
    norm = rng.uniform(0.5, 1.5, ncols).astype(np.float32)
    logits, am, mv = _head(tg, Q6K, mat, x, nrows, ncols, norm=norm)
    ref = _oracle(orc, Q6K, mat, x, nrows, ncols, norm=norm)
    _check(ref, logits, am, mv, 1e-4)


def test_head_generic_format(tg, orc):
    """Formats without a fused kernel (here Q4_K) take GEMV + argmax."""
    import tinygiant_amd.synth as S
    nrows, ncols, k = 1200, 2048, 4
    mat = S.matrix_host(Q4K, S.tensor_seed(14, 0, 0, 3), nrows, ncols)
    x = np.random.default_rng(3).standard_normal((k, ncols)).astype(np.float32)
    logits, am, mv = _head(tg, Q4K, mat, x, nrows, ncols)
    ref = _oracle(orc, Q4K, mat, x, nrows, ncols)
    _check(ref, logits, am, mv, 1e-5)
    _, am2, _ = _head(tg, Q4K, mat, x, nrows, ncols, want_logits=False)
    assert np.array_equal(am, am2)


def test_head_ties_take_the_first_row(tg, orc):
    """numpy.argmax's rule: all-zero logits -> row 0; two identical winning
    rows -> the first of them."""
    import tinygiant_amd.synth as S
    nrows, ncols, rb = 1024, 2048, 8 * 210
    x = np.random.default_rng(1).standard_normal((2, ncols)).astype(np.float32)
    zero = np.zeros(nrows * rb, np.uint8)
    _, am, mv = _head(tg, Q6K, zero, x, nrows, ncols)
    assert list(am) == [0, 0] and list(mv) == [0.0, 0.0]
    # rows 317 and 701 carry the same random row, every other row is zero
    src = S.matrix_host(Q6K, S.tensor_seed(15, 0, 0, 3), 1, ncols)
    mat = zero.copy()
    mat[317 * rb:318 * rb] = src
    mat[701 * rb:702 * rb] = src
    v = orc.matmul(Q6K, src, None, x[0], 1, ncols)[0]
    xs = x if v > 0 else -x   # make that row's logit positive for both inputs? only row 0 is known
    logits, am, _ = _head(tg, Q6K, mat, xs[:1], nrows, ncols)
    assert logits[0][317] == logits[0][701] > 0
    assert am[0] == 317


@pytest.mark.parametrize("k", [1, 5, 9, 16])
def test_head_q6k_full_vocabulary(tg, orc, k):
    """The Qwen3-30B-A3B output head at its full size, 151936 x 2048 q6_K
    (255,252,480 bytes; engine.py:347-354 with tg_matmul, csrc/libtinygiant.c:
    925-931), with the RMSNorm weight applied, over a k-row verify batch:
    every logit against the oracle and the fused argmax against the oracle's."""
    import tinygiant_amd.synth as S
    nrows, ncols = 151936, 2048
    rng = np.random.default_rng(151936 + k)
    mat = S.matrix_host(Q6K, S.tensor_seed(15, 0, 0, 3), nrows, ncols)
    x = rng.standard_normal((k, ncols)).astype(np.float32)
    norm = rng.uniform(0.5, 1.5, ncols).astype(np.float32)
    say(f"head full vocabulary k={k}")
    logits, am, mv = _head(tg, Q6K, mat, x, nrows, ncols, norm=norm)
    ref = _oracle(orc, Q6K, mat, x, nrows, ncols, norm=norm)
    _check(ref, logits, am, mv, 1e-5)


@pytest.mark.parametrize("k", [3, 7, 12])
def test_head_q6k_padded_row_counts(tg, orc, k):
    """Row counts between the kernel's instantiations (3 -> 4, 7 -> 8,
    12 -> 16): the unused input slots take part in the reduce-scatter as
    zeros and never reach the argmax."""
    import tinygiant_amd.synth as S
    nrows, ncols = 2501, 2048
    mat = S.matrix_host(Q6K, S.tensor_seed(16, 0, 0, 3), nrows, ncols)
    x = np.random.default_rng(100 + k).standard_normal((k, ncols)).astype(np.float32)
    logits, am, mv = _head(tg, Q6K, mat, x, nrows, ncols)
    ref = _oracle(orc, Q6K, mat, x, nrows, ncols)
    _check(ref, logits, am, mv, 1e-5)


def test_head_q6k_scratch_reused_across_calls(tg, orc):
    """Two calls on one scratch buffer: the argmax keys and the finish
    counter the kernel leaves behind are cleared by the next call."""
    import tinygiant_amd.synth as S
    lib = tg.lib()
    nrows, ncols, k = 1999, 2048, 5
    mat = S.matrix_host(Q6K, S.tensor_seed(17, 0, 0, 3), nrows, ncols)
    md = tg.DeviceArray(mat.nbytes)
    md.upload(mat)
    sd = tg.DeviceArray(lib.tg_hip_head_scratch_bytes(k, nrows, ncols))
    ad = tg.DeviceArray(k * 4)
    vd = tg.DeviceArray(k * 4)
    xd = tg.DeviceArray(k * ncols * 4)
    try:
        for seed in (1, 2):
            x = np.random.default_rng(seed).standard_normal((k, ncols)).astype(np.float32)
            if seed == 2:
                x = -x   # a different winner per row
            xd.upload(x)
            lib.tg_hip_head_argmax_dev(Q6K, md.ptr, xd.ptr, None, ctypes.c_float(1e-6), k, nrows, ncols, None,
                                       ad.ptr, vd.ptr, sd.ptr, None)
            lib.tg_hip_synchronize()
            am = ad.download(np.int32, k)
            mv = vd.download(np.float32, k)
            ref = _oracle(orc, Q6K, mat, x, nrows, ncols)
            for j in range(k):
                top2 = np.sort(ref[j])[-2:]
                if am[j] != int(np.argmax(ref[j])):
                    assert top2[1] - top2[0] <= 2e-5 * np.abs(ref).max(), (seed, j)
                assert abs(mv[j] - ref[j][am[j]]) <= 1e-5 * np.abs(ref).max(), (seed, j)
    finally:
        for a in (md, sd, ad, vd, xd):
            a.free()


class _head_kernel:
    """Sets the input-row count from which the head runs on int8 MFMA."""

    def __init__(self, tg, k):
        self.lib, self.k = tg.lib(), k

    def __enter__(self):
        self.prev = self.lib.tg_hip_set_head_mfma_min_k(self.k)

    def __exit__(self, *exc):
        self.lib.tg_hip_set_head_mfma_min_k(self.prev)


@pytest.mark.parametrize("k", [1, 2, 5, 9, 16])
def test_head_q6k_mfma_logits_bit_exact(tg, orc, k):
    """The int8 MFMA head (every k, forced on): each block's integer sum is
    exact and its term d * d_x * sum is added in block order, the oracle's
    row loop, so the logits equal the oracle's tg_matmul bit for bit (the
    oracle's float block sums stay below 2^24 here, where they are exact);
    3001 rows end in a partial 16-row item."""
    import tinygiant_amd.synth as S
    nrows, ncols = 3001, 2048
    say(f"head q6k mfma k={k}")
    mat = S.matrix_host(Q6K, S.tensor_seed(18, 0, 0, 3), nrows, ncols)
    x = np.random.default_rng(200 + k).standard_normal((k, ncols)).astype(np.float32)
    with _head_kernel(tg, 1):
        logits, am, mv = _head(tg, Q6K, mat, x, nrows, ncols)
    ref = _oracle(orc, Q6K, mat, x, nrows, ncols)
    assert logits.tobytes() == ref.tobytes(), np.abs(logits - ref).max() / np.abs(ref).max()
    _check(ref, logits, am, mv, 0.0)


def test_head_q6k_mfma_equals_dot4(tg, orc):
    """The same 9-row batch through both kernels: logits within the f32 bar
    of each other, the same argmax (no near tie in this batch)."""
    import tinygiant_amd.synth as S
    nrows, ncols, k = 4099, 2048, 9
    mat = S.matrix_host(Q6K, S.tensor_seed(19, 0, 0, 3), nrows, ncols)
    x = np.random.default_rng(9).standard_normal((k, ncols)).astype(np.float32)
    out = {}
    for name, kk in (("mfma", 1), ("dot4", 0)):
        with _head_kernel(tg, kk):
            out[name] = _head(tg, Q6K, mat, x, nrows, ncols)
    lm, am_m, _ = out["mfma"]
    ld, am_d, _ = out["dot4"]
    assert np.abs(lm - ld).max() <= 1e-5 * np.abs(ld).max()
    assert list(am_m) == list(am_d)


def test_head_q6k_mfma_ties_and_zero_rows(tg, orc):
    """numpy.argmax's rule on the MFMA kernel: an all-zero head gives row 0
    for every input row; two identical winning rows give the first."""
    import tinygiant_amd.synth as S
    nrows, ncols, rb, k = 1040, 2048, 8 * 210, 6
    x = np.random.default_rng(3).standard_normal((k, ncols)).astype(np.float32)
    zero = np.zeros(nrows * rb, np.uint8)
    with _head_kernel(tg, 1):
        _, am, mv = _head(tg, Q6K, zero, x, nrows, ncols)
        assert list(am) == [0] * k and list(mv) == [0.0] * k
        src = S.matrix_host(Q6K, S.tensor_seed(20, 0, 0, 3), 1, ncols)
        mat = zero.copy()
        mat[333 * rb:334 * rb] = src
        mat[1001 * rb:1002 * rb] = src
        logits, am, _ = _head(tg, Q6K, mat, x, nrows, ncols)
    for j in range(k):
        assert logits[j][333] == logits[j][1001]
        if logits[j][333] > 0:
            assert am[j] == 333
        else:
            assert logits[j][am[j]] == 0.0 and am[j] == 0


@pytest.mark.parametrize("k", [3, 4, 5])
@pytest.mark.parametrize("nrows", [1999, 40001])
def test_head_q6k_argmax_at_loop_exit(tg, orc, k, nrows):
    """Row counts where every wave leaves the row-group loop after one group
    (1999 rows: 125 workgroups of four waves) or after two and three (40001
    rows on the 1024-workgroup grid), with the next group's loads still in
    flight at the exit: the argmax-only kernel (no logits buffer) and the
    one that also writes logits, each against the oracle."""
    import tinygiant_amd.synth as S
    ncols = 2048
    say(f"head q6k loop exit k={k} nrows={nrows}")
    mat = S.matrix_host(Q6K, S.tensor_seed(21, 0, 0, 3), nrows, ncols)
    x = np.random.default_rng(300 + k).standard_normal((k, ncols)).astype(np.float32)
    ref = _oracle(orc, Q6K, mat, x, nrows, ncols)
    _, am, mv = _head(tg, Q6K, mat, x, nrows, ncols, want_logits=False)
    _check(ref, None, am, mv, 1e-5)
    for j in range(k):
        assert abs(mv[j] - ref[j][am[j]]) <= 1e-5 * np.abs(ref).max(), j
    logits, am2, mv2 = _head(tg, Q6K, mat, x, nrows, ncols)
    _check(ref, logits, am2, mv2, 1e-5)
    assert np.array_equal(am, am2) and np.array_equal(mv, mv2)
