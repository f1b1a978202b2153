"""GPU parity of libtinygiant_hip against the oracle, through the C ABI.

Bars (from the north-star contract and the reference's own tests):
  * q8 quants, scales, 32-element sums: bit-exact;
  * per-sub-block integer dot sums: bit-exact;
  * f32 outputs: max|gpu - oracle| <= 1e-5 * max|oracle| (the reference's
    MoE metric, csrc/test_libtinygiant.c:467-476), with a 1e-5 relative
    floor per row for GEMVs;
  * integer special cases (unit scales, integer x with amax 127): exact;
  * run-to-run bit identity (the GPU analogue of Test 8).
"""

import ctypes
import sys

import numpy as np
import pytest

import oracle as O
from tests import _formats as F
from tests.test_oracle_pins import _rand_row, _unit_row

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(4242)
TOL = 1e-5


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def close(got, ref, tol=TOL):
    scale = max(np.abs(ref).max(), 1e-30)
    err = np.abs(got.astype(np.float64) - ref).max()
    return err <= tol * scale, err / scale


@pytest.mark.parametrize("n,rows", [(32, 1), (256, 3), (768, 2), (2048, 4), (2880, 2)])
def test_quantize_q8_bit_exact(tg, orc, n, rows):
    say("quantize", n, rows)
    x = (RNG.standard_normal((rows, n)) * 10 ** RNG.uniform(-4, 4)).astype(np.float32)
    x[0, : n // 2] = 0
    if rows > 1:
        x[1] = RNG.integers(-127, 128, n)
        x[1, 0] = 127
    got = tg.quantize_q8(x)
    ref = orc.quantize_q8(x)
    assert got.tobytes() == ref.tobytes()


def test_quantize_q8_edge_values(tg, orc):
    say("quantize edges")
    x = np.zeros((3, 256), np.float32)
    x[1, :4] = [127.0, 0.5, 1.5, -2.5]
    x[2] = np.float32(1e-40) * RNG.standard_normal(256).astype(np.float32)   # denormals
    assert tg.quantize_q8(x).tobytes() == orc.quantize_q8(x).tobytes()


FMTS = [(O.FMT_Q4K, 2048), (O.FMT_Q4K, 768), (O.FMT_Q6K, 768), (O.FMT_Q6K, 2048),
        (O.FMT_MXFP4, 2880), (O.FMT_Q80, 2880), (O.FMT_Q4K, 4096)]


@pytest.mark.parametrize("fmt,ncols", FMTS)
def test_isums_bit_exact(tg, orc, fmt, ncols):
    say("isums", fmt, ncols)
    nrows = 37
    mat = np.concatenate([_rand_row(fmt, ncols) for _ in range(nrows)])
    x = RNG.standard_normal(ncols).astype(np.float32)
    got = tg.isums(fmt, mat, nrows, ncols, x)
    ref = orc.isums(fmt, mat, nrows, ncols, x)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("fmt,ncols", FMTS)
def test_matmul_vs_oracle(tg, orc, fmt, ncols):
    say("matmul", fmt, ncols)
    nrows = 300
    mat = np.concatenate([_rand_row(fmt, ncols) for _ in range(nrows)])
    x = RNG.standard_normal(ncols).astype(np.float32)
    bias = RNG.standard_normal(nrows).astype(np.float32)
    got = tg.matmul(fmt, mat, bias, x, nrows, ncols)
    ref = orc.matmul(fmt, mat, bias, x, nrows, ncols)
    ok, rel = close(got, ref)
    assert ok, rel


def test_matmul_q4k_768x2048(tg, orc):
    """The single fused matvec of the smallest workload at its exact shape:
    768 x 2048 q4_K (d, dmin U[1e-3, 2e-2], uniform scale and quant bytes),
    x ~ N(0, 1), through tg_matmul (csrc/libtinygiant.c:908-931), and its
    per-sub-block integer sums bit-exact."""
    import tinygiant_amd.synth as S
    say("matmul q4_K 768x2048")
    nrows, ncols = 768, 2048
    mat = S.matrix_host(O.FMT_Q4K, S.tensor_seed(20261201, 0, 0, 0), nrows, ncols)
    x = np.random.default_rng(768).standard_normal(ncols).astype(np.float32)
    got = tg.matmul(O.FMT_Q4K, mat, None, x, nrows, ncols)
    ref = orc.matmul(O.FMT_Q4K, mat, None, x, nrows, ncols)
    ok, rel = close(got, ref)
    assert ok, rel
    assert np.array_equal(tg.isums(O.FMT_Q4K, mat, nrows, ncols, x), orc.isums(O.FMT_Q4K, mat, nrows, ncols, x))


@pytest.mark.parametrize("fmt,ncols", FMTS)
def test_matmul_integer_cases_exact(tg, orc, fmt, ncols):
    say("matmul exact", fmt, ncols)
    nrows = 64
    mat = np.concatenate([_unit_row(fmt, ncols) for _ in range(nrows)])
    x = RNG.integers(-127, 128, ncols).astype(np.float32)
    x[::256] = 127
    got = tg.matmul(fmt, mat, None, x, nrows, ncols)
    ref = orc.matmul(fmt, mat, None, x, nrows, ncols)
    assert np.array_equal(got, ref)


def test_matmul_f16(tg, orc):
    say("matmul f16")
    nrows, ncols = 200, 768
    w = (RNG.standard_normal((nrows, ncols)) * 0.05).astype(np.float16)
    x = RNG.standard_normal(ncols).astype(np.float32)
    got = tg.matmul(O.FMT_F16, w.view(np.uint8), None, x, nrows, ncols)
    ref = orc.matmul(O.FMT_F16, w.view(np.uint8), None, x, nrows, ncols)
    ok, rel = close(got, ref)
    assert ok, rel


def test_matmul_run_to_run_identical(tg):
    say("matmul determinism")
    nrows, ncols = 1000, 2048
    mat = np.concatenate([_rand_row(O.FMT_Q6K, ncols) for _ in range(nrows)])
    x = RNG.standard_normal(ncols).astype(np.float32)
    a = tg.matmul(O.FMT_Q6K, mat, None, x, nrows, ncols)
    b = tg.matmul(O.FMT_Q6K, mat, None, x, nrows, ncols)
    assert a.tobytes() == b.tobytes()


def test_shutdown_then_reinit(tg):
    """tg_hip_shutdown releases the library's stream, arena and pinned rows;
    the next call sets them up again and computes the same bits."""
    say("shutdown + re-init")
    nrows, ncols = 300, 2048
    mat = np.concatenate([_rand_row(O.FMT_Q4K, ncols) for _ in range(nrows)])
    x = RNG.standard_normal(ncols).astype(np.float32)
    a = tg.matmul(O.FMT_Q4K, mat, None, x, nrows, ncols)
    lib = tg.lib()
    lib.tg_hip_shutdown()
    lib.tg_hip_shutdown()          # a second call finds nothing to release
    b = tg.matmul(O.FMT_Q4K, mat, None, x, nrows, ncols)
    assert a.tobytes() == b.tobytes()


def _experts(n, D, I, gate_fmt, down_fmts, seed):
    import tinygiant_amd.synth as S
    g, u, d = [], [], []
    for e in range(n):
        g.append(S.matrix_host(gate_fmt, S.tensor_seed(seed, 0, e, 0), I, D))
        u.append(S.matrix_host(gate_fmt, S.tensor_seed(seed, 0, e, 1), I, D))
        d.append(S.matrix_host(down_fmts[e], S.tensor_seed(seed, 0, e, 2), D, I))
    return g, u, d


def _check_moe(tg, orc, n, k, D, I, gate_fmt, down_fmts, act, biases, rw, x, base=None):
    """Stage-wise parity of one MoE call.

    The hidden rows are re-quantized to q8 between the two projections, so a
    last-bit difference in a hidden value (summation order, expf) can move a
    q8 rounding across .5 and change one integer; the end-to-end f32 bar is
    therefore asserted through the stages:
      A  hidden (gate/up + act) vs the oracle's          <= 1e-4 per pair row
         (the reference's bound for two accumulation orders of the same
         integer sums, csrc/test_libtinygiant.c:158-163; gpt-oss dots run to
         thousands before the clamp, and the oracle itself is 1.6e-5 from the
         float64 value there)
      Q  q8(GPU hidden) vs oracle q8 of the same values  bit-exact
      B  down + combine from the GPU's own hidden         <= 1e-5 of max|out|
      E  end to end vs the oracle                         <= 1e-5 whenever no
         q8 rounding of the hidden flipped (checked, and counted otherwise)
    """
    g, u, d = _experts(n, D, I, gate_fmt, down_fmts, 99)
    gb = ub = db = None
    if biases:
        gb = [RNG.uniform(-0.5, 0.5, I).astype(np.float32) for _ in range(n)]
        ub = [RNG.uniform(-0.5, 0.5, I).astype(np.float32) for _ in range(n)]
        db = [RNG.uniform(-0.05, 0.05, D).astype(np.float32) for _ in range(n)]
    out0 = np.zeros((k, D), np.float32) if base is None else base.copy()
    P = int(np.count_nonzero(rw))
    nbI = (I + 255) // 256
    h_ref = np.zeros((P, I), np.float32)
    ref = orc.moe_v2(g, u, d, gate_fmt, down_fmts, gb, ub, db, act, rw, x, out0.copy(), I, hidden_out=h_ref)
    h_gpu = np.zeros((P, I), np.float32)
    hq_gpu = np.zeros((P, nbI), orc.Q8_DTYPE)
    got = tg.moe_forward_rows_v2(g, u, d, gate_fmt, down_fmts, gb, ub, db, act, rw, x, out0.copy(), I,
                                 hidden_out=h_gpu, hq_out=hq_gpu)
    # A
    for p in range(P):
        ok, rel = close(h_gpu[p], h_ref[p], tol=1e-4)
        assert ok, ("hidden", p, rel)
    # Q
    assert hq_gpu.tobytes() == orc.quantize_q8(h_gpu).tobytes()
    # B
    ref_b = orc.moe_v2(g, u, d, gate_fmt, down_fmts, gb, ub, db, act, rw, x, out0.copy(), I, hidden_in=h_gpu)
    ok, rel = close(got, ref_b)
    assert ok, ("down+combine", rel)
    # E
    flips = int(np.count_nonzero(orc.quantize_q8(h_gpu)["qs"] != orc.quantize_q8(h_ref)["qs"]))
    ok, rel = close(got, ref)
    say(f"  end-to-end rel {rel:.2e}, hidden q8 flips {flips}")
    if flips == 0:
        assert ok, rel
    return got, ref


def test_moe_qwen_layer_one_token(tg, orc):
    """One Qwen3-30B-A3B MoE layer for one token: 8 experts, q4_K gate/up, q6_K down."""
    say("moe qwen k=1")
    import tinygiant_amd.synth as S
    rng = np.random.default_rng(5)
    experts, rw = S.routing_rows(rng, 1, 128, 8)
    x = rng.standard_normal((1, 2048)).astype(np.float32)
    _check_moe(tg, orc, len(experts), 1, 2048, 768, O.FMT_Q4K, [O.FMT_Q6K] * len(experts), O.ACT_SILU,
               False, rw, x)


@pytest.mark.parametrize("k,pool", [(2, 32), (5, 32), (9, 32), (5, 128), (9, 128)])
def test_moe_grouped_verify_rows(tg, orc, k, pool):
    """Self-speculative verify batch: K+1 rows, Zipf-skewed top-8 over a pool
    of 32 experts (many rows per expert) or all 128 of a Qwen3 layer."""
    say("moe grouped", k, pool)
    import tinygiant_amd.synth as S
    rng = np.random.default_rng(100 + k + pool)
    experts, rw = S.routing_rows(rng, k, pool, 8)
    x = rng.standard_normal((k, 2048)).astype(np.float32)
    base = rng.standard_normal((k, 2048)).astype(np.float32)
    _check_moe(tg, orc, len(experts), k, 2048, 768, O.FMT_Q4K, [O.FMT_Q6K] * len(experts), O.ACT_SILU,
               False, rw, x, base)


def test_moe_mixed_down_formats(tg, orc):
    """Reference Test 7 shape: mixed q4_K / q6_K down, sparse weights, k=6."""
    say("moe mixed")
    n, k = 8, 6
    fmts = [O.FMT_Q6K if e % 2 else O.FMT_Q4K for e in range(n)]
    rw = np.zeros((n, k), np.float32)
    for r in range(k):
        for j in range(3):
            rw[(r + j * 2) % n, r] = 0.2 + 0.1 * j
    x = (RNG.standard_normal((k, 2048)) * 0.01).astype(np.float32)
    _check_moe(tg, orc, n, k, 2048, 768, O.FMT_Q4K, fmts, O.ACT_SILU, False, rw, x)


def test_moe_wide_rows_fall_back(tg, orc):
    """Rows too wide for the expert-major phases' LDS staging (8 q8 rows of
    16384 values: 178 KiB against the device's 160 KiB) take the per-pair
    kernels instead of failing the launch."""
    say("moe wide rows")
    n, k, D, I = 2, 8, 16384, 256
    rw = np.full((n, k), 0.5, np.float32)
    x = (RNG.standard_normal((k, D)) * 0.1).astype(np.float32)
    _check_moe(tg, orc, n, k, D, I, O.FMT_Q4K, [O.FMT_Q6K] * n, O.ACT_SILU, False, rw, x)


def test_moe_f16_down(tg, orc):
    say("moe f16 down")
    n, k, D, I = 2, 2, 512, 256
    g, u, _ = _experts(n, D, I, O.FMT_Q4K, [O.FMT_Q4K] * n, 7)
    d = [(RNG.standard_normal(D * I) * 0.05).astype(np.float16).view(np.uint8) for _ in range(n)]
    rw = np.array([[0.7, 0.2], [0.3, 0.8]], np.float32)
    x = RNG.standard_normal((k, D)).astype(np.float32)
    ref = orc.moe_v2(g, u, d, O.FMT_Q4K, [O.FMT_F16] * n, None, None, None, O.ACT_SILU, rw, x,
                     np.zeros((k, D), np.float32), I)
    got = tg.moe_forward_rows_v2(g, u, d, O.FMT_Q4K, [O.FMT_F16] * n, None, None, None, O.ACT_SILU, rw, x,
                                 np.zeros((k, D), np.float32), I)
    ok, rel = close(got, ref)
    assert ok, rel


def test_moe_mxfp4_gptoss_biases(tg, orc):
    """Reference Test 10 shape: gpt-oss D=I=2880, mxfp4, gpt-oss activation, biases, k=3."""
    say("moe mxfp4 gptoss")
    n, k = 2, 3
    rw = np.array([[0.6, 0.0, 0.3], [0.4, 1.0, 0.7]], np.float32)
    x = RNG.uniform(-1, 1, (k, 2880)).astype(np.float32)
    _check_moe(tg, orc, n, k, 2880, 2880, O.FMT_MXFP4, [O.FMT_MXFP4] * n, O.ACT_GPTOSS, True, rw, x)


def test_moe_edge_cases(tg, orc):
    say("moe edges")
    D, I = 512, 256
    g, u, d = _experts(2, D, I, O.FMT_Q4K, [O.FMT_Q6K] * 2, 3)
    x = RNG.standard_normal((2, D)).astype(np.float32)
    base = RNG.standard_normal((2, D)).astype(np.float32)
    # every weight zero: output untouched
    out = tg.moe_forward_rows_v2(g, u, d, O.FMT_Q4K, [O.FMT_Q6K] * 2, None, None, None, O.ACT_SILU,
                                 np.zeros((2, 2), np.float32), x, base.copy(), I)
    assert np.array_equal(out, base)
    # one expert active for one row, the other row untouched
    rw = np.array([[0.5, 0.0], [0.0, 0.0]], np.float32)
    out = tg.moe_forward_rows_v2(g, u, d, O.FMT_Q4K, [O.FMT_Q6K] * 2, None, None, None, O.ACT_SILU, rw, x,
                                 base.copy(), I)
    ref = orc.moe_v2(g, u, d, O.FMT_Q4K, [O.FMT_Q6K] * 2, None, None, None, O.ACT_SILU, rw, x, base.copy(), I)
    assert np.array_equal(out[1], base[1])
    ok, rel = close(out, ref)
    assert ok, rel


def test_moe_prefill_64_rows(tg, orc):
    """Short prefill: 64 rows over a 16-expert pool."""
    say("moe prefill 64")
    import tinygiant_amd.synth as S
    rng = np.random.default_rng(64)
    experts, rw = S.routing_rows(rng, 64, 16, 4)
    x = rng.standard_normal((64, 2048)).astype(np.float32)
    _check_moe(tg, orc, len(experts), 64, 2048, 768, O.FMT_Q4K, [O.FMT_Q6K] * len(experts), O.ACT_SILU,
               False, rw, x)


@pytest.mark.parametrize("k,pool,top,mixed", [(1, 128, 8, False), (9, 32, 8, False), (6, 8, 3, True),
                                               (64, 16, 4, False)])
def test_moe_expert_major_equals_per_pair(tg, orc, k, pool, top, mixed):
    """Q4_K / Q6_K phases run expert-major (each weight row read once for all
    pairs of its expert, q8 rows staged eight at a time in LDS), with the q8
    and the combine inside the phases or in launches of their own, or one
    workgroup column per pair: the same operations per pair, so the same
    bits in every mode, also past eight pairs per expert and with mixed down
    formats."""
    say("moe expert-major vs per-pair", k, pool, top, mixed)
    import tinygiant_amd.synth as S
    rng = np.random.default_rng(700 + k)
    experts, rw = S.routing_rows(rng, k, pool, top)
    n = len(experts)
    fmts = [O.FMT_Q6K if (e % 2 or not mixed) else O.FMT_Q4K for e in range(n)]
    g, u, d = _experts(n, 2048, 768, O.FMT_Q4K, fmts, 41)
    x = rng.standard_normal((k, 2048)).astype(np.float32)
    base = rng.standard_normal((k, 2048)).astype(np.float32)
    P = int(np.count_nonzero(rw))
    lib = tg.lib()
    outs = []
    prev = lib.tg_hip_set_moe_expert_major(7)
    prev_qk = lib.tg_hip_set_moe_qk_min_rows(0)   # the v_dot4 phases, whose bits these modes share
    try:
        for on in (7, 0, 1, 5, 3, 15):
            lib.tg_hip_set_moe_expert_major(on)
            h = np.zeros((P, 768), np.float32)
            o = tg.moe_forward_rows_v2(g, u, d, O.FMT_Q4K, fmts, None, None, None, O.ACT_SILU, rw, x, base.copy(),
                                       768, hidden_out=h)
            outs.append((h, o))
    finally:
        lib.tg_hip_set_moe_expert_major(prev)
        lib.tg_hip_set_moe_qk_min_rows(prev_qk)
    say("  pairs", P, "most per expert", int(np.count_nonzero(rw, axis=1).max()))
    for h, o in outs[1:]:
        assert h.tobytes() == outs[0][0].tobytes()
        assert o.tobytes() == outs[0][1].tobytes()
    ref = orc.moe_v2(g, u, d, O.FMT_Q4K, fmts, None, None, None, O.ACT_SILU, rw, x, base.copy(), 768,
                     hidden_in=outs[0][0])
    ok, rel = close(outs[0][1], ref)
    assert ok, rel


@pytest.mark.parametrize("k", [1, 3])
def test_moe_expert_major_mxfp4_equals_per_pair(tg, orc, k):
    """gpt-oss shape (D = I = 2880: a partial last 256-block per row), MXFP4
    gate/up/down with biases and the gpt-oss activation, at most 3 pairs per
    expert (below the MFMA phases): expert-major phases in every mode give
    the per-pair kernels' bits."""
    say("moe expert-major mxfp4", k)
    import tinygiant_amd.synth as S
    rng = np.random.default_rng(900 + k)
    experts, rw = S.routing_rows(rng, k, 8, 4)
    n, D, I = len(experts), 2880, 2880
    fmts = [O.FMT_MXFP4] * n
    g, u, d = _experts(n, D, I, O.FMT_MXFP4, fmts, 43)
    gb = [rng.uniform(-0.5, 0.5, I).astype(np.float32) for _ in range(n)]
    ub = [rng.uniform(-0.5, 0.5, I).astype(np.float32) for _ in range(n)]
    db = [rng.uniform(-0.05, 0.05, D).astype(np.float32) for _ in range(n)]
    x = rng.uniform(-1, 1, (k, D)).astype(np.float32)
    base = rng.standard_normal((k, D)).astype(np.float32)
    P = int(np.count_nonzero(rw))
    assert int(np.count_nonzero(rw, axis=1).max()) < 4
    lib = tg.lib()
    outs = []
    prev = lib.tg_hip_set_moe_expert_major(7)
    try:
        for on in (7, 0, 1, 15):
            lib.tg_hip_set_moe_expert_major(on)
            h = np.zeros((P, I), np.float32)
            o = tg.moe_forward_rows_v2(g, u, d, O.FMT_MXFP4, fmts, gb, ub, db, O.ACT_GPTOSS, rw, x, base.copy(), I,
                                       hidden_out=h)
            outs.append((h, o))
    finally:
        lib.tg_hip_set_moe_expert_major(prev)
    for h, o in outs[1:]:
        assert h.tobytes() == outs[0][0].tobytes()
        assert o.tobytes() == outs[0][1].tobytes()
    ref = orc.moe_v2(g, u, d, O.FMT_MXFP4, fmts, gb, ub, db, O.ACT_GPTOSS, rw, x, base.copy(), I,
                     hidden_in=outs[0][0])
    ok, rel = close(outs[0][1], ref)
    assert ok, rel


def test_moe_registered_equals_staged(tg, orc):
    """tg_mlock (HBM-resident weights) and the per-call staging path agree bit for bit."""
    say("moe registered vs staged")
    n, k, D, I = 4, 3, 2048, 768
    g, u, d = _experts(n, D, I, O.FMT_Q4K, [O.FMT_Q6K] * n, 11)
    rw = RNG.uniform(0.1, 1, (n, k)).astype(np.float32)
    x = RNG.standard_normal((k, D)).astype(np.float32)
    staged = tg.moe_forward_rows_v2(g, u, d, O.FMT_Q4K, [O.FMT_Q6K] * n, None, None, None, O.ACT_SILU, rw, x,
                                    np.zeros((k, D), np.float32), I)
    L = tg.lib()
    for arrs in (g, u, d):
        for a in arrs:
            assert L.tg_mlock(a.ctypes.data, a.nbytes) == 0
    resident = tg.moe_forward_rows_v2(g, u, d, O.FMT_Q4K, [O.FMT_Q6K] * n, None, None, None, O.ACT_SILU, rw, x,
                                      np.zeros((k, D), np.float32), I)
    again = tg.moe_forward_rows_v2(g, u, d, O.FMT_Q4K, [O.FMT_Q6K] * n, None, None, None, O.ACT_SILU, rw, x,
                                   np.zeros((k, D), np.float32), I)
    for arrs in (g, u, d):
        for a in arrs:
            assert L.tg_hip_unregister(a.ctypes.data) == 0
    assert staged.tobytes() == resident.tobytes() == again.tobytes()


def test_legacy_entry_points(tg, orc):
    say("legacy wrappers")
    D, I = 512, 256
    L = tg.lib()
    g, u, d = _experts(1, D, I, O.FMT_Q4K, [O.FMT_Q6K], 21)
    x = RNG.standard_normal(D).astype(np.float32)
    # expert_forward_mixed with q6_K down (code 2)
    got = np.zeros(D, np.float32)
    L.tg_expert_forward_mixed(g[0].ctypes.data, u[0].ctypes.data, d[0].ctypes.data, 2, x.ctypes.data,
                              got.ctypes.data, ctypes.c_float(0.75), D, I)
    ref = orc.expert_forward_mixed(g[0], u[0], d[0], 2, x, np.zeros(D, np.float32), 0.75, D, I)
    assert close(got, ref)[0]
    # expert_forward: one all-Q4_K [gate|up|down] buffer
    import tinygiant_amd.synth as S
    gate_bytes = I * (D // 256) * 144
    down_q4 = S.matrix_host(O.FMT_Q4K, 5, D, I)
    blob = np.concatenate([g[0], u[0], down_q4])
    got = np.zeros(D, np.float32)
    L.tg_expert_forward(blob.ctypes.data, x.ctypes.data, got.ctypes.data, ctypes.c_float(0.5), D, I)
    ref = orc.expert_forward(blob, x, np.zeros(D, np.float32), 0.5, D, I)
    assert close(got, ref)[0]
    assert blob.nbytes == 2 * gate_bytes + down_q4.nbytes
    # expert_forward_rows: k rows with per-row weights
    k = 3
    xs = RNG.standard_normal((k, D)).astype(np.float32)
    w = np.array([0.2, 0.5, 0.3], np.float32)
    got = np.zeros((k, D), np.float32)
    L.tg_expert_forward_rows(g[0].ctypes.data, u[0].ctypes.data, d[0].ctypes.data, 2, xs.ctypes.data,
                             got.ctypes.data, w.ctypes.data, k, D, I)
    ref = np.zeros((k, D), np.float32)
    for r in range(k):
        orc.expert_forward_mixed(g[0], u[0], d[0], 2, xs[r], ref[r], float(w[r]), D, I)
    assert close(got, ref)[0]
    # tg_moe_forward: zeroes the output, sums weighted all-Q4_K experts
    ptrs = (ctypes.c_void_p * 2)(blob.ctypes.data, blob.ctypes.data)
    ew = np.array([0.25, 0.5], np.float32)
    got = np.full(D, 3.0, np.float32)
    L.tg_moe_forward(ctypes.addressof(ptrs), ew.ctypes.data, 2, x.ctypes.data, got.ctypes.data, D, I)
    ref = orc.expert_forward(blob, x, np.zeros(D, np.float32), 0.25, D, I)
    ref = orc.expert_forward(blob, x, ref, 0.5, D, I)
    assert close(got, ref)[0]


def test_device_plan_matches_host_call(tg):
    """tg_hip_moe_plan_* on HBM-resident weights == tg_moe_forward_rows_v2."""
    say("plan vs v2")
    import tinygiant_amd.synth as S
    n, k, D, I = 8, 1, 2048, 768
    g, u, d = _experts(n, D, I, O.FMT_Q4K, [O.FMT_Q6K] * n, 31)
    rng = np.random.default_rng(9)
    rw = S.router_weights(rng, n).reshape(n, 1)
    x = rng.standard_normal((k, D)).astype(np.float32)
    want = tg.moe_forward_rows_v2(g, u, d, O.FMT_Q4K, [O.FMT_Q6K] * n, None, None, None, O.ACT_SILU, rw, x,
                                  np.zeros((k, D), np.float32), I)
    L = tg.lib()
    bufs = [tg.DeviceArray(a.nbytes) for a in g + u + d]
    for b, a in zip(bufs, g + u + d):
        b.upload(a)
    gp = (ctypes.c_void_p * n)(*[b.ptr for b in bufs[:n]])
    up = (ctypes.c_void_p * n)(*[b.ptr for b in bufs[n:2 * n]])
    dp = (ctypes.c_void_p * n)(*[b.ptr for b in bufs[2 * n:]])
    fm = np.full(n, O.FMT_Q6K, np.int32)
    plan = L.tg_hip_moe_plan_create(ctypes.addressof(gp), ctypes.addressof(up), ctypes.addressof(dp), O.FMT_Q4K,
                                    fm.ctypes.data, None, None, None, O.ACT_SILU, n, rw.ctypes.data, k, D, I)
    assert plan
    xin = tg.DeviceArray(x.nbytes)
    xin.upload(x)
    out = tg.DeviceArray(x.nbytes)
    out.upload(np.zeros_like(x))
    L.tg_hip_moe_plan_run(plan, xin.ptr, out.ptr, None)
    L.tg_hip_synchronize()
    got = out.download(np.float32, k * D).reshape(k, D)
    L.tg_hip_moe_plan_destroy(plan)
    assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("kind,n", [(0, 144 * 1001), (2, 210 * 999), (3, 17 * 2001), (-1, 4099)])
def test_synth_fill_device_equals_host(tg, kind, n):
    say("synth", kind)
    buf = tg.DeviceArray(n + 64)
    tg.lib().tg_hip_synth_fill(kind, 777, buf.ptr, n, None)
    tg.lib().tg_hip_synchronize()
    assert np.array_equal(buf.download(np.uint8, n), tg.synth_host(kind, 777, n))
