"""Pins the CPU oracle (oracle/tg_oracle.c) before it is trusted as the
checker of the HIP path.

The reference ships no golden vectors (its tests draw inputs from libc
rand(), csrc/test_libtinygiant.c:94-130), and csrc/libtinygiant.c needs
<arm_neon.h>, which this x86 image lacks, so it cannot be built here.  Each
oracle function is therefore pinned by checks chosen so that a plausible
mistake fails one of them:
  * closed forms (f16 and e8m0 decode for every pattern, q8 special cases);
  * an independent numpy restatement (q8 quantizer; format decoders in
    tests/_formats.py written from the byte layouts, not from the oracle);
  * integer special cases where the float path must return the exact
    integer sum (d=1, dmin=0, unit sub-scales, x integer with amax=127);
  * the reference test's own invariants: dequantize-then-dot (Test 2, 9),
    x4 == x1 (Tests 5, 6), MoE == per-row expert composition (Test 7),
    MXFP4 + gpt-oss activation + biases vs float64 (Test 10), threaded ==
    serial (Test 8);
  * the SiLU activation on exactly known gate/up values (closed forms) and
    the Qwen3 expert path against a float64 dequantized model.
"""

import numpy as np
import pytest

import oracle as O
from tests import _formats as F

RNG = np.random.default_rng(20261201)


def test_f16_decode_every_pattern(orc):
    h = np.arange(65536, dtype=np.uint16)
    got = np.array([orc.f16_to_f32(int(v)) for v in h], np.float32)
    finite = ((h >> 10) & 0x1F) != 31
    ref = h.view(np.float16).astype(np.float32)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    # exponent 31: the reference's 32-bit shift yields 0xB7800000 | m << 13
    m = (h[~finite] & 0x3FF).astype(np.uint32)
    assert np.array_equal(got[~finite].view(np.uint32), np.uint32(0xB7800000) | (m << 13))


def test_e8m0_half_every_exponent(orc):
    for e in range(256):
        assert orc.e8m0_half(e) == np.float32(np.ldexp(1.0, e - 128)), e


def _numpy_q8(x):
    """Independent numpy restatement of quantize_q8 (csrc/libtinygiant.c:169-208)."""
    x = np.asarray(x, np.float32)
    n = x.shape[0]
    nb = (n + 255) // 256
    xp = np.zeros(nb * 256, np.float32)
    xp[:n] = x
    blocks = xp.reshape(nb, 256)
    amax = np.abs(blocks).max(axis=1).astype(np.float32)
    scale = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore", over="ignore"):
        inv = np.where(amax > 0, np.float32(127) / amax, np.float32(0)).astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        v = np.rint((blocks * inv[:, None]).astype(np.float32)).astype(np.float64)
    # AArch64 FCVTNS: saturate to int32, NaN -> 0; qs keeps the low byte
    v = np.where(np.isnan(v), 0.0, np.clip(v, -2.0 ** 31, 2.0 ** 31 - 1))
    q = v.astype(np.int64)
    bs = q.reshape(nb, 8, 32).sum(-1)
    wrap = lambda a: ((a + 2 ** 31) % 2 ** 32 - 2 ** 31).astype(np.int32)
    return scale, (q & 0xFF).astype(np.uint8).view(np.int8), wrap(bs), wrap(bs.sum(-1))


@pytest.mark.parametrize("n", [32, 256, 768, 2048, 2880])
def test_quantize_q8_matches_numpy(orc, n):
    for trial in range(5):
        x = (RNG.standard_normal(n) * 10 ** RNG.uniform(-3, 3)).astype(np.float32)
        if trial == 1:
            x[: n // 2] = 0.0
        if trial == 2:
            x = (x * np.float32(1e-42)).astype(np.float32)    # denormal blocks
        got = orc.quantize_q8(x)
        scale, q, bs, tot = _numpy_q8(x)
        assert np.array_equal(got["scale"].view(np.uint32), scale.view(np.uint32))
        assert np.array_equal(got["qs"], q)
        assert np.array_equal(got["bsums"], bs)
        assert np.array_equal(got["sum"], tot)


def test_quantize_q8_closed_forms(orc):
    z = orc.quantize_q8(np.zeros(256, np.float32))
    assert z["scale"] == 0 and not z["qs"].any() and not z["bsums"].any()
    # integer values with amax 127: scale 1, q == x
    x = RNG.integers(-127, 128, 512).astype(np.float32)
    x[3] = 127.0
    x[300] = -127.0
    q = orc.quantize_q8(x)
    assert np.all(q["scale"] == 1.0)
    assert np.array_equal(q["qs"].reshape(-1).astype(np.int64), x.astype(np.int64))
    # +-amax map to +-127; ties round half to even (x*inv = 0.5 and 1.5 exactly)
    y = np.zeros(256, np.float32)
    y[0], y[1], y[2], y[3] = 127.0, 0.5, 1.5, -2.5
    qy = orc.quantize_q8(y)["qs"].reshape(-1)
    assert list(qy[:4]) == [127, 0, 2, -2]
    # amax so small that 127/amax overflows: inv = inf, x*inv = +-inf saturates
    # to +-2^31 (low byte 0xFF / 0x00), zeros give NaN -> 0
    t = np.zeros(256, np.float32)
    t[0], t[1] = np.float32(1e-40), np.float32(-1e-40)
    qt = orc.quantize_q8(t)
    assert list(qt["qs"].reshape(-1)[:3]) == [-1, 0, 0]
    assert qt["bsums"].reshape(-1)[0] == np.int32(-1)      # INT32_MAX + INT32_MIN wraps to -1
    # partial last block (2880 = 11*256 + 64) is zero padded
    w = RNG.standard_normal(2880).astype(np.float32)
    qw = orc.quantize_q8(w)
    assert qw.shape == (12,) and not qw[11]["qs"][64:].any() and not qw[11]["bsums"][2:].any()


FMT_SHAPES = [(O.FMT_Q4K, 2048), (O.FMT_Q4K, 768), (O.FMT_Q6K, 768), (O.FMT_Q6K, 2048),
              (O.FMT_MXFP4, 2880), (O.FMT_Q80, 2880)]


def _rand_row(fmt, ncols, tg_synth=True):
    rb = O.row_bytes(fmt, ncols)
    row = RNG.integers(0, 256, rb, dtype=np.uint8)
    if fmt == O.FMT_Q4K:
        b = row.reshape(-1, 144)
        b[:, 0:2] = np.frombuffer(np.float16(RNG.uniform(1e-3, 2e-2)).tobytes(), np.uint8)
        b[:, 2:4] = np.frombuffer(np.float16(RNG.uniform(1e-3, 2e-2)).tobytes(), np.uint8)
    elif fmt == O.FMT_Q6K:
        b = row.reshape(-1, 210)
        b[:, 208:210] = np.frombuffer(np.float16(RNG.uniform(1e-3, 2e-2)).tobytes(), np.uint8)
    elif fmt == O.FMT_MXFP4:
        row.reshape(-1, 17)[:, 0] = RNG.integers(118, 131, ncols // 32)
    elif fmt == O.FMT_Q80:
        row.reshape(-1, 34)[:, 0:2] = np.frombuffer(np.float16(0.0625).tobytes(), np.uint8)
    return row


@pytest.mark.parametrize("fmt,ncols", FMT_SHAPES)
def test_isums_match_bruteforce(orc, fmt, ncols):
    for _ in range(4):
        row = _rand_row(fmt, ncols)
        x = RNG.standard_normal(ncols).astype(np.float32)
        got = orc.isums(fmt, row, 1, ncols, x)[0]
        ref = F.brute_isums(fmt, row, ncols, orc.quantize_q8(x))
        assert np.array_equal(got.astype(np.int64), ref)


def _unit_row(fmt, ncols):
    """Scales that make the float path return the exact integer sum."""
    rb = O.row_bytes(fmt, ncols)
    row = RNG.integers(0, 256, rb, dtype=np.uint8)
    if fmt == O.FMT_Q4K:
        b = row.reshape(-1, 144)
        b[:, 0:2] = [0x00, 0x3C]        # d = 1
        b[:, 2:4] = 0                   # dmin = 0
        b[:, 4:16] = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]   # sc = 1, m = 0 for all 8
    elif fmt == O.FMT_Q6K:
        b = row.reshape(-1, 210)
        b[:, 192:208] = 1
        b[:, 208:210] = [0x00, 0x3C]
    elif fmt == O.FMT_MXFP4:
        row.reshape(-1, 17)[:, 0] = 128
    elif fmt == O.FMT_Q80:
        row.reshape(-1, 34)[:, 0:2] = [0x00, 0x3C]
    return row


@pytest.mark.parametrize("fmt,ncols", FMT_SHAPES)
def test_float_dot_exact_on_integer_cases(orc, fmt, ncols):
    # x integer-valued with amax 127 => every q8 scale is 1 and q == x
    row = _unit_row(fmt, ncols)
    x = RNG.integers(-127, 128, ncols).astype(np.float32)
    x[::256] = 127.0
    xq = orc.quantize_q8(x)
    exact = F.brute_isums(fmt, row, ncols, xq).sum()
    # (MXFP4: e = 128 makes half(e) = 2^0, so the doubled table values are the weights)
    assert abs(exact) < 2 ** 24
    assert orc.dot(fmt, row, xq, ncols) == np.float32(exact)
    if fmt == O.FMT_Q4K:
        # dmin and m: dot = d*sc*isum - dmin*m*bsum, with dmin = 2, m = 3 on every sub-block
        r2 = row.copy().reshape(-1, 144)
        r2[:, 2:4] = [0x00, 0x40]
        r2[:, 8:12] = 3
        r2[:, 12:16] = 0x31
        bs = xq["bsums"].reshape(-1).astype(np.int64)[: ncols // 32]
        want = exact - 2.0 * 3.0 * bs.sum()
        assert orc.dot(fmt, r2.reshape(-1), xq, ncols) == np.float32(want)


@pytest.mark.parametrize("fmt,ncols", FMT_SHAPES)
def test_dequant_then_dot(orc, fmt, ncols):
    """Fused q8 dot == dequantized weights . dequantized q8 activations."""
    for _ in range(3):
        row = _rand_row(fmt, ncols)
        x = RNG.standard_normal(ncols).astype(np.float32)
        xq = orc.quantize_q8(x)
        xd = (F.q8_ints(xq).reshape(-1, 256) * xq["scale"][:, None].astype(np.float64)).reshape(-1)[:ncols]
        ref = float(F.dequant_row(fmt, row, ncols) @ xd)
        got = orc.dot(fmt, row, xq, ncols)
        scale = np.abs(F.dequant_row(fmt, row, ncols) * xd).sum()
        assert abs(got - ref) <= 2e-6 * scale + 1e-6, (got, ref)


@pytest.mark.parametrize("fmt,ncols", [(O.FMT_Q4K, 2048), (O.FMT_Q6K, 768), (O.FMT_MXFP4, 2880)])
def test_x4_matches_x1(orc, fmt, ncols):
    row = _rand_row(fmt, ncols)
    xs = [orc.quantize_q8(RNG.standard_normal(ncols).astype(np.float32) * 0.1) for _ in range(4)]
    o4 = orc.dot_x4(fmt, row, xs, ncols)
    for r in range(4):
        o1 = orc.dot(fmt, row, xs[r], ncols)
        assert abs(o1 - o4[r]) <= 1e-5 * max(abs(o1), 1e-3)


def test_f16_dot_vs_float64(orc):
    ncols = 768
    w = (RNG.standard_normal(ncols) * 0.05).astype(np.float16)
    x = RNG.standard_normal(ncols).astype(np.float32)
    got = orc.dot(O.FMT_F16, w.view(np.uint8), None, ncols, xf=x)
    ref = float(w.astype(np.float64) @ x.astype(np.float64))
    assert abs(got - ref) <= 1e-5 * np.abs(w.astype(np.float64) * x).sum()


def test_q4k_scalar_matches_dequant(orc):
    ncols, nrows = 512, 5
    mat = np.concatenate([_rand_row(O.FMT_Q4K, ncols) for _ in range(nrows)])
    x = (RNG.standard_normal(ncols) * 0.05).astype(np.float32)
    got = orc.matmul_q4k_scalar(mat, x, nrows, ncols)
    rb = O.row_bytes(O.FMT_Q4K, ncols)
    for r in range(nrows):
        w = F.dequant_row(O.FMT_Q4K, mat[r * rb:(r + 1) * rb], ncols)
        ref = float(w @ x)
        assert abs(got[r] - ref) <= 1e-4 * np.abs(w * x).sum()


def test_rms_norm_vs_float64(orc):
    x = RNG.standard_normal(2048).astype(np.float32)
    w = RNG.uniform(0.5, 1.5, 2048).astype(np.float32)
    got = orc.rms_norm(x, w, 1e-6)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd * xd).mean() + 1e-6) * w
    assert np.max(np.abs(got - ref)) <= 1e-6 * np.abs(ref).max()


def test_matmul_threaded_equals_serial(orc):
    """Reference Test 8: the row chunking is invisible in the result."""
    ncols, nrows = 2048, 300
    mat = np.concatenate([_rand_row(O.FMT_Q4K, ncols) for _ in range(nrows)])
    x = (RNG.standard_normal(ncols) * 0.02).astype(np.float32)
    orc.set_threads(1)
    o1 = orc.matmul(O.FMT_Q4K, mat, None, x, nrows, ncols)
    orc.set_threads(4)
    o4 = orc.matmul(O.FMT_Q4K, mat, None, x, nrows, ncols)
    orc.set_threads(1)
    assert np.array_equal(o1.view(np.uint32), o4.view(np.uint32))
    # and each row is the single-row dot plus bias
    bias = RNG.standard_normal(nrows).astype(np.float32)
    ob = orc.matmul(O.FMT_Q4K, mat, bias, x, nrows, ncols)
    xq = orc.quantize_q8(x)
    rb = O.row_bytes(O.FMT_Q4K, ncols)
    for r in (0, 7, 299):
        assert ob[r] == np.float32(orc.dot(O.FMT_Q4K, mat[r * rb:(r + 1) * rb], xq, ncols) + bias[r])


def _moe_weights(n, D, I, down_fmts, seed):
    rng = np.random.default_rng(seed)
    gates, ups, downs = [], [], []
    global RNG
    saved, RNG = RNG, rng
    try:
        for e in range(n):
            gates.append(np.concatenate([_rand_row(O.FMT_Q4K, D) for _ in range(I)]))
            ups.append(np.concatenate([_rand_row(O.FMT_Q4K, D) for _ in range(I)]))
            downs.append(np.concatenate([_rand_row(down_fmts[e], I) for _ in range(D)]))
    finally:
        RNG = saved
    return gates, ups, downs


def test_moe_v2_equals_per_row_expert_composition(orc):
    """Reference Test 7: tg_moe_forward_rows == per-row tg_expert_forward_mixed."""
    D, I, k, n = 512, 256, 6, 4
    fmts = [O.FMT_Q4K, O.FMT_Q6K, O.FMT_Q4K, O.FMT_Q6K]
    gates, ups, downs = _moe_weights(n, D, I, fmts, 7)
    x = (RNG.standard_normal((k, D)) * 0.5).astype(np.float32)
    rw = np.zeros((n, k), np.float32)
    for r in range(k):
        for j in range(3):
            rw[(r + 2 * j) % n, r] = 0.2 + 0.1 * j
    ref = np.zeros((k, D), np.float32)
    for r in range(k):
        for e in range(n):
            if rw[e, r] != 0:
                code = 2 if fmts[e] == O.FMT_Q6K else 0
                orc.expert_forward_mixed(gates[e], ups[e], downs[e], code, x[r], ref[r], rw[e, r], D, I)
    got = orc.moe_v2(gates, ups, downs, O.FMT_Q4K, fmts, None, None, None, O.ACT_SILU, rw, x,
                     np.zeros((k, D), np.float32), I)
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.abs(ref).max()
    # the single-row groups take the x1 kernels: rows alone must match exactly
    solo = orc.moe_v2(gates[:1], ups[:1], downs[:1], O.FMT_Q4K, fmts[:1], None, None, None,
                      O.ACT_SILU, rw[:1, :1], x[:1], np.zeros((1, D), np.float32), I)
    one = np.zeros(D, np.float32)
    orc.expert_forward_mixed(gates[0], ups[0], downs[0], 0, x[0], one, rw[0, 0], D, I)
    if rw[0, 0] != 0:
        assert np.array_equal(solo[0], one)


def test_moe_v2_mxfp4_gptoss_biases_vs_float64(orc):
    """Reference Test 10: MXFP4 experts, gpt-oss activation and biases against a
    float64 dequantized reference, within the q8 quantization error."""
    D = I = 2880      # 11 full q8 blocks + a zero-padded one
    k, n = 3, 2
    rng = np.random.default_rng(77)
    mats = []
    for e in range(n):
        trio = []
        for (nr, nc) in ((I, D), (I, D), (D, I)):
            m = rng.integers(0, 256, nr * nc // 32 * 17, dtype=np.uint8)
            m.reshape(-1, 17)[:, 0] = rng.integers(112, 118, nr * nc // 32)
            trio.append(m)
        mats.append(trio)
    bg = [rng.uniform(-0.5, 0.5, I).astype(np.float32) for _ in range(n)]
    bu = [rng.uniform(-0.5, 0.5, I).astype(np.float32) for _ in range(n)]
    bd = [rng.uniform(-0.05, 0.05, D).astype(np.float32) for _ in range(n)]
    x = rng.uniform(-1, 1, (k, D)).astype(np.float32)
    rw = np.array([[0.6, 0.0, 0.3], [0.4, 1.0, 0.7]], np.float32)
    got = orc.moe_v2([m[0] for m in mats], [m[1] for m in mats], [m[2] for m in mats], O.FMT_MXFP4,
                     [O.FMT_MXFP4] * n, bg, bu, bd, O.ACT_GPTOSS, rw, x, np.zeros((k, D), np.float32), I)
    ref = np.zeros((k, D))
    for e in range(n):
        G = F.dequant_row(O.FMT_MXFP4, mats[e][0], I * D).reshape(I, D)
        U = F.dequant_row(O.FMT_MXFP4, mats[e][1], I * D).reshape(I, D)
        Dn = F.dequant_row(O.FMT_MXFP4, mats[e][2], D * I).reshape(D, I)
        for r in range(k):
            if rw[e, r] == 0:
                continue
            g = G @ x[r] + bg[e]
            u = U @ x[r] + bu[e]
            g = np.minimum(g, 7.0)
            u = np.clip(u, -7.0, 7.0)
            h = g / (1 + np.exp(-1.702 * g)) * (u + 1)
            ref[r] += rw[e, r] * (Dn @ h + bd[e])
    assert np.max(np.abs(got - ref)) <= 0.03 * np.abs(ref).max()


def _silu64(g, u):
    """SiLU gating in float64: g * sigmoid(g) * u (csrc/libtinygiant.c:1256)."""
    g = np.asarray(g, np.float64)
    with np.errstate(over="ignore"):
        return g / (1.0 + np.exp(-g)) * np.asarray(u, np.float64)


def _q4k_one_hot_rows(rows, ncols, pos, nib):
    """Q4_K rows with d = 1, dmin = 0, unit sub-scales and every nibble 0
    except nibble nib[r] at column pos[r]: with an integer x of amax 127 the
    row's dot is exactly nib[r] * x[pos[r]]."""
    nb = ncols // 256
    m = np.zeros((rows, nb, 144), np.uint8)
    m[:, :, 0:2] = [0x00, 0x3C]
    m[:, :, 4:16] = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]
    for r in range(rows):
        b, p = divmod(int(pos[r]), 256)
        g, j = divmod(p, 64)
        if j < 32:
            m[r, b, 16 + 32 * g + j] |= np.uint8(nib[r])
        else:
            m[r, b, 16 + 32 * g + j - 32] |= np.uint8(nib[r] << 4)
    return m.reshape(-1)


def test_silu_activation_closed_form(orc):
    """The SiLU gating h = g / (1 + exp(-g)) * u of both oracle copies
    (act_fn of the MoE path and the inline one of tg_expert_forward_mixed,
    csrc/libtinygiant.c:1256 and :1105-1110) on exactly known g and u.

    Gate and up rows are one-hot Q4_K rows with unit scales and x is integer
    with amax 127, so every gate and up dot is an exact integer (g in
    [-150, 150], including 0).  The hidden values are read from the MoE
    path's stage hook and, through an F16 identity down matrix, from the
    single-expert path; both must equal the float64 formula to a few f32
    ulps.  Closed forms: g = 0 or u = 0 gives 0, g >> 0 gives g * u,
    g << 0 gives 0."""
    D = I = 256
    rng = np.random.default_rng(9)
    x = rng.integers(-10, 11, D).astype(np.float32)
    x[0] = 127.0
    x[1:6] = [0, 1, -1, 10, -10]
    pos_g = rng.integers(1, D, I)
    pos_u = rng.integers(1, D, I)
    nib_g = rng.integers(0, 16, I)
    nib_u = rng.integers(0, 16, I)
    # pinned rows: g = 0, u = 0, g = +150, g = -150, g = +-1
    pos_g[:6], nib_g[:6] = [1, 4, 4, 5, 2, 3], [7, 15, 15, 15, 1, 1]
    pos_u[:6], nib_u[:6] = [4, 1, 4, 2, 4, 4], [3, 9, 2, 5, 1, 1]
    gate = _q4k_one_hot_rows(I, D, pos_g, nib_g)
    up = _q4k_one_hot_rows(I, D, pos_u, nib_u)
    g = nib_g * x[pos_g].astype(np.float64)
    u = nib_u * x[pos_u].astype(np.float64)
    assert g[0] == 0 and u[1] == 0 and g[2] == 150 and g[3] == -150
    assert g.min() < -50 and g.max() > 50 and np.count_nonzero(np.abs(g) < 4) > 8
    ref = _silu64(g, u)
    down_q6 = _rand_row(O.FMT_Q6K, I)
    down_q6 = np.concatenate([down_q6] * D)
    hid = np.zeros((1, I), np.float32)
    orc.moe_v2([gate], [up], [down_q6], O.FMT_Q4K, [O.FMT_Q6K], None, None, None, O.ACT_SILU,
               np.ones((1, 1), np.float32), x.reshape(1, D), np.zeros((1, D), np.float32), I, hidden_out=hid)
    tol = 4 * np.finfo(np.float32).eps * np.abs(ref) + 1e-30
    assert np.all(np.abs(hid[0] - ref) <= tol)
    assert hid[0, 0] == 0 and hid[0, 1] == 0 and hid[0, 2] == np.float32(150 * u[2])
    assert abs(hid[0, 3]) < 1e-30
    # the single-expert path's inline SiLU, read through an F16 identity down
    eye = np.eye(D, I, dtype=np.float16).view(np.uint8).reshape(-1)
    out = np.zeros(D, np.float32)
    orc.expert_forward_mixed(gate, up, eye, 1, x, out, 1.0, D, I)
    assert np.all(np.abs(out - ref) <= tol)
    assert out[0] == 0 and out[1] == 0 and out[2] == np.float32(150 * u[2])


def test_moe_v2_silu_q4k_q6k_vs_float64(orc):
    """The Qwen3 expert path (q4_K gate/up, q6_K down, SiLU, router-weighted
    combine; csrc/libtinygiant.c:1279-1437) against a float64 dequantized
    model, within the q8 quantization error (the bound of reference Test 10).
    The inputs are scaled so the gate values span the SiLU's curved range,
    and the test checks that a sign error in the activation (g * sigmoid(-g))
    or swapped gate and up operands would miss the bar."""
    D, I, k, n = 512, 256, 3, 3
    gates, ups, downs = _moe_weights(n, D, I, [O.FMT_Q6K] * n, 41)
    rng = np.random.default_rng(42)
    x = (rng.standard_normal((k, D)) * 0.04).astype(np.float32)
    rw = np.array([[0.5, 0.0, 0.2], [0.3, 0.6, 0.0], [0.2, 0.4, 0.8]], np.float32)
    got = orc.moe_v2(gates, ups, downs, O.FMT_Q4K, [O.FMT_Q6K] * n, None, None, None, O.ACT_SILU, rw, x,
                     np.zeros((k, D), np.float32), I)
    ref = np.zeros((k, D))
    flip = np.zeros((k, D))
    swap = np.zeros((k, D))
    gs = []
    for e in range(n):
        G = F.dequant_row(O.FMT_Q4K, gates[e], I * D).reshape(I, D)
        U = F.dequant_row(O.FMT_Q4K, ups[e], I * D).reshape(I, D)
        Dn = F.dequant_row(O.FMT_Q6K, downs[e], D * I).reshape(D, I)
        for r in range(k):
            if rw[e, r] == 0:
                continue
            g, u = G @ x[r], U @ x[r]
            gs.append(g)
            ref[r] += rw[e, r] * (Dn @ _silu64(g, u))
            flip[r] += rw[e, r] * (Dn @ (g / (1.0 + np.exp(g)) * u))
            swap[r] += rw[e, r] * (Dn @ _silu64(u, g))
    gs = np.concatenate(gs)
    assert 1.0 < np.std(gs) < 20.0, np.std(gs)
    bar = 0.03 * np.abs(ref).max()
    assert np.max(np.abs(got - ref)) <= bar
    assert np.max(np.abs(flip - ref)) > 5 * bar and np.max(np.abs(swap - ref)) > 5 * bar


def test_moe_v2_skips_exact_zero_and_accumulates(orc):
    D, I, k, n = 512, 256, 2, 2
    gates, ups, downs = _moe_weights(n, D, I, [O.FMT_Q6K] * n, 3)
    x = RNG.standard_normal((k, D)).astype(np.float32)
    base = RNG.standard_normal((k, D)).astype(np.float32)
    rw = np.array([[0.5, 0.0], [0.0, 0.0]], np.float32)
    out = orc.moe_v2(gates, ups, downs, O.FMT_Q4K, [O.FMT_Q6K] * n, None, None, None, O.ACT_SILU, rw, x,
                     base.copy(), I)
    assert np.array_equal(out[1], base[1])         # row 1 has no expert: untouched
    only = orc.moe_v2(gates[:1], ups[:1], downs[:1], O.FMT_Q4K, [O.FMT_Q6K], None, None, None, O.ACT_SILU,
                      rw[:1, :1], x[:1], np.zeros((1, D), np.float32), I)
    assert np.array_equal(out[0], base[0] + only[0])


def test_route_oracle_selection_and_softmax(orc):
    """The router restatement against a full sort and softmax closed forms."""
    rng = np.random.default_rng(5)
    for n_exp, dim, top_k in ((16, 32, 4), (128, 64, 8), (32, 16, 1)):
        router = rng.standard_normal((n_exp, dim)).astype(np.float32)
        x = rng.standard_normal(dim).astype(np.float32)
        bias = rng.standard_normal(n_exp).astype(np.float32)
        logits, idx, w = orc.route(router, bias, x, top_k)
        full = np.argsort(-logits.astype(np.float64), kind="stable")
        assert list(idx) == list(full[:top_k])
        assert np.allclose(logits, router.astype(np.float64) @ x.astype(np.float64) + bias, rtol=1e-5, atol=1e-5)
        assert abs(float(w.sum()) - 1.0) < 1e-6
        assert np.all(np.diff(w) <= 0)
        ref = np.exp(logits[idx].astype(np.float64) - logits[idx].max())
        assert np.allclose(w, ref / ref.sum(), rtol=1e-6, atol=1e-7)
    # equal logits get equal weights
    router = np.ones((8, 4), np.float32)
    _, idx, w = orc.route(router, None, np.ones(4, np.float32), 4)
    assert np.allclose(w, 0.25)



def test_route_oracle_restricted_selection(orc):
    """Router.select(restrict=True) (tinygiant/router.py:46-54): the top_k of
    the resident experts by a brute-force filter of the fully sorted logits,
    weights equal to an unrestricted route over just those experts' rows
    (the softmax of their own logits), and the unrestricted selection when
    fewer than top_k experts are resident."""
    rng = np.random.default_rng(11)
    for n_exp, dim, top_k, n_res in ((128, 64, 8, 64), (32, 16, 4, 5), (16, 8, 2, 2)):
        router = rng.standard_normal((n_exp, dim)).astype(np.float32)
        bias = rng.standard_normal(n_exp).astype(np.float32)
        x = rng.standard_normal(dim).astype(np.float32)
        resident = np.zeros(n_exp, bool)
        resident[rng.choice(n_exp, n_res, replace=False)] = True
        logits, idx, w = orc.route(router, bias, x, top_k, resident=resident)
        full = np.argsort(-logits.astype(np.float64), kind="stable")
        assert list(idx) == [e for e in full if resident[e]][:top_k]
        sub = np.flatnonzero(resident)
        _, sidx, sw = orc.route(router[sub], bias[sub], x, top_k)
        assert list(sub[sidx]) == list(idx)
        assert np.array_equal(sw, w)
    # fewer resident experts than top_k: unrestricted
    router = rng.standard_normal((16, 8)).astype(np.float32)
    x = rng.standard_normal(8).astype(np.float32)
    resident = np.zeros(16, bool)
    resident[:3] = True
    a = orc.route(router, None, x, 4, resident=resident)
    b = orc.route(router, None, x, 4)
    assert list(a[1]) == list(b[1]) and np.array_equal(a[2], b[2])

# ---- decode attention (tg_attention_v2, csrc/libtinygiant.c:939-983) ----

def _attn_case(seed, D=256, nh=8, nkv=2, hd=32, kv_max=40, kv_len=17, zero_q=False, bias=True, norms=True):
    """F16 projections (exact f32 dots), random cache rows below kv_len, RoPE
    tables of a 10000-base NeoX rotation."""
    rng = np.random.default_rng(seed)
    qd, kd = nh * hd, nkv * hd

    def f16(rows, cols, scale=0.1):
        return (rng.standard_normal((rows, cols)) * scale).astype(np.float16).view(np.uint8).reshape(-1)

    w = [np.zeros(qd * D * 2, np.uint8) if zero_q else f16(qd, D), f16(kd, D), f16(kd, D), f16(D, qd)]
    b = [rng.standard_normal(n).astype(np.float32) * 0.1 for n in (qd, kd, kd, D)] if bias else None
    if zero_q and b is not None:
        b[0] = np.zeros(qd, np.float32)
    qn = rng.uniform(0.5, 1.5, hd).astype(np.float32) if norms else None
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32) if norms else None
    half = hd // 2
    ang = np.arange(kv_max)[:, None] / (10000.0 ** (np.arange(half)[None, :] * 2.0 / hd))
    rc, rs = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    kv_k = np.zeros((nkv, kv_max, hd), np.float32)
    kv_v = np.zeros((nkv, kv_max, hd), np.float32)
    kv_k[:, :kv_len] = rng.standard_normal((nkv, kv_len, hd))
    kv_v[:, :kv_len] = rng.standard_normal((nkv, kv_len, hd))
    x = rng.standard_normal(D).astype(np.float32)
    return dict(w=w, b=b, qn=qn, kn=kn, rc=rc, rs=rs, kv_k=kv_k, kv_v=kv_v, x=x, D=D, nh=nh, nkv=nkv, hd=hd,
                kv_max=kv_max, kv_len=kv_len)


def _attn_run(orc, c, window=0, sinks=None, rc=None, rs=None):
    F16 = O.FMT_F16
    return orc.attention_v2((F16,) * 4, c["w"], c["b"], c["qn"], c["kn"], sinks, c["kv_k"], c["kv_v"], c["kv_len"],
                            c["kv_max"], window, c["rc"] if rc is None else rc, c["rs"] if rs is None else rs, c["x"],
                            c["D"], c["nh"], c["nkv"], c["hd"], c["kv_len"], 1e-6)


def _proj64(c, i, rows):
    m = c["w"][i].view(np.float16).astype(np.float64).reshape(rows, -1)
    inp = c["x"].astype(np.float64)
    y = m @ inp
    return y + (c["b"][i] if c["b"] is not None else 0.0)


def test_attention_one_position_returns_v(orc):
    """kv_len 0: the softmax over one position is 1, so each head's output is
    its KV head's new V row, exactly."""
    c = _attn_case(1, kv_len=0)
    _, att = _attn_run(orc, c)
    ratio = c["nh"] // c["nkv"]
    for h in range(c["nh"]):
        assert np.array_equal(att[h * c["hd"]:(h + 1) * c["hd"]], c["kv_v"][h // ratio, 0])


def test_attention_zero_query_is_mean_of_v(orc):
    """Zero Q weights and bias: every score is 0, the softmax is uniform and
    each head's output is the mean of its KV head's V rows in the window."""
    for window in (0, 6):
        c = _attn_case(2, zero_q=True)
        _, att = _attn_run(orc, c, window=window)
        seq = c["kv_len"] + 1
        start = seq - window if window and seq > window else 0
        ratio = c["nh"] // c["nkv"]
        for h in range(c["nh"]):
            want = c["kv_v"][h // ratio, start:seq].astype(np.float64).mean(axis=0)
            assert np.abs(att[h * c["hd"]:(h + 1) * c["hd"]] - want).max() < 1e-5


def test_attention_window_one_and_huge_sink(orc):
    """A window of 1 attends only the new row (output = new V exactly); a sink
    logit far above every score takes all the weight (output 0)."""
    c = _attn_case(3)
    _, att = _attn_run(orc, c, window=1)
    ratio = c["nh"] // c["nkv"]
    for h in range(c["nh"]):
        assert np.array_equal(att[h * c["hd"]:(h + 1) * c["hd"]], c["kv_v"][h // ratio, c["kv_len"]])
    c = _attn_case(3)
    _, att = _attn_run(orc, c, sinks=np.full(c["nh"], 1e4, np.float32))
    assert np.abs(att).max() == 0.0


def test_attention_unit_rope_stores_normed_k(orc):
    """cos 1 / sin 0 tables make RoPE the identity: the stored K row is the
    QK-normed projection (float64 within 1e-5)."""
    c = _attn_case(4)
    ones = np.ones_like(c["rc"])
    zeros = np.zeros_like(c["rs"])
    _attn_run(orc, c, rc=ones, rs=zeros)
    k = _proj64(c, 1, c["nkv"] * c["hd"]).reshape(c["nkv"], c["hd"])
    k = k / np.sqrt((k * k).mean(axis=1, keepdims=True) + 1e-6) * c["kn"].astype(np.float64)
    assert np.abs(c["kv_k"][:, c["kv_len"]] - k).max() < 1e-5 * np.abs(k).max()
    v = _proj64(c, 2, c["nkv"] * c["hd"]).reshape(c["nkv"], c["hd"])
    assert np.abs(c["kv_v"][:, c["kv_len"]] - v).max() < 1e-5 * np.abs(v).max()


@pytest.mark.parametrize("window,sink", [(0, False), (9, True)])
def test_attention_vs_float64(orc, window, sink):
    """The whole step against a float64 restatement: projections, QK norm,
    RoPE as complex rotation, GQA head mapping, window, sinks, output
    projection of the attention output."""
    c = _attn_case(5 + window)
    nh, nkv, hd, L = c["nh"], c["nkv"], c["hd"], c["kv_len"]
    sinks = np.random.default_rng(7).standard_normal(nh).astype(np.float32) if sink else None
    cache_k, cache_v = c["kv_k"].astype(np.float64), c["kv_v"].astype(np.float64)
    out, att = _attn_run(orc, c, window=window, sinks=sinks)
    q = _proj64(c, 0, nh * hd).reshape(nh, hd)
    k = _proj64(c, 1, nkv * hd).reshape(nkv, hd)
    v = _proj64(c, 2, nkv * hd).reshape(nkv, hd)
    q = q / np.sqrt((q * q).mean(axis=1, keepdims=True) + 1e-6) * c["qn"]
    k = k / np.sqrt((k * k).mean(axis=1, keepdims=True) + 1e-6) * c["kn"]
    half = hd // 2
    rot = c["rc"][L].astype(np.float64) + 1j * c["rs"][L].astype(np.float64)

    def rope(a):
        z = (a[:, :half] + 1j * a[:, half:]) * rot
        return np.concatenate([z.real, z.imag], axis=1)

    q, k = rope(q), rope(k)
    cache_k[:, L], cache_v[:, L] = k, v
    seq = L + 1
    start = seq - window if window and seq > window else 0
    att64 = np.zeros((nh, hd))
    for h in range(nh):
        s = cache_k[h // (nh // nkv), start:seq] @ q[h] / np.sqrt(hd)
        logits = np.concatenate([s, [sinks[h]]]) if sink else s
        p = np.exp(logits - logits.max())
        p = p / p.sum()
        att64[h] = p[:len(s)] @ cache_v[h // (nh // nkv), start:seq]
    assert np.abs(att - att64.reshape(-1)).max() < 1e-5 * np.abs(att64).max()
    assert np.abs(c["kv_k"][:, L] - k).max() < 1e-5 * np.abs(k).max()
    o = c["w"][3].view(np.float16).astype(np.float64).reshape(c["D"], -1) @ att.astype(np.float64) + c["b"][3]
    assert np.abs(out - o).max() < 1e-5 * np.abs(o).max()
