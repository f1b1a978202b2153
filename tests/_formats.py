"""Independent numpy decoders of the weight block formats, written from the
byte layouts of csrc/libtinygiant.c (Q4_K :23,:210-222; Q6_K :24,:380-401;
MXFP4 :503-528; Q8_0 :572-590).  Used to brute-force integer dot sums and
dequantize-then-dot references; they share no code with the oracle."""

import numpy as np

KV = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12], np.int64)


def f16(u16):
    return np.asarray(u16, np.uint16).view(np.float16).astype(np.float32)


def q4k_decode(row, nb):
    """-> nib[nb,256] (0..15), sc[nb,8], m[nb,8], d[nb], dmin[nb]"""
    b = np.asarray(row, np.uint8).reshape(nb, 144)
    d = f16(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
    dmin = f16(b[:, 2].astype(np.uint16) | (b[:, 3].astype(np.uint16) << 8))
    s = b[:, 4:16].astype(np.int64)
    sc = np.zeros((nb, 8), np.int64)
    m = np.zeros((nb, 8), np.int64)
    for j in range(4):
        sc[:, j] = s[:, j] & 63
        m[:, j] = s[:, j + 4] & 63
    for j in range(4, 8):
        sc[:, j] = (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 6) << 4)
        m[:, j] = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    qs = b[:, 16:].astype(np.int64)
    nib = np.zeros((nb, 256), np.int64)
    for g in range(4):
        nib[:, 64 * g:64 * g + 32] = qs[:, 32 * g:32 * g + 32] & 0xF
        nib[:, 64 * g + 32:64 * g + 64] = qs[:, 32 * g:32 * g + 32] >> 4
    return nib, sc, m, d, dmin


def q6k_decode(row, nb):
    """-> q[nb,256] (-32..31), sc[nb,16] (int8), d[nb]"""
    b = np.asarray(row, np.uint8).reshape(nb, 210)
    ql = b[:, :128].astype(np.int64)
    qh = b[:, 128:192].astype(np.int64)
    sc = b[:, 192:208].view(np.int8).astype(np.int64)
    d = f16(b[:, 208].astype(np.uint16) | (b[:, 209].astype(np.uint16) << 8))
    q = np.zeros((nb, 256), np.int64)
    for h in range(2):
        for L in range(32):
            hh = qh[:, 32 * h + L]
            a, c = ql[:, 64 * h + L], ql[:, 64 * h + L + 32]
            q[:, 128 * h + L] = ((a & 15) | ((hh & 3) << 4)) - 32
            q[:, 128 * h + L + 32] = ((c & 15) | (((hh >> 2) & 3) << 4)) - 32
            q[:, 128 * h + L + 64] = ((a >> 4) | (((hh >> 4) & 3) << 4)) - 32
            q[:, 128 * h + L + 96] = ((c >> 4) | ((hh >> 6) << 4)) - 32
    return q, sc, d


def mxfp4_decode(row, nsub):
    """-> kv[nsub,32] (doubled e2m1 ints), e[nsub]"""
    b = np.asarray(row, np.uint8).reshape(nsub, 17)
    codes = b[:, 1:].astype(np.int64)
    v = np.concatenate([KV[codes & 15], KV[codes >> 4]], axis=1)
    return v, b[:, 0].astype(np.int64)


def q80_decode(row, nsub):
    b = np.asarray(row, np.uint8).reshape(nsub, 34)
    d = f16(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
    return b[:, 2:].view(np.int8).astype(np.int64), d


def q8_ints(xq):
    """flat int64 quants of a q8 row (structured blocks)"""
    return xq["qs"].reshape(-1).astype(np.int64)


def brute_isums(fmt, row, ncols, xq):
    """Per-sub-block integer sums, same indexing as or_isums / tg_hip_isums."""
    x = q8_ints(xq)
    if fmt == 0:
        nb = ncols // 256
        nib = q4k_decode(row, nb)[0]
        return (nib * x[:nb * 256].reshape(nb, 256)).reshape(nb, 8, 32).sum(-1).reshape(-1)
    if fmt == 2:
        nb = ncols // 256
        q = q6k_decode(row, nb)[0]
        return (q * x[:nb * 256].reshape(nb, 256)).reshape(nb, 16, 16).sum(-1).reshape(-1)
    if fmt == 3:
        v, _ = mxfp4_decode(row, ncols // 32)
        return (v * x[:ncols].reshape(-1, 32)).sum(-1)
    if fmt == 4:
        q, _ = q80_decode(row, ncols // 32)
        return (q * x[:ncols].reshape(-1, 32)).sum(-1)
    raise ValueError(fmt)


def dequant_row(fmt, row, ncols):
    """float64 dequantized weights (the reference test's dequant references,
    csrc/test_libtinygiant.c:111-130 and :520-532)."""
    if fmt == 0:
        nb = ncols // 256
        nib, sc, m, d, dmin = q4k_decode(row, nb)
        sc_e = np.repeat(sc, 32, axis=1)
        m_e = np.repeat(m, 32, axis=1)
        return (d[:, None].astype(np.float64) * sc_e * nib - dmin[:, None].astype(np.float64) * m_e).reshape(-1)
    if fmt == 2:
        nb = ncols // 256
        q, sc, d = q6k_decode(row, nb)
        return (d[:, None].astype(np.float64) * np.repeat(sc, 16, axis=1) * q).reshape(-1)
    if fmt == 3:
        v, e = mxfp4_decode(row, ncols // 32)
        return (np.ldexp(1.0, (e - 128).astype(np.int64))[:, None] * v).reshape(-1)
    if fmt == 4:
        q, d = q80_decode(row, ncols // 32)
        return (d[:, None].astype(np.float64) * q).reshape(-1)
    if fmt == 1:
        return np.asarray(row, np.uint8).view(np.float16).astype(np.float64)
    raise ValueError(fmt)
