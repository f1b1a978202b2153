/*
 * tg_oracle.c -- CPU restatement (test infrastructure only) of the reference
 * arithmetic in csrc/libtinygiant.c.  See tg_oracle.h for the rules of use.
 *
 * Build: make -C oracle   (gcc -O2 -ffp-contract=off -fopenmp, no fast-math)
 *
 * Parity status of each function is recorded next to it ("pinned by ...").
 * Integer results are exact restatements; float results follow the
 * reference's expression grouping so that only FMA contraction (Apple clang
 * contracts, this build does not) and libm expf differ from a reference build.
 */
#include "tg_oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK 256
#define Q4K_BYTES 144
#define Q6K_BYTES 210
#define MXFP4_BYTES 17
#define Q80_BYTES 34
#define MM_ROWS 64          /* csrc/libtinygiant.c:341 */
#define MOE_I_ROWS 96       /* csrc/libtinygiant.c:1245 */
#define MOE_D_ROWS 256      /* csrc/libtinygiant.c:1246 */

static int g_threads = 1;

void or_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int or_get_threads(void) { return g_threads; }

int or_q8_nblocks(int ncols) { return (ncols + QK - 1) / QK; }

static void die(const char *msg) {
    fprintf(stderr, "tg_oracle: %s\n", msg);
    abort();
}

/* Restates f16_to_f32 (csrc/libtinygiant.c:128-137) bit for bit, including
 * its exponent-31 path, which builds (255+112)<<23 in 32-bit unsigned
 * arithmetic (the sign bit is set by the overflow).
 * Pinned by: exhaustive comparison with numpy float16 for every finite
 * pattern (tests/test_oracle_pins.py). */
float or_f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0) {
        if (m == 0) {
            float r;
            memcpy(&r, &s, 4);
            return r;
        }
        while (!(m & 0x400u)) {
            m <<= 1;
            e--;
        }
        e++;
        m &= ~0x400u;
    } else if (e == 31) {
        e = 255;
    }
    uint32_t f = s | ((e + 112u) << 23) | (m << 13);
    float r;
    memcpy(&r, &f, 4);
    return r;
}

/* Restates get_scale_min_k4 (csrc/libtinygiant.c:146-155).
 * Pinned by: the dequantize-then-dot identity and the d=1/dmin=0 integer
 * special cases in tests/test_oracle_pins.py. */
void or_get_scale_min_k4(int j, const uint8_t *s, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* Restates e8m0_to_fp32_half (csrc/libtinygiant.c:516-519): 2^(e-128),
 * with e<2 built as the denormal 0x00200000<<e.
 * Pinned by: closed form ldexp(1, e-128) for every e (tests). */
float or_e8m0_half(uint8_t e) {
    uint32_t bits = e < 2 ? (0x00200000u << e) : ((uint32_t)(e - 1) << 23);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Restates fmt_row_bytes (csrc/libtinygiant.c:596-604). */
size_t or_row_bytes(int fmt, int ncols) {
    switch (fmt) {
        case OR_FMT_Q4K: return (size_t)(ncols / QK) * Q4K_BYTES;
        case OR_FMT_Q6K: return (size_t)(ncols / QK) * Q6K_BYTES;
        case OR_FMT_MXFP4: return (size_t)(ncols / 32) * MXFP4_BYTES;
        case OR_FMT_Q80: return (size_t)(ncols / 32) * Q80_BYTES;
        default: return (size_t)ncols * 2;
    }
}

/* vcvtnq_s32_f32: round to nearest (ties to even), saturate to int32,
 * NaN -> 0 (the AArch64 FCVTNS rule the reference relies on at :194). */
static int32_t cvtn_s32(float v) {
    if (v != v) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)rintf(v);
}

/* Restates quantize_q8 (csrc/libtinygiant.c:169-208): per 256-block,
 * amax = max|x|, scale = amax/127 (correctly rounded f32 division),
 * inv = amax>0 ? 127/amax : 0, q = round-half-even(x*inv), 32-element
 * sub-block sums, zero-filled padding past ncols (ncols % 32 == 0).
 * Pinned by: closed-form special cases (amax 0, values at +-amax, integer
 * inputs with amax 127) and an independent numpy restatement (tests). */
void or_quantize_q8(const float *x, or_q8_block *out, int ncols) {
    if (ncols % 32) die("quantize_q8: ncols must be a multiple of 32");
    int nb = or_q8_nblocks(ncols);
    for (int b = 0; b < nb; b++) {
        const float *xb = x + (size_t)b * QK;
        int n = ncols - b * QK < QK ? ncols - b * QK : QK;
        float amax = 0.f;
        for (int i = 0; i < n; i++) {
            float a = fabsf(xb[i]);
            amax = a > amax ? a : amax;
        }
        float sc = amax / 127.f;
        float inv = amax > 0 ? 127.f / amax : 0.f;
        out[b].scale = sc;
        /* sums wrap like the reference's vaddq_s32; qs keeps the low byte of
         * the 32-bit value (vmovn_s32 then vmovn_s16 truncate) */
        uint32_t total = 0;
        for (int j = 0; j < 8; j++) {
            uint32_t s = 0;
            if (j * 32 < n) {
                for (int i = j * 32; i < (j + 1) * 32; i++) {
                    float v = xb[i] * inv;
                    int32_t q = cvtn_s32(v);
                    out[b].qs[i] = (int8_t)(uint8_t)((uint32_t)q & 0xFFu);
                    s += (uint32_t)q;
                }
            } else {
                memset(out[b].qs + j * 32, 0, 32);
            }
            out[b].bsums[j] = (int32_t)s;
            total += s;
        }
        out[b].sum = (int32_t)total;
    }
}

/* ---- Q4_K (csrc/libtinygiant.c:223-337) ---- */

static int32_t q4k_isum(const uint8_t *qs, const int8_t *xq, int sub) {
    /* sub-block `sub` of a block: group g = sub/2, lo nibbles for even sub,
     * hi nibbles for odd sub, paired with xq[32*sub .. 32*sub+31] */
    int g = sub >> 1, hi = sub & 1;
    int32_t acc = 0;
    for (int j = 0; j < 32; j++) {
        int v = hi ? (qs[32 * g + j] >> 4) : (qs[32 * g + j] & 0xF);
        acc += v * (int32_t)xq[32 * sub + j];
    }
    return acc;
}

/* Restates dot_q4k_q8 (:223-272).  Pinned by: integer special cases
 * (d=1, dmin=0, sc=1 => output equals the exact integer sum), dequant-then-dot
 * identity (reference Test 2), brute-force numpy integer GEMV (tests). */
float or_dot_q4k_q8(const uint8_t *row, const or_q8_block *xq, int bpr) {
    float total = 0;
    for (int b = 0; b < bpr; b++) {
        const uint8_t *bl = row + (size_t)b * Q4K_BYTES;
        uint16_t dr, dmr;
        memcpy(&dr, bl, 2);
        memcpy(&dmr, bl + 2, 2);
        float d = or_f16_to_f32(dr), dmin = or_f16_to_f32(dmr);
        const uint8_t *scales = bl + 4, *qs = bl + 16;
        float block_sum = 0;
        for (int g = 0; g < 4; g++) {
            uint8_t sc_lo, m_lo, sc_hi, m_hi;
            or_get_scale_min_k4(2 * g, scales, &sc_lo, &m_lo);
            or_get_scale_min_k4(2 * g + 1, scales, &sc_hi, &m_hi);
            int32_t ilo = q4k_isum(qs, xq[b].qs, 2 * g);
            int32_t ihi = q4k_isum(qs, xq[b].qs, 2 * g + 1);
            block_sum += d * (float)sc_lo * (float)ilo - dmin * (float)m_lo * (float)xq[b].bsums[2 * g];
            block_sum += d * (float)sc_hi * (float)ihi - dmin * (float)m_hi * (float)xq[b].bsums[2 * g + 1];
        }
        total += xq[b].scale * block_sum;
    }
    return total;
}

/* Restates dot_q4k_q8_x4 (:276-337): same integers, one 4-term float
 * expression per group. Pinned by: x4 == x1 within 1e-5 (reference Test 5)
 * and exact equality on the integer special cases. */
void or_dot_q4k_q8_x4(const uint8_t *row, const or_q8_block *const xq[4], int bpr, float out[4]) {
    float tot[4] = {0, 0, 0, 0};
    for (int b = 0; b < bpr; b++) {
        const uint8_t *bl = row + (size_t)b * Q4K_BYTES;
        uint16_t dr, dmr;
        memcpy(&dr, bl, 2);
        memcpy(&dmr, bl + 2, 2);
        float d = or_f16_to_f32(dr), dmin = or_f16_to_f32(dmr);
        const uint8_t *scales = bl + 4, *qs = bl + 16;
        float bs[4] = {0, 0, 0, 0};
        for (int g = 0; g < 4; g++) {
            uint8_t sc_lo, m_lo, sc_hi, m_hi;
            or_get_scale_min_k4(2 * g, scales, &sc_lo, &m_lo);
            or_get_scale_min_k4(2 * g + 1, scales, &sc_hi, &m_hi);
            float dsl = d * (float)sc_lo, dml = dmin * (float)m_lo;
            float dsh = d * (float)sc_hi, dmh = dmin * (float)m_hi;
            for (int r = 0; r < 4; r++) {
                const or_q8_block *x = &xq[r][b];
                int32_t ilo = q4k_isum(qs, x->qs, 2 * g);
                int32_t ihi = q4k_isum(qs, x->qs, 2 * g + 1);
                bs[r] += dsl * (float)ilo - dml * (float)x->bsums[2 * g]
                       + dsh * (float)ihi - dmh * (float)x->bsums[2 * g + 1];
            }
        }
        for (int r = 0; r < 4; r++) tot[r] += xq[r][b].scale * bs[r];
    }
    for (int r = 0; r < 4; r++) out[r] = tot[r];
}

/* ---- Q6_K (csrc/libtinygiant.c:384-487) ---- */

/* 6-bit value of element e (0..255) of a Q6_K block, minus 32. */
static int q6k_val(const uint8_t *bl, int e) {
    const uint8_t *ql = bl, *qh = bl + 128;
    int h = e >> 7, r = e & 127;      /* half, position within half */
    int q = r >> 5, L = r & 31;       /* quarter (q1..q4), lane 0..31 */
    uint8_t lq = ql[64 * h + L + ((q & 1) ? 32 : 0)];
    int low = (q & 2) ? (lq >> 4) : (lq & 0xF);
    int high = (qh[32 * h + L] >> (2 * q)) & 3;
    return (low | (high << 4)) - 32;
}

/* Integer sum of the 16-element group s (elements 16s..16s+15), whose scale
 * is sc[s]: the reference's d1..d4 for (half, l) map to s = 8h + l/16 + 2q. */
static int32_t q6k_isum(const uint8_t *bl, const int8_t *xq, int s) {
    int32_t acc = 0;
    for (int i = 0; i < 16; i++) acc += q6k_val(bl, 16 * s + i) * (int32_t)xq[16 * s + i];
    return acc;
}

/* Restates dot_q6k_q8 (:403-443): block_sum accumulates sc*isum in the
 * order half -> l (0,16) -> d1..d4; total += d*sx*block_sum.
 * Pinned by: integer special cases (d=1, sc=1), dequant-then-dot identity,
 * the reference's own byte-loop scalar restatement
 * (csrc/test_libtinygiant.c:64-92) re-derived independently in numpy (tests). */
float or_dot_q6k_q8(const uint8_t *row, const or_q8_block *xq, int bpr) {
    float total = 0;
    for (int b = 0; b < bpr; b++) {
        const uint8_t *bl = row + (size_t)b * Q6K_BYTES;
        const int8_t *sc = (const int8_t *)(bl + 192);
        uint16_t dr;
        memcpy(&dr, bl + 208, 2);
        float d = or_f16_to_f32(dr);
        float block_sum = 0;
        for (int h = 0; h < 2; h++)
            for (int l = 0; l < 32; l += 16)
                for (int q = 0; q < 4; q++) {
                    int s = 8 * h + l / 16 + 2 * q;
                    block_sum += (float)sc[s] * (float)q6k_isum(bl, xq[b].qs, s);
                }
        total += d * xq[b].scale * block_sum;
    }
    return total;
}

/* Restates dot_q6k_q8_x4 (:445-487); float order per row equals x1. */
void or_dot_q6k_q8_x4(const uint8_t *row, const or_q8_block *const xq[4], int bpr, float out[4]) {
    for (int r = 0; r < 4; r++) out[r] = or_dot_q6k_q8(row, xq[r], bpr);
}

/* ---- MXFP4 (csrc/libtinygiant.c:511-570) ---- */

static const int8_t kv_mxfp4[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

static int32_t mxfp4_isum(const uint8_t *bl, const int8_t *xqs) {
    int32_t acc = 0;
    for (int i = 0; i < 16; i++) {
        acc += kv_mxfp4[bl[1 + i] & 0xF] * (int32_t)xqs[i];
        acc += kv_mxfp4[bl[1 + i] >> 4] * (int32_t)xqs[16 + i];
    }
    return acc;
}

/* Restates dot_mxfp4_q8 (:533-547): sub-block s uses q8 block s>>3 at
 * offset (s&7)*32; total += scale*half(e)*acc.
 * Pinned by: e=128 integer special case, dequant-then-dot (reference Test 9). */
float or_dot_mxfp4_q8(const uint8_t *row, const or_q8_block *xq, int ncols) {
    int n_sub = ncols / 32;
    float total = 0;
    for (int s = 0; s < n_sub; s++) {
        const or_q8_block *xb = &xq[s >> 3];
        const uint8_t *bl = row + (size_t)s * MXFP4_BYTES;
        int32_t acc = mxfp4_isum(bl, xb->qs + (s & 7) * 32);
        total += xb->scale * or_e8m0_half(bl[0]) * (float)acc;
    }
    return total;
}

void or_dot_mxfp4_q8_x4(const uint8_t *row, const or_q8_block *const xq[4], int ncols, float out[4]) {
    for (int r = 0; r < 4; r++) out[r] = or_dot_mxfp4_q8(row, xq[r], ncols);
}

/* Restates dot_q80_q8 (:576-590). Pinned by: dequant-then-dot (Test 9). */
float or_dot_q80_q8(const uint8_t *row, const or_q8_block *xq, int ncols) {
    int n_sub = ncols / 32;
    float total = 0;
    for (int s = 0; s < n_sub; s++) {
        const or_q8_block *xb = &xq[s >> 3];
        const int8_t *xqs = xb->qs + (s & 7) * 32;
        const uint8_t *bl = row + (size_t)s * Q80_BYTES;
        uint16_t dr;
        memcpy(&dr, bl, 2);
        int32_t acc = 0;
        for (int i = 0; i < 32; i++) acc += (int32_t)(int8_t)bl[2 + i] * (int32_t)xqs[i];
        total += xb->scale * or_f16_to_f32(dr) * (float)acc;
    }
    return total;
}

/* IEEE half -> float (what vcvt_f32_f16 does in the vector loop below). */
static float ieee_f16(uint16_t h) {
    if (((h >> 10) & 0x1F) == 31) {
        uint32_t f = ((uint32_t)(h & 0x8000u) << 16) | 0x7F800000u | ((uint32_t)(h & 0x3FFu) << 13);
        float r;
        memcpy(&r, &f, 4);
        return r;
    }
    return or_f16_to_f32(h);
}

/* Restates matvec_f16 for one row (csrc/libtinygiant.c:635-653): eight fused
 * lane accumulators (two float32x4 FMA chains over steps of 8) using the
 * IEEE conversion, the lanes summed as vaddvq_f32(acc0 + acc1) =
 * ((l0+l1)+(l2+l3)), then a scalar tail through f16_to_f32.
 * Pinned by: float64 dot within 1e-5 relative (tests). */
float or_dot_f16(const uint16_t *row, const float *x, int ncols) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 7 < ncols; i += 8)
        for (int l = 0; l < 8; l++) acc[l] = fmaf(ieee_f16(row[i + l]), x[i + l], acc[l]);
    float t0 = acc[0] + acc[4], t1 = acc[1] + acc[5], t2 = acc[2] + acc[6], t3 = acc[3] + acc[7];
    float sum = (t0 + t1) + (t2 + t3);
    for (; i < ncols; i++) sum += or_f16_to_f32(row[i]) * x[i];
    return sum;
}

int or_isums(int fmt, const uint8_t *row, const or_q8_block *xq, int ncols, int32_t *out) {
    int n = 0;
    if (fmt == OR_FMT_Q4K) {
        for (int b = 0; b < ncols / QK; b++)
            for (int s = 0; s < 8; s++) out[n++] = q4k_isum(row + (size_t)b * Q4K_BYTES + 16, xq[b].qs, s);
    } else if (fmt == OR_FMT_Q6K) {
        for (int b = 0; b < ncols / QK; b++)
            for (int s = 0; s < 16; s++) out[n++] = q6k_isum(row + (size_t)b * Q6K_BYTES, xq[b].qs, s);
    } else if (fmt == OR_FMT_MXFP4) {
        for (int s = 0; s < ncols / 32; s++)
            out[n++] = mxfp4_isum(row + (size_t)s * MXFP4_BYTES, xq[s >> 3].qs + (s & 7) * 32);
    } else if (fmt == OR_FMT_Q80) {
        for (int s = 0; s < ncols / 32; s++) {
            const uint8_t *bl = row + (size_t)s * Q80_BYTES;
            const int8_t *xqs = xq[s >> 3].qs + (s & 7) * 32;
            int32_t acc = 0;
            for (int i = 0; i < 32; i++) acc += (int32_t)(int8_t)bl[2 + i] * (int32_t)xqs[i];
            out[n++] = acc;
        }
    } else {
        die("isums: format has no integer sums");
    }
    return n;
}

/* dot_fmt / dot_fmt_x4 (csrc/libtinygiant.c:611-631) */
static float dot_fmt(int fmt, const uint8_t *row, const or_q8_block *xq, const float *xf, int ncols) {
    switch (fmt) {
        case OR_FMT_Q4K: return or_dot_q4k_q8(row, xq, ncols / QK);
        case OR_FMT_Q6K: return or_dot_q6k_q8(row, xq, ncols / QK);
        case OR_FMT_MXFP4: return or_dot_mxfp4_q8(row, xq, ncols);
        case OR_FMT_Q80: return or_dot_q80_q8(row, xq, ncols);
        default:
            if (!xf) die("F16 weights need the f32 input (the reference dereferences NULL here)");
            return or_dot_f16((const uint16_t *)row, xf, ncols);
    }
}

static void dot_fmt_x4(int fmt, const uint8_t *row, const or_q8_block *const xq[4], int ncols, float out[4]) {
    switch (fmt) {
        case OR_FMT_Q4K: or_dot_q4k_q8_x4(row, xq, ncols / QK, out); return;
        case OR_FMT_Q6K: or_dot_q6k_q8_x4(row, xq, ncols / QK, out); return;
        case OR_FMT_MXFP4: or_dot_mxfp4_q8_x4(row, xq, ncols, out); return;
        default:
            for (int r = 0; r < 4; r++) out[r] = dot_fmt(fmt, row, xq[r], NULL, ncols);
    }
}

/* Restates tg_matmul (csrc/libtinygiant.c:908-931): q8 the input (not for
 * F16), out[r] = dot + bias[r], 64-row tasks. */
void or_matmul(int fmt, const void *mat, const float *bias, const float *input,
               float *output, int nrows, int ncols) {
    int nb = or_q8_nblocks(ncols);
    or_q8_block *xq = (or_q8_block *)malloc(sizeof(or_q8_block) * (size_t)(nb > 0 ? nb : 1));
    if (fmt != OR_FMT_F16) or_quantize_q8(input, xq, ncols);
    size_t rb = or_row_bytes(fmt, ncols);
    int ntask = (nrows + MM_ROWS - 1) / MM_ROWS;
#pragma omp parallel for schedule(dynamic) num_threads(g_threads)
    for (int t = 0; t < ntask; t++) {
        int r0 = t * MM_ROWS, r1 = r0 + MM_ROWS < nrows ? r0 + MM_ROWS : nrows;
        for (int r = r0; r < r1; r++)
            output[r] = dot_fmt(fmt, (const uint8_t *)mat + (size_t)r * rb, xq, input, ncols) +
                        (bias ? bias[r] : 0.f);
    }
    free(xq);
}

/* Restates tg_matmul_q4k_scalar (csrc/libtinygiant.c:1511-1546): the
 * reference's f32-input (unquantized) Q4_K row dot. */
void or_matmul_q4k_scalar(const uint8_t *mat, const float *input, float *output, int nrows, int ncols) {
    int bpr = ncols / QK;
    for (int r = 0; r < nrows; r++) {
        const uint8_t *q4 = mat + (size_t)r * bpr * Q4K_BYTES;
        float total = 0;
        for (int b = 0; b < bpr; b++) {
            const uint8_t *bl = q4 + b * Q4K_BYTES;
            uint16_t dr, dmr;
            memcpy(&dr, bl, 2);
            memcpy(&dmr, bl + 2, 2);
            float d = or_f16_to_f32(dr), dmin = or_f16_to_f32(dmr);
            const uint8_t *scales = bl + 4, *qs = bl + 16;
            const float *xb = input + b * QK;
            for (int g = 0; g < 4; g++) {
                uint8_t sc_lo, m_lo, sc_hi, m_hi;
                or_get_scale_min_k4(2 * g, scales, &sc_lo, &m_lo);
                or_get_scale_min_k4(2 * g + 1, scales, &sc_hi, &m_hi);
                for (int j = 0; j < 32; j++) {
                    uint8_t v = qs[g * 32 + j];
                    float vlo = d * sc_lo * (float)(v & 0xF) - dmin * m_lo;
                    float vhi = d * sc_hi * (float)(v >> 4) - dmin * m_hi;
                    total += vlo * xb[g * 64 + j] + vhi * xb[g * 64 + 32 + j];
                }
            }
        }
        output[r] = total;
    }
}

/* Restates tg_rms_norm (csrc/libtinygiant.c:680-698): four fused lane
 * accumulators of x*x, summed pairwise, then x*scale*w. */
void or_rms_norm(const float *x, const float *weight, float *out, int dim, float eps) {
    float acc[4] = {0, 0, 0, 0};
    int i = 0;
    for (; i + 3 < dim; i += 4)
        for (int l = 0; l < 4; l++) acc[l] = fmaf(x[i + l], x[i + l], acc[l]);
    float ss = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    for (; i < dim; i++) ss += x[i] * x[i];
    float scale = 1.f / sqrtf(ss / dim + eps);
    for (i = 0; i < dim; i++) out[i] = (x[i] * scale) * weight[i];
}

/* Restates apply_rope_inplace (csrc/libtinygiant.c:702-719): NeoX halves,
 * x1' = x1*c - x2*s (vmlsq: multiply, then subtract), x2' = x2*c + x1*s
 * (vfmaq: fused).  Pinned by: pos 0 with cos 1 / sin 0 is the identity, the
 * rotation of each (x1, x2) pair against complex multiplication in float64,
 * and the norm of each pair kept (tests/test_oracle_pins.py). */
static void rope_inplace(float *x, int n_heads, int head_dim, const float *cos_t, const float *sin_t, int pos) {
    int half = head_dim / 2;
    const float *c = cos_t + (size_t)pos * half, *s = sin_t + (size_t)pos * half;
    for (int h = 0; h < n_heads; h++) {
        float *xh = x + (size_t)h * head_dim;
        for (int i = 0; i < half; i++) {
            float x1 = xh[i], x2 = xh[half + i];
            float p = x2 * s[i];
            xh[i] = x1 * c[i] - p;
            xh[half + i] = fmaf(x1, s[i], x2 * c[i]);
        }
    }
}

/* Restates head_task (csrc/libtinygiant.c:862-904) for one query head:
 * scores over [start, seq_len) with the dot as four fused lane sums added
 * pairwise (vaddvq) plus a scalar tail, max seeded with the sink logit (or
 * -1e30), sum of exps seeded with exp(sink - max) (or 0), then
 * out += (e_t / sum) * v_t (fused in 4-wide steps, plain in the tail).
 * Pinned by: one position gives v exactly, identical keys give the mean of
 * V, a window of 1 attends only the newest position, a huge sink drives the
 * output to zero, and a float64 softmax attention on random inputs. */
static void head_attend(const float *q_h, const float *k_cache, const float *v_cache, float *out_h, int start,
                        int seq_len, int head_dim, float inv_sqrt, const float *sink) {
    int n = seq_len - start;
    float *sc = (float *)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    float mx = sink ? *sink : -1e30f;
    for (int t = start; t < seq_len; t++) {
        const float *kt = k_cache + (size_t)t * head_dim;
        float acc[4] = {0, 0, 0, 0};
        int d = 0;
        for (; d + 3 < head_dim; d += 4)
            for (int l = 0; l < 4; l++) acc[l] = fmaf(q_h[d + l], kt[d + l], acc[l]);
        float dot = (acc[0] + acc[1]) + (acc[2] + acc[3]);
        for (; d < head_dim; d++) dot += q_h[d] * kt[d];
        sc[t - start] = dot * inv_sqrt;
        if (sc[t - start] > mx) mx = sc[t - start];
    }
    float sum = sink ? expf(*sink - mx) : 0.f;
    for (int t = start; t < seq_len; t++) {
        sc[t - start] = expf(sc[t - start] - mx);
        sum += sc[t - start];
    }
    float inv = 1.f / sum;
    memset(out_h, 0, (size_t)head_dim * sizeof(float));
    for (int t = start; t < seq_len; t++) {
        float w = sc[t - start] * inv;
        const float *vt = v_cache + (size_t)t * head_dim;
        int d = 0;
        for (; d + 3 < head_dim; d += 4)
            for (int l = 0; l < 4; l++) out_h[d + l] = fmaf(w, vt[d + l], out_h[d + l]);
        for (; d < head_dim; d++) out_h[d] += w * vt[d];
    }
    free(sc);
}

/* Restates tg_attention_v2 (csrc/libtinygiant.c:939-983): q8 of the input,
 * Q/K/V projections (dot + bias, F16 from the f32 input), the optional QK
 * RMS norm per head (only when q_norm_w is given, k with k_norm_w), RoPE at
 * pos, the K/V rows stored at kv_len of each KV head, GQA attention of every
 * query head over [start, kv_len] with the optional sink and sliding window,
 * and the output projection through tg_matmul (q8 of the attention output).
 * The projections are or_matmul (pinned above); the rest is pinned as noted
 * on rope_inplace and head_attend. */
void or_attention_v2(int fmt_q, int fmt_k, int fmt_v, int fmt_o, const void *wq, const void *wk, const void *wv,
                     const void *wo, const float *bq, const float *bk, const float *bv, const float *bo,
                     const float *q_norm_w, const float *k_norm_w, const float *sinks, float *kv_k, float *kv_v,
                     int kv_len, int kv_max, int window, const float *rope_cos, const float *rope_sin,
                     const float *input, float *output, int embed_dim, int n_heads, int n_kv_heads, int head_dim,
                     int pos, float eps, float *att_out) {
    int q_dim = n_heads * head_dim, kv_dim = n_kv_heads * head_dim, ratio = n_heads / n_kv_heads;
    float *q = (float *)malloc(sizeof(float) * (size_t)q_dim);
    float *k = (float *)malloc(sizeof(float) * (size_t)kv_dim);
    float *v = (float *)malloc(sizeof(float) * (size_t)kv_dim);
    float *att = (float *)malloc(sizeof(float) * (size_t)q_dim);
    or_matmul(fmt_q, wq, bq, input, q, q_dim, embed_dim);
    or_matmul(fmt_k, wk, bk, input, k, kv_dim, embed_dim);
    or_matmul(fmt_v, wv, bv, input, v, kv_dim, embed_dim);
    if (q_norm_w) {
        for (int h = 0; h < n_heads; h++)
            or_rms_norm(q + (size_t)h * head_dim, q_norm_w, q + (size_t)h * head_dim, head_dim, eps);
        for (int h = 0; h < n_kv_heads; h++)
            or_rms_norm(k + (size_t)h * head_dim, k_norm_w, k + (size_t)h * head_dim, head_dim, eps);
    }
    rope_inplace(q, n_heads, head_dim, rope_cos, rope_sin, pos);
    rope_inplace(k, n_kv_heads, head_dim, rope_cos, rope_sin, pos);
    for (int h = 0; h < n_kv_heads; h++) {
        memcpy(kv_k + ((size_t)h * kv_max + kv_len) * head_dim, k + (size_t)h * head_dim, sizeof(float) * head_dim);
        memcpy(kv_v + ((size_t)h * kv_max + kv_len) * head_dim, v + (size_t)h * head_dim, sizeof(float) * head_dim);
    }
    int seq_len = kv_len + 1;
    int start = (window > 0 && seq_len > window) ? seq_len - window : 0;
    float inv_sqrt = 1.f / sqrtf((float)head_dim);
    for (int h = 0; h < n_heads; h++) {
        int kh = h / ratio;
        head_attend(q + (size_t)h * head_dim, kv_k + (size_t)kh * kv_max * head_dim,
                    kv_v + (size_t)kh * kv_max * head_dim, att + (size_t)h * head_dim, start, seq_len, head_dim,
                    inv_sqrt, sinks ? &sinks[h] : NULL);
    }
    if (att_out) memcpy(att_out, att, sizeof(float) * (size_t)q_dim);
    or_matmul(fmt_o, wo, bo, att, output, embed_dim, q_dim);
    free(q);
    free(k);
    free(v);
    free(att);
}

/* act_fn (csrc/libtinygiant.c:1250-1257) */
static float act_fn(int act, float g, float u) {
    if (act == OR_ACT_GPTOSS) {
        if (g > 7.f) g = 7.f;
        if (u > 7.f) u = 7.f;
        else if (u < -7.f) u = -7.f;
        return g / (1.f + expf(-1.702f * g)) * (u + 1.f);
    }
    return g / (1.f + expf(-g)) * u;
}

/* Restates tg_moe_forward_rows_v2 (csrc/libtinygiant.c:1386-1437) with
 * moe_phase_a (:1279-1327) and moe_phase_b (:1329-1384):
 *  - every input row is quantized once;
 *  - each expert gathers the rows whose weight is not exactly 0;
 *  - phase A: gate/up dots (+bias) -> act -> hidden, rows in groups of 4
 *    (x1 kernels when a group holds one row);
 *  - phase B: hidden rows re-quantized, down dot, part = w*(dot + bias);
 *  - output[row] += part, experts in index order (accumulates into output).
 * Pinned by: per-row composition of or_expert_forward_mixed (reference
 * Test 7), float64 dequantized reference for MXFP4+GPTOSS+biases (Test 10),
 * integer special cases end to end (tests). */
void or_moe_forward_rows_v2(const uint8_t *const *gate_ptrs, const uint8_t *const *up_ptrs,
                            const void *const *down_ptrs, int gate_fmt, const int *down_fmts,
                            const float *const *gate_bias, const float *const *up_bias,
                            const float *const *down_bias, int act, int n_experts,
                            const float *row_weights, const float *inputs, float *output,
                            int k, int D, int I) {
    or_moe_forward_rows_v2_ex(gate_ptrs, up_ptrs, down_ptrs, gate_fmt, down_fmts, gate_bias, up_bias,
                              down_bias, act, n_experts, row_weights, inputs, output, k, D, I, NULL, NULL);
}

/* Stage hooks for stage-wise parity: hidden_out receives phase A's hidden
 * rows and hidden_in replaces them before phase B, both [pairs][I] with the
 * pairs numbered expert-major in gather order. */
void or_moe_forward_rows_v2_ex(const uint8_t *const *gate_ptrs, const uint8_t *const *up_ptrs,
                               const void *const *down_ptrs, int gate_fmt, const int *down_fmts,
                               const float *const *gate_bias, const float *const *up_bias,
                               const float *const *down_bias, int act, int n_experts,
                               const float *row_weights, const float *inputs, float *output,
                               int k, int D, int I, const float *hidden_in, float *hidden_out) {
    if (gate_fmt == OR_FMT_F16) die("F16 gate/up weights are not supported (reference dereferences NULL)");
    int gbpr = or_q8_nblocks(D), dbpr = or_q8_nblocks(I);
    int *n_rows = (int *)calloc((size_t)n_experts, sizeof(int));
    int *rows = (int *)malloc(sizeof(int) * (size_t)n_experts * k);
    float *wts = (float *)malloc(sizeof(float) * (size_t)n_experts * k);
    or_q8_block *xq_rows = (or_q8_block *)malloc(sizeof(or_q8_block) * (size_t)k * gbpr);
    float *hidden = (float *)malloc(sizeof(float) * (size_t)n_experts * k * I);
    float *parts = (float *)calloc((size_t)n_experts * k * D, sizeof(float));
    for (int r = 0; r < k; r++) or_quantize_q8(inputs + (size_t)r * D, xq_rows + (size_t)r * gbpr, D);
    for (int e = 0; e < n_experts; e++) {
        int n = 0;
        for (int r = 0; r < k; r++) {
            float w = row_weights[(size_t)e * k + r];
            if (w == 0.f) continue;
            rows[e * k + n] = r;
            wts[e * k + n] = w;
            n++;
        }
        n_rows[e] = n;
    }
    size_t grow = or_row_bytes(gate_fmt, D);
    int nci = (I + MOE_I_ROWS - 1) / MOE_I_ROWS, ncd = (D + MOE_D_ROWS - 1) / MOE_D_ROWS;

#pragma omp parallel for schedule(dynamic) num_threads(g_threads)
    for (int task = 0; task < n_experts * nci; task++) {
        int e = task / nci, ch = task % nci, n = n_rows[e];
        if (n == 0) continue;
        int r0 = ch * MOE_I_ROWS, r1 = r0 + MOE_I_ROWS < I ? r0 + MOE_I_ROWS : I;
        const float *gb = gate_bias ? gate_bias[e] : NULL, *ub = up_bias ? up_bias[e] : NULL;
        float *hid = hidden + (size_t)e * k * I;
        for (int b = 0; b < n; b += 4) {
            int m = n - b < 4 ? n - b : 4;
            if (m == 1) {
                const or_q8_block *x = xq_rows + (size_t)rows[e * k + b] * gbpr;
                for (int r = r0; r < r1; r++) {
                    float gv = dot_fmt(gate_fmt, gate_ptrs[e] + (size_t)r * grow, x, NULL, D);
                    float uv = dot_fmt(gate_fmt, up_ptrs[e] + (size_t)r * grow, x, NULL, D);
                    if (gb) { gv += gb[r]; uv += ub[r]; }
                    hid[(size_t)b * I + r] = act_fn(act, gv, uv);
                }
                continue;
            }
            const or_q8_block *px[4];
            for (int j = 0; j < 4; j++) px[j] = xq_rows + (size_t)rows[e * k + b + (j < m ? j : m - 1)] * gbpr;
            for (int r = r0; r < r1; r++) {
                float g4[4], u4[4];
                dot_fmt_x4(gate_fmt, gate_ptrs[e] + (size_t)r * grow, px, D, g4);
                dot_fmt_x4(gate_fmt, up_ptrs[e] + (size_t)r * grow, px, D, u4);
                for (int j = 0; j < m; j++) {
                    float gv = g4[j], uv = u4[j];
                    if (gb) { gv += gb[r]; uv += ub[r]; }
                    hid[(size_t)(b + j) * I + r] = act_fn(act, gv, uv);
                }
            }
        }
    }

    if (hidden_out || hidden_in) {
        size_t p = 0;
        for (int e = 0; e < n_experts; e++)
            for (int j = 0; j < n_rows[e]; j++, p++) {
                float *h = hidden + ((size_t)e * k + j) * I;
                if (hidden_out) memcpy(hidden_out + p * I, h, sizeof(float) * (size_t)I);
                if (hidden_in) memcpy(h, hidden_in + p * I, sizeof(float) * (size_t)I);
            }
    }

#pragma omp parallel for schedule(dynamic) num_threads(g_threads)
    for (int task = 0; task < n_experts * ncd; task++) {
        int e = task / ncd, ch = task % ncd, n = n_rows[e];
        if (n == 0) continue;
        int r0 = ch * MOE_D_ROWS, r1 = r0 + MOE_D_ROWS < D ? r0 + MOE_D_ROWS : D;
        const float *hid = hidden + (size_t)e * k * I;
        float *part = parts + (size_t)e * k * D;
        const float *wt = wts + (size_t)e * k;
        const float *db = down_bias ? down_bias[e] : NULL;
        int fmt = down_fmts[e];
        if (fmt == OR_FMT_F16) {
            const uint16_t *w = (const uint16_t *)down_ptrs[e];
            for (int j = 0; j < n; j++)
                for (int r = r0; r < r1; r++) {
                    float v = or_dot_f16(w + (size_t)r * I, hid + (size_t)j * I, I);
                    part[(size_t)j * D + r] = wt[j] * (v + (db ? db[r] : 0.f));
                }
            continue;
        }
        size_t rb = or_row_bytes(fmt, I);
        or_q8_block *xq = (or_q8_block *)malloc(sizeof(or_q8_block) * (size_t)n * dbpr);
        for (int j = 0; j < n; j++) or_quantize_q8(hid + (size_t)j * I, xq + (size_t)j * dbpr, I);
        for (int b = 0; b < n; b += 4) {
            int m = n - b < 4 ? n - b : 4;
            if (m == 1) {
                for (int r = r0; r < r1; r++) {
                    float v = dot_fmt(fmt, (const uint8_t *)down_ptrs[e] + (size_t)r * rb, xq + (size_t)b * dbpr, NULL, I);
                    part[(size_t)b * D + r] = wt[b] * (v + (db ? db[r] : 0.f));
                }
                continue;
            }
            const or_q8_block *px[4];
            for (int j = 0; j < 4; j++) px[j] = xq + (size_t)(b + (j < m ? j : m - 1)) * dbpr;
            for (int r = r0; r < r1; r++) {
                float o[4];
                dot_fmt_x4(fmt, (const uint8_t *)down_ptrs[e] + (size_t)r * rb, px, I, o);
                float bias = db ? db[r] : 0.f;
                for (int j = 0; j < m; j++) part[(size_t)(b + j) * D + r] = wt[b + j] * (o[j] + bias);
            }
        }
        free(xq);
    }

    for (int e = 0; e < n_experts; e++)
        for (int j = 0; j < n_rows[e]; j++) {
            float *o = output + (size_t)rows[e * k + j] * D;
            const float *p = parts + ((size_t)e * k + j) * D;
            for (int i = 0; i < D; i++) o[i] += p[i];
        }
    free(n_rows); free(rows); free(wts); free(xq_rows); free(hidden); free(parts);
}

/* Restates tg_expert_forward (csrc/libtinygiant.c:1040-1080): one all-Q4_K
 * expert stored as [gate | up | down]; output += weight * down(silu(g)*u). */
void or_expert_forward(const uint8_t *q4_data, const float *input, float *output,
                       float weight, int D, int I) {
    size_t gate_bytes = (size_t)I * (D / QK) * Q4K_BYTES;
    const void *down = q4_data + 2 * gate_bytes;
    or_expert_forward_mixed(q4_data, q4_data + gate_bytes, down, OR_FMT_Q4K, input, output, weight, D, I);
}

/* Restates tg_expert_forward_mixed (csrc/libtinygiant.c:1084-1128): down
 * format 1 = f16 (unquantized hidden), 2 = q6_K, anything else = q4_K. */
void or_expert_forward_mixed(const uint8_t *gate, const uint8_t *up, const void *down,
                             int down_format, const float *input, float *output,
                             float weight, int D, int I) {
    int gb = D / QK, db = I / QK;
    or_q8_block *xe = (or_q8_block *)malloc(sizeof(or_q8_block) * (size_t)gb);
    or_q8_block *xi = (or_q8_block *)malloc(sizeof(or_q8_block) * (size_t)(db > 0 ? db : 1));
    float *g = (float *)malloc(sizeof(float) * (size_t)I), *u = (float *)malloc(sizeof(float) * (size_t)I);
    float *h = (float *)malloc(sizeof(float) * (size_t)I), *dn = (float *)malloc(sizeof(float) * (size_t)D);
    or_quantize_q8(input, xe, D);
    for (int r = 0; r < I; r++) g[r] = or_dot_q4k_q8(gate + (size_t)r * gb * Q4K_BYTES, xe, gb);
    for (int r = 0; r < I; r++) u[r] = or_dot_q4k_q8(up + (size_t)r * gb * Q4K_BYTES, xe, gb);
    for (int i = 0; i < I; i++) {
        float silu = g[i] / (1.f + expf(-g[i]));
        h[i] = silu * u[i];
    }
    if (down_format == OR_FMT_F16) {
        for (int r = 0; r < D; r++) dn[r] = or_dot_f16((const uint16_t *)down + (size_t)r * I, h, I);
    } else {
        or_quantize_q8(h, xi, I);
        for (int r = 0; r < D; r++)
            dn[r] = down_format == OR_FMT_Q6K
                        ? or_dot_q6k_q8((const uint8_t *)down + (size_t)r * db * Q6K_BYTES, xi, db)
                        : or_dot_q4k_q8((const uint8_t *)down + (size_t)r * db * Q4K_BYTES, xi, db);
    }
    for (int i = 0; i < D; i++) output[i] += weight * dn[i];
    free(xe); free(xi); free(g); free(u); free(h); free(dn);
}
