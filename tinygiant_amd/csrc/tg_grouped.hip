/*
 * tg_grouped.hip -- MXFP4 expert phases on block-scaled MFMA with the weights
 * staged in LDS: moe_phase_a / moe_phase_b of csrc/libtinygiant.c:1279-1384
 * with the per-block dot of dot_mxfp4_q8 (:533-547), for any number of pairs
 * per expert (a verify batch, a prefill).
 *
 * Arithmetic.  An MXFP4 block holds 32 e2m1 codes under one e8m0 exponent e.
 * The reference's term for a block is  d_x * half(e) * sum_i kv[c_i] * x_i
 * with kv[c] = 2 * e2m1(c), half(e) = 2^(e-128) and x_i the q8 integers.
 * v_mfma_scale_f32_16x16x128_f8f6f4 multiplies e2m1 A operands under e8m0
 * scales 2^(e-127) by fp8 B operands, so with A = the raw codes and scale e
 * each product is exactly kv[c] * half(e) * b.  A q8 integer x in [-127, 127]
 * is 16 * hi + lo with hi = x >> 4 in [-8, 7] and lo = x & 15, both exact in
 * fp8 e4m3; the hi half runs with B scale 2^4.  The block sums are exact;
 * only the f32 additions of four blocks inside the MFMA and of the q8 scale
 * groups differ in order from the reference's block-by-block sum.
 *
 * Operand layout (measured on gfx950): A lane l = weight row l % 16 and
 * K = 32 (l / 16) + j for nibble j of its four dwords (low nibble first), so
 * the 16 code bytes of a block are the lane's A operand as they lie in memory
 * (K = 2t: value t, K = 2t + 1: value 16 + t); the lane's A scale is the
 * e8m0 of (row l % 16, K block l / 16).  B lane l = pair l % 16, bytes 0..15
 * at K = 16 (l / 16) + j, bytes 16..31 at K = 64 + 16 (l / 16) + j - 16.
 * D lane l, register v = weight row 4 (l / 16) + v, pair l % 16.
 *
 * Work item = 16 weight rows of one expert (a "slab": 16 consecutive rows are
 * one contiguous, 16-byte aligned byte range).  Persistent workgroups walk
 * cost-balanced runs of items; each holds the next item's slabs in registers
 * (coalesced 16-byte loads, in flight while the current item computes) and
 * stores them to LDS; its NWAVE waves split the blocks of a row into ranges
 * and run the expert's pairs against the resident slab, 16 per pass; 256
 * threads then add the waves' partial sums in wave order and write one
 * result each.
 * HBM sees each weight byte once however many pairs the expert holds; the
 * fp8 halves of a pass stay in registers from one item to the next of the
 * same expert.
 */
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <algorithm>

#include "tg_device.hpp"
#include "tg_kernels.h"
#include "tg_xchg.hpp"

namespace tg {

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int MXB = 17;                 /* bytes per MXFP4 block */
constexpr int GB = 4;                   /* blocks per MFMA (K = 128) */
constexpr int NWAVE = 8;                /* waves per workgroup, each one range of blocks */
constexpr int NT = 64 * NWAVE;
constexpr int CHUNKS = 4;               /* 16-byte slab chunks per thread and matrix */
constexpr uint32_t MAX_SLAB = CHUNKS * NT * 16;
constexpr int XB = 12;                  /* blocks of q8 operands per batch */
constexpr int NG = XB / GB;
constexpr uint32_t OOB = 0x80000000u;   /* past every buffer: the load reads zero */
constexpr int FMT_FP8 = 0, FMT_FP4 = 4; /* MFMA operand formats */
constexpr int NPRE = 4;                 /* passes whose pair rows and weights are fetched with the expert */
constexpr int SCALE_1 = 127, SCALE_16 = 131;

/* Slab bytes are read once per call: nontemporal loads (measured 3-6%
 * faster on a 64-token gpt-oss prefill than regular ones; the Q4_K / Q6_K
 * phases, whose lanes share 16-byte pieces of a line, lose with them). */
constexpr int CPOL_NT = 2;
__device__ inline u32x4 ld16_nt(Buf b, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(b.r, (int)off, 0, CPOL_NT);
}

/* Read-only tables through explicit address spaces: wave-uniform reads of
 * the constant space become scalar loads (counted apart from the vector
 * loads), per-lane reads of the global space in-order vector loads. */
template <class T>
__device__ inline T ldc(const T *p, size_t i) {
    return ((const __attribute__((address_space(4))) T *)(uintptr_t)p)[i];
}
template <class T>
__device__ inline T ldg(const T *p, size_t i) {
    return ((const __attribute__((address_space(1))) T *)(uintptr_t)p)[i];
}

/* fp8 e4m3 code of an integer in [-15, 15] (exact) */
__device__ inline uint32_t e4m3_int(int n) {
    if (n == 0) return 0;
    const uint32_t m = (uint32_t)(n < 0 ? -n : n);
    const uint32_t e = 31u - (uint32_t)__builtin_clz(m);   /* 0..3 */
    return (n < 0 ? 0x80u : 0u) | ((e + 7u) << 3) | ((m << (3u - e)) & 7u);
}

}  // namespace

/* dst[r][b][part][32]: for q8 row r and block b of 32 values, the fp8 codes of
 * hi = x >> 4 (part 0) and lo = x & 15 (part 1) in MFMA K order (position 2t
 * holds value t, 2t + 1 value 16 + t).  One thread per 4 output bytes. */
__global__ __launch_bounds__(256) void k_mx_split(Q8Rows q, int nrows, int nblk, uint8_t *dst) {
    const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;   /* 4-byte group */
    const size_t per_row = (size_t)nblk * 16;
    if (i >= (size_t)nrows * per_row) return;
    const int r = (int)(i / per_row), rem = (int)(i % per_row);
    const int b = rem / 16, part = (rem / 8) & 1, p0 = (rem % 8) * 4;
    const int8_t *x = q.qs + (size_t)r * q.nb * 256 + (size_t)b * 32;
    uint32_t w = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int p = p0 + j;
        const int v = x[(p & 1) ? 16 + (p >> 1) : (p >> 1)];
        const int half = part == 0 ? (v >> 4) : (v & 15);
        w |= e4m3_int(half) << (8 * j);
    }
    *(uint32_t *)(dst + (size_t)r * nblk * 64 + (size_t)b * 64 + part * 32 + p0) = w;
}

/* The e8m0 scale byte 255 means 2^127 to the reference (e8m0_to_fp32_half,
 * csrc/libtinygiant.c:516-519) and NaN to the block-scaled MFMA (OCP MX), and
 * 2^127 times the products overflows the MFMA's f32 sums where the
 * reference's integer block sum times its scales may stay finite: a layer
 * with such a block takes the v_dot4 phases.  One thread per block. */
__global__ __launch_bounds__(256) void k_mx_scan_e255(const uint8_t *__restrict__ p, uint64_t nblocks,
                                                      unsigned *flag) {
    const uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x;
    const bool hit = i < nblocks && p[i * MXB] == 255;
    if (__ballot(hit) && (threadIdx.x & 63) == __builtin_ctzll(__ballot(hit))) atomicOr(flag, 1u);
}

void launch_mx_scan_e255(const uint8_t *p, uint64_t nbytes, unsigned *flag_dev, hipStream_t st) {
    const uint64_t nb = nbytes / MXB;
    if (nb == 0) return;
    hipLaunchKernelGGL(k_mx_scan_e255, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, st, p, nb, flag_dev);
}

void launch_mx_split(const Q8Rows &q, int nrows, int ncols, uint8_t *dst, hipStream_t st) {
    const size_t n = (size_t)nrows * (ncols / 32) * 16;
    if (n == 0) return;
    hipLaunchKernelGGL(k_mx_split, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, q, nrows, ncols / 32, dst);
}

namespace {

/* fp8 halves of one batch of XB blocks of a wave's range (NG groups of GB
 * blocks), MT tiles of pairs, plus the q8 scale of each group */
template <int MT>
struct XBatch {
    v8i hi[MT][NG], lo[MT][NG];
    float d[MT][NG];
};

struct XSrc {
    Buf sp;           /* fp8 halves, [rows][nblk][2][32] */
    Buf d;            /* q8 scales */
    int nblk, nb8;
};

template <int MT>
__device__ inline void load_batch(XBatch<MT> &s, const XSrc &o, int b0, int b1, int nt, const int *xrow, int g) {
#pragma unroll
    for (int t = 0; t < MT; t++) {
        if (t > 0 && t >= nt) break;
        const bool ok = xrow[t] >= 0;
        const uint32_t row = (uint32_t)(ok ? xrow[t] : 0);
        const uint32_t rbase = row * (uint32_t)o.nblk * 64u + 16u * (g & 1);
#pragma unroll
        for (int q = 0; q < NG; q++) {
            const int ba = b0 + GB * q + (g >> 1), bb = ba + 2;   /* blocks of bytes 0..15 and 16..31 */
            const uint32_t oa = ok && ba < b1 ? rbase + (uint32_t)ba * 64u : OOB;
            const uint32_t ob = ok && bb < b1 ? rbase + (uint32_t)bb * 64u : OOB;
            const uint32_t oa2 = oa == OOB ? OOB : oa + 32u, ob2 = ob == OOB ? OOB : ob + 32u;
            const int bq = b0 + GB * q;
            const uint32_t od = ok && bq < b1 ? (row * o.nb8 + (uint32_t)(bq >> 3)) * 4u : OOB;
            const u32x4 h0 = ld16(o.sp, oa), h1 = ld16(o.sp, ob), l0 = ld16(o.sp, oa2), l1 = ld16(o.sp, ob2);
            const uint32_t dv = ld4(o.d, od);
            s.hi[t][q] = v8i{(int)h0.x, (int)h0.y, (int)h0.z, (int)h0.w, (int)h1.x, (int)h1.y, (int)h1.z, (int)h1.w};
            s.lo[t][q] = v8i{(int)l0.x, (int)l0.y, (int)l0.z, (int)l0.w, (int)l1.x, (int)l1.y, (int)l1.z, (int)l1.w};
            s.d[t][q] = __uint_as_float(dv);
        }
    }
}

/* One batch of NG groups starting at block b0: every LDS read of the batch
 * first (the lane's block codes and e byte of each group and matrix), then
 * per group and matrix two chained MFMAs per tile.  A block past b1 reads
 * the last block's codes against B operands and a q8 scale of zero. */
template <int NM, int MT>
__device__ inline void mma_batch(const uint32_t *lds, uint32_t sstride, uint32_t rb, const XBatch<MT> &s, int b0,
                                 int b1, int nt, int lane, float (&acc)[NM][MT][4]) {
    const int g = lane >> 4, c16 = lane & 15;
    uint32_t w[NG][NM][5], sft[NG][NM];
#pragma unroll
    for (int q = 0; q < NG; q++) {
        const int b = min(b0 + GB * q + g, b1 - 1);
#pragma unroll
        for (int m = 0; m < NM; m++) {
            const uint32_t pos = m * sstride + (uint32_t)c16 * rb + (uint32_t)b * MXB;   /* the block's e byte */
            const uint32_t *dw = lds + (pos >> 2);
#pragma unroll
            for (int i = 0; i < 5; i++) w[q][m][i] = dw[i];
            sft[q][m] = pos & 3u;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < NG; q++)
#pragma unroll
        for (int m = 0; m < NM; m++) {
            const uint32_t s8 = 8u * (sft[q][m] + 1u);   /* codes start one byte after e: 8 .. 32 bits */
            const uint32_t *ww = w[q][m];
            v8i av;
            av[0] = (int)(uint32_t)((((uint64_t)ww[1] << 32) | ww[0]) >> s8);
            av[1] = (int)(uint32_t)((((uint64_t)ww[2] << 32) | ww[1]) >> s8);
            av[2] = (int)(uint32_t)((((uint64_t)ww[3] << 32) | ww[2]) >> s8);
            av[3] = (int)(uint32_t)((((uint64_t)ww[4] << 32) | ww[3]) >> s8);
            av[4] = av[5] = av[6] = av[7] = 0;
            const int e = (int)((ww[0] >> (8u * sft[q][m])) & 0xFFu);
#pragma unroll
            for (int t = 0; t < MT; t++) {
                if (t > 0 && t >= nt) break;   /* uniform; tile 0 always holds a pair */
                const v4f z = {0.f, 0.f, 0.f, 0.f};
                v4f r = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, s.hi[t][q], z, FMT_FP4, FMT_FP8, 0, e,
                                                                        0, SCALE_16);
                r = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, s.lo[t][q], r, FMT_FP4, FMT_FP8, 0, e, 0,
                                                                    SCALE_1);
                const float d = s.d[t][q];
                acc[m][t][0] += d * r[0];
                acc[m][t][1] += d * r[1];
                acc[m][t][2] += d * r[2];
                acc[m][t][3] += d * r[3];
            }
        }
}

/* 16-byte staging chunks per thread and matrix for rows of rb bytes */
__host__ __device__ inline int mx_chunks(uint32_t rb) { return 16u * rb <= 3u * NT * 16 ? 3 : CHUNKS; }

/* LDS bytes of one matrix's slab: 16 rows, 16 bytes of slack for the last
 * lane's five-dword read, and room for every staging chunk (the stores are
 * unconditional; chunks past the slab hold zeros) */
__host__ __device__ inline uint32_t mx_slab_stride(uint32_t rb) {
    const uint32_t need = 16u * rb + 16u, chunks = (uint32_t)mx_chunks(rb) * NT * 16;
    return ((need > chunks ? need : chunks) + 15u) & ~15u;
}

size_t mx_lds_bytes(int nm, int mt, int cols) {
    const int nblk = cols / 32;
    return (size_t)nm * mx_slab_stride((uint32_t)nblk * MXB)   /* slabs */
           + (size_t)NWAVE * nm * mt * 4 * 64 * 4;             /* partial sums of every wave */
}

}  // namespace

/* DOWN = false, phase A (gate/up, NM = 2):
 *   hidden[p][r] = act(gate_r . xq_p + bg[r], up_r . xq_p + bu[r])
 * DOWN = true, phase B (NM = 1), experts whose down matrix is MXFP4:
 *   part[p][r] = w_p * (down_r . hq_p + bd[r])
 * Persistent: workgroup i takes a contiguous run of items of about equal
 * cost (slab load plus passes of 16 pairs); an item is (active expert,
 * 16-row slab).  NT threads; dynamic LDS = mx_lds_bytes; CH 16-byte chunks
 * per thread and matrix hold a slab (16 * CH * NT bytes at most). */
template <int NM, int MT, int CH, bool DOWN>
__global__ __launch_bounds__(NT) void k_moe_mx(MoeArgs a) {
    static_assert(MT == 1, "the epilogue maps one tile of 16 pairs onto 256 threads");
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    const int rows = DOWN ? a.D : a.I, cols = DOWN ? a.I : a.D;
    const int nblk = cols / 32;
    const uint32_t rb = (uint32_t)nblk * MXB;
    const uint32_t slab = 16u * rb, sstride = mx_slab_stride(rb);
    const int nslab = (rows + 15) / 16;
    const int *act = DOWN ? a.mx_act + a.n_act_a : a.mx_act;
    const int nact = DOWN ? a.n_act_b : a.n_act_a;
    const int nitems = nact * nslab;
    float *red = (float *)((uint8_t *)lds + NM * sstride);   /* [NWAVE][NM][4][64] */
    /* w is wave-uniform (readfirstlane), so every condition below that
     * decides which loads a wave issues is a scalar branch */
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, g = lane >> 4,
              c16 = lane & 15;
    const uint32_t mbytes = (uint32_t)rows * rb;              /* rows past the end read zero */
    /* epilogue thread (tid < 256): register ev of D lane el, i.e. weight row
     * 4 (el / 16) + ev of the slab and pair el % 16 of the tile */
    const int ev = tid >> 6, el = tid & 63;

    /* this wave's block range, a multiple of GB blocks long */
    const int cw = (((nblk + NWAVE - 1) / NWAVE) + GB - 1) / GB * GB;
    const int b0w = min(nblk, w * cw), b1w = min(nblk, b0w + cw);
    XSrc xs;
    const Q8Rows &q = DOWN ? a.hq : a.xq;
    const int qrows = DOWN ? a.P : a.k;
    xs.nblk = nblk;
    xs.nb8 = q.nb;
    xs.sp = make_buf(DOWN ? a.hp : a.xp, (uint32_t)((size_t)qrows * nblk * 64));
    xs.d = make_buf(q.d, (uint32_t)((size_t)qrows * q.nb * 4));

    /* the expert of the item being issued, and its matrices */
    int iss_ai = -1;
    Buf iss_w[NM];
    u32x4 vA[NM][CH], vB[NM][CH];   /* slabs of two items ahead, alternating */
    auto set_issuer = [&](int ai) {
        iss_ai = ai;
        const int e = ldc(act, ai);
#pragma unroll
        for (int m = 0; m < NM; m++) {
            const uint64_t base = DOWN ? ldc(a.down, e) : (m ? ldc(a.up, e) : ldc(a.gate, e));
            iss_w[m] = make_buf((const void *)(uintptr_t)base, mbytes);
        }
    };
    XBatch<MT> xb;
    int xrow[MT];
    /* this workgroup's run of items: an equal share of the total cost */
    const int *cum = DOWN ? a.mx_cum + a.n_act_a + 1 : a.mx_cum;
    auto item_at = [&](long c) {
        int lo = 0, hi = nact;   /* largest i with cum[i] <= c */
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (ldc(cum, mid) <= c) lo = mid;
            else hi = mid;
        }
        const int per = (ldc(cum, lo + 1) - ldc(cum, lo)) / nslab;
        return min(nitems, lo * nslab + (int)((c - ldc(cum, lo) + per - 1) / per));
    };
    const long total = nact ? ldc(cum, nact) : 0;
    int it = nact ? item_at(total * blockIdx.x / gridDim.x) : 0;
    const int it_end = blockIdx.x + 1 == gridDim.x ? nitems : (nact ? item_at(total * (blockIdx.x + 1) / gridDim.x) : 0);
    if (it >= it_end) return;   /* uniform */

    /* an item's slabs; an item past the run reads zeros (no memory access),
     * so every item issues the same loads */
    auto issue = [&](u32x4 (&v)[NM][CH], int item) {
        const bool ok = item < it_end;
        if (ok && item / nslab != iss_ai) set_issuer(item / nslab);
        const uint32_t off = (uint32_t)(item % nslab) * 16u * rb;
#pragma unroll
        for (int m = 0; m < NM; m++) {
#pragma unroll
            for (int c = 0; c < CH; c++) {
                const uint32_t i = (uint32_t)(tid + NT * c) * 16u;
                v[m][c] = ld16_nt(iss_w[m], ok && i < slab ? off + i : OOB);
            }
        }
    };

    /* per-expert state: the expert's pairs, biases (empty buffers read
     * zero) and the input rows of its first 16 pairs */
    struct Expert {
        int ai, p0, ne;
        bool has0, has1;
        Buf bias[2];
    };
    const Buf prow_buf = make_buf(a.p_row, (uint32_t)a.P * 4u), pw_buf = make_buf(a.p_w, (uint32_t)a.P * 4u);
    auto expert = [&](int ai) {
        Expert x;
        x.ai = ai;
        const int e = ldc(act, ai);
        x.p0 = ldc(a.p_off, e);
        x.ne = ldc(a.p_off, e + 1) - x.p0;
        const float *b0p = DOWN ? (a.dbias ? (const float *)(uintptr_t)ldc(a.dbias, e) : nullptr)
                                : (a.gbias ? (const float *)(uintptr_t)ldc(a.gbias, e) : nullptr);
        const float *b1p = DOWN ? nullptr : (a.ubias ? (const float *)(uintptr_t)ldc(a.ubias, e) : nullptr);
        x.has0 = b0p != nullptr;
        x.has1 = b1p != nullptr;
        x.bias[0] = make_buf(b0p, b0p ? (uint32_t)rows * 4u : 0u);
        x.bias[1] = make_buf(b1p, b1p ? (uint32_t)rows * 4u : 0u);
        return x;
    };
    /* input row of pair j of an expert (phase A: its q8 row, phase B: the
     * pair itself), unmasked (zero past the expert's pairs) and with -1
     * there; the pair's router weight */
    auto pair_row_raw = [&](const Expert &x, int j) -> int {
        if (DOWN) return x.p0 + j;
        return (int)ld4(prow_buf, j < x.ne ? (uint32_t)(x.p0 + j) * 4u : OOB);
    };
    auto pair_row = [&](const Expert &x, int j) -> int {
        const int r = pair_row_raw(x, j);
        return j < x.ne ? r : -1;
    };
    auto pair_w = [&](const Expert &x, int j) -> float {
        return __uint_as_float(ld4(pw_buf, j < x.ne ? (uint32_t)(x.p0 + j) * 4u : OOB));
    };
    /* epilogue thread (tid < 256) row of an item's slab */
    auto ep_row = [&](int item) { return (item % nslab) * 16 + 4 * (el >> 4) + ev; };

    /* pair rows (unmasked: the mask is applied where a pass takes them, so
     * the load is not waited for at once) and (phase B) weights of an
     * expert's first NPRE passes */
    int xrows[NPRE], nxrows[NPRE];
    float wts[NPRE], nwts[NPRE];
    auto fetch_pairs = [&](const Expert &x, int (&rr)[NPRE], float (&ww)[NPRE]) {
#pragma unroll
        for (int k = 0; k < NPRE; k++) {
            rr[k] = pair_row_raw(x, 16 * k + c16);
            ww[k] = DOWN ? pair_w(x, 16 * k + (el & 15)) : 0.f;
        }
    };

    /* first item: its slabs, q8 operands, biases and pair weights, then the
     * second item's slabs */
    Expert cur = expert(it / nslab), nxt = cur;
    fetch_pairs(cur, xrows, wts);
    wait_copies();   /* a wait the compiler sees: the pair loads are not pending in the item loop */
    xrow[0] = c16 < cur.ne ? xrows[0] : -1;
    issue(vA, it);
    load_batch<MT>(xb, xs, b0w, min(b1w, b0w + XB), 1, xrow, g);
    int er = ep_row(it);
    float bias0 = __uint_as_float(ld4(cur.bias[0], (uint32_t)er * 4u));
    float bias1 = __uint_as_float(ld4(cur.bias[1], (uint32_t)er * 4u));
    float wt = wts[0];
    __builtin_amdgcn_sched_barrier(0);
    issue(vB, it + 1);

    /* Per item, loads are issued in one fixed order: the next expert's pair
     * rows (when it changes), then after the compute the next item's q8
     * operands (unless kept) and biases, then the slabs two items ahead (past
     * the run they read zeros).  Loads complete in order, so the compiler's
     * wait for an item's slab leaves the next item's slab in flight, and
     * every slab has a whole item of lead. */
    float acc[NM][MT][4];
    /* one pass: the partial sums of every wave to LDS, then 256 threads add
     * them in wave order and write one result each */
    auto finish = [&](int t0) {
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int vv = 0; vv < 4; vv++) red[((w * NM + m) * 4 + vv) * 64 + lane] = acc[m][0][vv];
        bar_lds();
        const int j = t0 + (el & 15);
        if (tid < 256 && j < cur.ne && er < rows) {
            float r2[NM];
#pragma unroll
            for (int m = 0; m < NM; m++) {
                float sum = red[(m * 4 + ev) * 64 + el];
#pragma unroll
                for (int ww = 1; ww < NWAVE; ww++) sum += red[((ww * NM + m) * 4 + ev) * 64 + el];
                r2[m] = sum;
            }
            const int p = cur.p0 + j;
            if (DOWN) {
                a.part[(size_t)p * a.D + er] = wt * (r2[0] + (cur.has0 ? bias0 : 0.f));
            } else {
                float gv = r2[0], uv = r2[NM - 1];
                if (cur.has0) gv += bias0;
                if (cur.has1) uv += bias1;
                a.hidden[(size_t)p * a.I + er] = act_fn(a.act, gv, uv);
            }
        }
    };
    auto zero = [&]() {
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int vv = 0; vv < 4; vv++) acc[m][0][vv] = 0.f;
    };
    auto step = [&](u32x4 (&v)[NM][CH]) {
        const int nx = it + 1;
        const bool has_nx = nx < it_end;
        const bool new_ex = has_nx && nx / nslab != cur.ai;
        if (new_ex) {
            nxt = expert(nx / nslab);
            fetch_pairs(nxt, nxrows, nwts);
        }
        bar_lds();   /* the previous item is done with LDS */
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int c = 0; c < CH; c++)
                *(u32x4 *)((uint8_t *)lds + m * sstride + (uint32_t)(tid + NT * c) * 16u) = v[m][c];
        bar_lds();
        zero();
        mma_batch<NM, MT>(lds, sstride, rb, xb, b0w, min(b1w, b0w + XB), 1, lane, acc);
        for (int bb = b0w + XB; bb < b1w; bb += XB) {   /* rows wider than NWAVE * XB blocks */
            load_batch(xb, xs, bb, min(b1w, bb + XB), 1, xrow, g);
            mma_batch<NM, MT>(lds, sstride, rb, xb, bb, min(b1w, bb + XB), 1, lane, acc);
        }
        finish(0);
        /* further passes over the resident slab for an expert with more than
         * 16 pairs */
        for (int t0 = 16 * MT, k = 1; t0 < cur.ne; t0 += 16 * MT, k++) {
            bar_lds();   /* red is rewritten by this pass */
            int r = 0;
            float wk = 0.f;
#pragma unroll
            for (int q = 1; q < NPRE; q++)
                if (k == q) {
                    r = xrows[q];
                    wk = wts[q];
                }
            xrow[0] = k < NPRE ? (t0 + c16 < cur.ne ? r : -1) : pair_row(cur, t0 + c16);
            if (DOWN) wt = k < NPRE ? wk : pair_w(cur, t0 + (el & 15));
            zero();
            for (int bb = b0w; bb < b1w; bb += XB) {
                load_batch(xb, xs, bb, min(b1w, bb + XB), 1, xrow, g);
                mma_batch<NM, MT>(lds, sstride, rb, xb, bb, min(b1w, bb + XB), 1, lane, acc);
            }
            finish(t0);
            /* a wait the compiler sees: the pass's own loads (issued after
             * the next slabs, which they waited for already) are not left
             * pending where the compiler merges paths */
            wait_copies();
        }
        /* the next item's q8 operands (unless this item's first-pass ones
         * serve it: same expert, one pass, one batch), biases, pair weights */
        if (has_nx) {
            const bool keep = !new_ex && cur.ne <= 16 * MT && b1w - b0w <= XB;
            if (new_ex) {
                /* the new expert's pair loads (issued after the next slabs,
                 * so this waits for those too) */
                wait_copies();
                cur = nxt;
#pragma unroll
                for (int q = 0; q < NPRE; q++) {
                    xrows[q] = nxrows[q];
                    wts[q] = nwts[q];
                }
            }
            xrow[0] = c16 < cur.ne ? xrows[0] : -1;
            if (!keep) load_batch<MT>(xb, xs, b0w, min(b1w, b0w + XB), 1, xrow, g);
            er = ep_row(nx);
            bias0 = __uint_as_float(ld4(cur.bias[0], (uint32_t)er * 4u));
            bias1 = __uint_as_float(ld4(cur.bias[1], (uint32_t)er * 4u));
            wt = wts[0];
        }
        /* then the slabs two items ahead, into the registers just stored */
        __builtin_amdgcn_sched_barrier(0);
        issue(v, it + 2);
        it = nx;
    };
    while (it < it_end) {
        step(vA);
        if (it >= it_end) break;
        step(vB);
    }
}

/* Tiles of 16 pairs per pass.  One: an expert with more than 16 pairs runs
 * further passes over its resident slab. */
constexpr int MX_TILES = 1;

/* the device must allow the LDS to one workgroup, and the slab must fit the
 * staging registers */
bool grouped_lds_ok(int D, int I) {
    static int max_lds = -1;
    if (max_lds < 0) {
        int dev = 0;
        max_lds = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
            max_lds = 0;
    }
    return mx_lds_bytes(2, MX_TILES, D) <= (size_t)max_lds && mx_lds_bytes(1, MX_TILES, I) <= (size_t)max_lds &&
           (uint32_t)(D / 32) * MXB * 16 <= MAX_SLAB && (uint32_t)(I / 32) * MXB * 16 <= MAX_SLAB;
}

/* persistent grid: the workgroups that can be resident at once */
template <class K>
static unsigned mx_grid(K kern, size_t lds, int nitems) {
    int dev = 0, cus = 0, per = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kern, NT, lds) != hipSuccess || per < 1) per = 1;
    return (unsigned)std::max(1, std::min(std::max(cus, 1) * per, nitems));
}

template <int NM, bool DOWN>
static void launch_mx(const MoeArgs &a, int cols, int nitems, hipStream_t st) {
    if (nitems == 0) return;
    const size_t lds = mx_lds_bytes(NM, MX_TILES, cols);
    if (mx_chunks((uint32_t)(cols / 32) * MXB) == 3) {
        auto k = k_moe_mx<NM, MX_TILES, 3, DOWN>;
        hipLaunchKernelGGL(k, dim3(mx_grid(k, lds, nitems)), dim3(NT), lds, st, a);
    } else {
        auto k = k_moe_mx<NM, MX_TILES, CHUNKS, DOWN>;
        hipLaunchKernelGGL(k, dim3(mx_grid(k, lds, nitems)), dim3(NT), lds, st, a);
    }
}

void launch_moe_a_mx(const MoeArgs &a, hipStream_t st) {
    launch_mx<2, false>(a, a.D, a.n_act_a * ((a.I + 15) / 16), st);
}

void launch_moe_b_mx(const MoeArgs &a, hipStream_t st) {
    launch_mx<1, true>(a, a.I, a.n_act_b * ((a.D + 15) / 16), st);
}

}  // namespace tg
