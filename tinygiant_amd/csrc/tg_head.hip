/*
 * tg_head.hip -- output head over a batch of rows with the argmax fused in.
 *
 * The reference runs, per row r of a verify batch, tg_rms_norm then
 * tg_matmul over the vocab x D output head (tinygiant/engine.py:347-354;
 * tg_matmul is csrc/libtinygiant.c:908-931 with dot_q6k_q8 :384-443) and
 * takes numpy.argmax of each row's logits (tinygiant/specdec.py:77,90,
 * engine.py:187).  Here the head is read once for all k rows:
 *
 *   k_head_q6k<K,L> Q6_K head with 2048 columns: every lane owns one 128-value
 *                   half-block of one vocab row, decodes its 6-bit codes once
 *                   and dots them with the k q8 rows staged in LDS; the 16
 *                   lanes of a row are summed by DPP; the next row group's
 *                   weights are loaded while the current one is computed.
 *                   A wave's group (4 rows, contiguous) is loaded as aligned
 *                   16-byte pieces, 1 KiB an instruction, and regrouped into
 *                   half-blocks through the wave's own LDS region.
 *                   Each lane ends with one input row's sum (a DPP
 *                   reduce-scatter over the 16 lanes); each workgroup keeps
 *                   the best (logit, row) per input row, commits it with one
 *                   64-bit atomic max, and the last workgroup to finish
 *                   writes the argmax.
 *   k_head_q6k_mfma the same head on int8 MFMA for 8 or more rows: 16 vocab
 *                   rows an item staged in LDS, one 256-block per wave, logits formed and
 *                   added block by block as the reference does (bit-equal
 *                   to it where its float block sums are exact).
 *   k_argmax_rows   argmax of materialized logits (any format, via k_gemv).
 *
 * Argmax keys pack an order-preserving image of the f32 logit above the
 * complement of the row index, so the maximum key is the largest logit and,
 * among equal logits, the first row -- numpy.argmax's tie rule.
 *
 * The finish is ordered by the atomics themselves, all relaxed and all on the
 * device-coherent words best[]: a workgroup's atomicMax returns (its result
 * is stored before the workgroup barrier) before thread 0 takes the ticket,
 * so every key is in best[] before the ticket that sees gridDim.x - 1, and
 * the last workgroup reads best[] with device-scope atomic loads.  Release /
 * acquire orderings on the ticket would add nothing the keys need and make
 * every workgroup write back and invalidate its L2 (buffer_wbl2 / buffer_inv):
 * measured 45.5 -> 70.4 us for the 1-row head.
 */
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "tg_common.h"
#include "tg_device.hpp"
#include "tg_head.h"
#include "tg_xchg.hpp"

namespace tg {

namespace {

constexpr int NBH = 8;          /* 256-blocks per head row (2048 columns) */
constexpr int HPR = 2 * NBH;    /* half-blocks (lanes) per row */
constexpr int RPW = 64 / HPR;   /* rows per wave */
constexpr int HRB = NBH * 210;  /* Q6_K head row bytes */
constexpr int XST = 144;        /* LDS stride of a staged 128-value half (bank spread) */
constexpr int HT = 512;         /* threads per head workgroup */
constexpr int HW = HT / 64;
constexpr int HGB = RPW * HRB;  /* a wave's row group: 6,720 contiguous bytes */
constexpr int HGP = HGB / 1024; /* its whole KiB (6), then 36 lanes of 16 bytes */
static_assert(HGB % 16 == 0 && HGB - 1024 * HGP <= 1024, "group pieces");

__device__ inline uint64_t argmax_key(float v, uint32_t row) {
    uint32_t u = v == 0.f ? 0u : __float_as_uint(v);   /* -0 ties with +0, as in numpy */
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint64_t)(0xFFFFFFFFu - row);
}
__device__ inline float key_value(uint64_t key) {
    uint32_t u = (uint32_t)(key >> 32);
    u = (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u;
    return __uint_as_float(u);
}

/* One lane's Q6_K half-block (64 B of ql, 32 B of qh, 8 sub-scales, d). */
struct HHalf {
    u32x4 la0, la1, lb0, lb1, h0, h1;
    u32x2 sc;
    uint32_t d;   /* the f16 bits */
};
/* A wave's row group as lane pieces: lane l holds bytes 16 l + 1024 j of
 * it (j < HGP), and lanes l < 36 also bytes 1024 HGP + 16 l.  Each load
 * instruction reads 1 KiB of contiguous, aligned bytes; loads of the lanes'
 * own half-blocks (16-byte pieces 105 bytes apart, half of them at 2 mod 4)
 * touched eight times as many cache lines and ran ~1.25x slower. */
struct HGroup {
    u32x4 p[HGP + 1];
};
/* Its loads, tracked by the compiler, from byte `base` of the matrix (the
 * whole offset in the VGPR: a raw buffer's range check covers that offset
 * and not the SGPR one, and loads past the matrix read zero; the lanes past
 * the group's last piece take an offset beyond any head and read nothing) */
__device__ inline HGroup load_group(Buf b, uint32_t base, int lane) {
    HGroup g;
    const int o = (int)(base + 16u * (uint32_t)lane);
#pragma unroll
    for (int j = 0; j < HGP; j++) g.p[j] = __builtin_amdgcn_raw_buffer_load_b128(b.r, o + 1024 * j, 0, 0);
    const bool tail = 16 * lane < HGB - 1024 * HGP;
    g.p[HGP] = __builtin_amdgcn_raw_buffer_load_b128(b.r, tail ? o + 1024 * HGP : (int)0x80000000u, 0, 0);
    return g;
}
/* An empty statement that reads every register of a group: the compiler
 * waits for its loads there, on every path (a path that skipped a piece
 * would leave its load pending into the next turn of the loop, where its
 * registers get reused and the compiler then waits for every load, the
 * prefetch included). */
__device__ inline void consume(const HGroup &g) {
    asm volatile("" ::"v"(g.p[0]), "v"(g.p[1]), "v"(g.p[2]), "v"(g.p[3]), "v"(g.p[4]), "v"(g.p[5]), "v"(g.p[6]));
}
static_assert(HGP == 6, "consume() names every piece");
/* The group into the wave's LDS region, as the matrix lays it out */
__device__ inline void stage_group(uint8_t *wl, const HGroup &g, int lane) {
#pragma unroll
    for (int j = 0; j < HGP; j++) *reinterpret_cast<u32x4 *>(wl + 1024 * j + 16 * lane) = g.p[j];
    if (16 * lane < HGB - 1024 * HGP) *reinterpret_cast<u32x4 *>(wl + 1024 * HGP + 16 * lane) = g.p[HGP];
}
/* The half-block h of the block that starts at byte a of the region.  A
 * block starts at 210 b of its row, so the fields of odd blocks lie at
 * 2 mod 4: the covering dwords are read from a & ~3 and shifted by a & 3
 * (0 or 2) bytes. */
__device__ inline HHalf read_half(const uint8_t *wl, uint32_t a, int h) {
    const uint32_t sh = a & 3u;
    const uint32_t *p = reinterpret_cast<const uint32_t *>(wl + (a & ~3u));
    auto al = [&](const uint32_t *q, int i) { return __builtin_amdgcn_alignbyte(q[i + 1], q[i], sh); };
    uint32_t l[17], t[9], c[3];
#pragma unroll
    for (int i = 0; i < 17; i++) l[i] = p[16 * h + i];
#pragma unroll
    for (int i = 0; i < 9; i++) t[i] = p[32 + 8 * h + i];
#pragma unroll
    for (int i = 0; i < 3; i++) c[i] = p[48 + 2 * h + i];
    HHalf r;
    r.la0 = u32x4{al(l, 0), al(l, 1), al(l, 2), al(l, 3)};
    r.la1 = u32x4{al(l, 4), al(l, 5), al(l, 6), al(l, 7)};
    r.lb0 = u32x4{al(l, 8), al(l, 9), al(l, 10), al(l, 11)};
    r.lb1 = u32x4{al(l, 12), al(l, 13), al(l, 14), al(l, 15)};
    r.h0 = u32x4{al(t, 0), al(t, 1), al(t, 2), al(t, 3)};
    r.h1 = u32x4{al(t, 4), al(t, 5), al(t, 6), al(t, 7)};
    r.sc = u32x2{al(c, 0), al(c, 1)};
    r.d = (p[52] >> (8u * sh)) & 0xFFFFu;
    return r;
}

__device__ inline uint32_t pick(const u32x4 &v, int c) { return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w; }

}  // namespace

/* One step of the segment reduce-scatter below: the lanes of each pair
 * (given by the DPP pattern CTRL) split the first M slots, the lane with
 * `hi` set keeping the upper half, and add what the partner sends; once one
 * slot is left the step only adds. */
template <int CTRL, int M>
__device__ inline void rs_step(float *v, bool hi) {
    if constexpr (M >= 2) {
#pragma unroll
        for (int i = 0; i < M / 2; i++) {
            const float send = hi ? v[i] : v[i + M / 2];
            const float keep = hi ? v[i + M / 2] : v[i];
            v[i] = keep + dpp_f<CTRL>(0.f, send);
        }
    } else {
        v[0] += dpp_f<CTRL>(0.f, v[0]);
    }
}
/* Sums N slots (N a power of two <= 16) over the 16 lanes of each row of a
 * wave and leaves slot hb >> (4 - log2 N) in lane hb: a butterfly over the
 * lane pairs hb ^ 15, hb ^ 7, hb ^ 2, hb ^ 1 (the four masks are independent,
 * so each lane ends with all 16 lanes' share of its slot). */
template <int N>
__device__ inline float rscatter16(float *v, int hb) {
    rs_step<0x140, N>(v, (hb & 8) != 0);                    /* row_mirror */
    rs_step<0x141, (N >= 2 ? N / 2 : 1)>(v, (hb & 4) != 0);  /* row_half_mirror */
    rs_step<0x4E, (N >= 4 ? N / 4 : 1)>(v, (hb & 2) != 0);   /* quad_perm 2,3,0,1 */
    rs_step<0xB1, (N >= 8 ? N / 8 : 1)>(v, (hb & 1) != 0);   /* quad_perm 1,0,3,2 */
    return v[0];
}

constexpr int pow2_at_least(int k) { return k <= 1 ? 1 : k <= 2 ? 2 : k <= 4 ? 4 : k <= 8 ? 8 : 16; }
constexpr int log2_of(int n) { return n <= 1 ? 0 : n == 2 ? 1 : n == 4 ? 2 : n == 8 ? 3 : 4; }

/* Q6_K head, 2048 columns, k <= K input rows (q8 rows in x).  best[0..k)
 * receive the argmax keys and best[16] counts finished workgroups; both
 * start at zero (cleared by the kernel that quantizes x).  The last
 * workgroup to finish writes idx[j] / val[j]. */
template <int K, bool LOGITS>
__global__ __launch_bounds__(HT, K <= 9 ? 4 : 2) void k_head_q6k(const uint8_t *__restrict__ W, int nrows, Q8Rows x, int k,
                                                 float *logits, unsigned long long *best, int32_t *idx, float *val) {
    constexpr int N = pow2_at_least(K);
    __shared__ __attribute__((aligned(16))) int8_t xq[K][HPR * XST];
    __shared__ __attribute__((aligned(16))) int32_t xs[K][NBH * 16];   /* -32 x the 16-value sums */
    __shared__ float xd[K][NBH];
    __shared__ unsigned long long wb_best[K][HW * RPW];
    __shared__ int last_wg;
    __shared__ __attribute__((aligned(16))) uint8_t wgrp[HW][HGB];   /* each wave's staged group */

    /* stage the k q8 rows: 128-value halves at XST strides */
    for (int t = threadIdx.x; t < k * NBH * 64; t += HT) {
        const int j = t / (NBH * 64), rem = t % (NBH * 64), b = rem >> 6, w = rem & 63;
        const uint32_t v = reinterpret_cast<const uint32_t *>(x.qs + ((size_t)j * NBH + b) * 256)[w];
        *reinterpret_cast<uint32_t *>(&xq[j][(2 * b + (w >> 5)) * XST + 4 * (w & 31)]) = v;
    }
    for (int t = threadIdx.x; t < k * NBH * 16; t += HT) xs[t / (NBH * 16)][t % (NBH * 16)] = -32 * x.s16[t];
    for (int t = threadIdx.x; t < k * NBH; t += HT) xd[t / NBH][t % NBH] = x.d[t];
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int hb = lane & (HPR - 1), b = hb >> 1, h = hb & 1, rsub = lane / HPR;
    /* after the reduce-scatter lane hb holds input row `slot`; with N < 16
     * several lanes hold the same one and the first of them owns it */
    const int slot = hb >> (4 - log2_of(N));
    const bool owner = (hb & (16 / N - 1)) == 0 && slot < k;
    /* wave-uniform (readfirstlane): the loop branches on scalars */
    const int gw = __builtin_amdgcn_readfirstlane(blockIdx.x * HW + (threadIdx.x >> 6)), nw = gridDim.x * HW;
    const int nq = (nrows + RPW - 1) / RPW;
    uint64_t mybest = 0;

    /* Row group q of this lane: its half-block.  Two register sets take
     * turns: the loads of the next group go out (the scheduling barrier
     * keeps them first) before the current group is computed, and the
     * compiler waits for the current one with the next one's 8 loads still
     * in flight (the group past the last reads zero past the end).  The
     * argmax-only kernel stores nothing in the loop: with stores pending
     * beside the loads the compiler's waits become vmcnt(0). */
    const Buf wbuf = make_buf(W, (uint32_t)((size_t)nrows * HRB));
    uint8_t *wl = wgrp[threadIdx.x >> 6];
    const uint32_t lane_off = (uint32_t)(rsub * HRB + b * 210);   /* the lane's block in the group */
    auto group_at = [&](int qq) { return load_group(wbuf, (uint32_t)(HGB * qq), lane); };
    int q = gw;
    auto step = [&](HGroup &grp, HGroup &nxt) {
        nxt = group_at(q + nw);
        __builtin_amdgcn_sched_barrier(0);
        consume(grp);
        /* the previous group's reads of the region are issued before these
         * writes (the LDS runs a wave's instructions in order), and the
         * reads below after them */
        asm volatile("" ::: "memory");
        stage_group(wl, grp, lane);
        asm volatile("" ::: "memory");
        const HHalf cur = read_half(wl, lane_off, h);
        const uint32_t row = (uint32_t)(RPW * q + rsub);
        /* 6-bit codes of the half (q = ql nibble | qh pair << 4), decoded once */
        const uint32_t m4 = 0x0F0F0F0Fu, m2 = 0x30303030u;
        uint32_t qc[4][8];
#pragma unroll
        for (int jj = 0; jj < 8; jj++) {
            const int c = jj & 3;
            const uint32_t la = pick(jj < 4 ? cur.la0 : cur.la1, c), lb = pick(jj < 4 ? cur.lb0 : cur.lb1, c);
            const uint32_t hh = pick(jj < 4 ? cur.h0 : cur.h1, c);
            qc[0][jj] = (la & m4) | ((hh << 4) & m2);
            qc[1][jj] = (lb & m4) | ((hh << 2) & m2);
            qc[2][jj] = ((la >> 4) & m4) | (hh & m2);
            qc[3][jj] = ((lb >> 4) & m4) | ((hh >> 2) & m2);
        }
        int sc[8];
#pragma unroll
        for (int i = 0; i < 8; i++) sc[i] = (int)(int8_t)((i < 4 ? cur.sc.x : cur.sc.y) >> (8 * (i & 3)));
        const float dw = ref_f16(cur.d);
        float vv[N];
#pragma unroll
        for (int j = 0; j < N; j++) vv[j] = 0.f;
#pragma unroll
        for (int j = 0; j < K; j++) {
            if (j < k) {
                const u32x4 *xp = reinterpret_cast<const u32x4 *>(&xq[j][hb * XST]);
                /* the 16-value sums start at -32 x the x sums: the -32 offset of
                 * the 6-bit codes */
                const u32x4 s0 = *reinterpret_cast<const u32x4 *>(&xs[j][b * 16 + 8 * h]);
                const u32x4 s1 = *reinterpret_cast<const u32x4 *>(&xs[j][b * 16 + 8 * h + 4]);
                int S[8] = {(int)s0.x, (int)s0.y, (int)s0.z, (int)s0.w, (int)s1.x, (int)s1.y, (int)s1.z, (int)s1.w};
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const u32x4 x0 = xp[2 * g], x1 = xp[2 * g + 1];
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) S[2 * g] = dot4(qc[g][jj], pick(x0, jj), S[2 * g]);
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) S[2 * g + 1] = dot4(qc[g][4 + jj], pick(x1, jj), S[2 * g + 1]);
                }
                int A = 0;
#pragma unroll
                for (int i = 0; i < 8; i++) A += __mul24(sc[i], S[i]);   /* |S| < 2^18 */
                vv[j] = dw * xd[j][b] * (float)A;
            }
        }
        const float v = rscatter16<N>(vv, hb);
        if (owner && row < (uint32_t)nrows) {
            if (LOGITS) logits[(size_t)slot * nrows + row] = v;
            const uint64_t key = argmax_key(v, row);
            mybest = key > mybest ? key : mybest;
        }
        q += nw;
    };
    /* the wave's groups in pairs, one exit at the loop's top (an exit after
     * the first step of a pair would join the loop's head with that step's
     * loads pending, and the compiler would wait for them there), then the
     * odd one */
    const int nsteps = q < nq ? (nq - 1 - q) / nw + 1 : 0;
    HGroup s0 = group_at(q), s1;
    int i = 0;
    for (; i + 2 <= nsteps; i += 2) {
        step(s0, s1);
        step(s1, s0);
    }
    if (i < nsteps) step(s0, s1);
    /* workgroup best per input row, then one atomic max each */
    if (owner && slot < K) wb_best[slot][(threadIdx.x >> 6) * RPW + rsub] = mybest;
    __syncthreads();
    if ((int)threadIdx.x < k) {
        uint64_t m = 0;
        for (int i = 0; i < HW * RPW; i++) m = wb_best[threadIdx.x][i] > m ? wb_best[threadIdx.x][i] : m;
        /* the returned value is stored (to a slot already read), so the max
         * has been performed before this thread reaches the barrier below */
        wb_best[threadIdx.x][0] = atomicMax(&best[threadIdx.x], (unsigned long long)m);
    }
    __syncthreads();
    if (threadIdx.x == 0) last_wg = atomicAdd(&best[16], 1ull) == (unsigned long long)(gridDim.x - 1);
    __syncthreads();
    if (last_wg == 1 && (int)threadIdx.x < k) {
        const uint64_t key = __hip_atomic_load(&best[threadIdx.x], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        idx[threadIdx.x] = (int32_t)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFu));
        if (val) val[threadIdx.x] = key_value(key);
    }
}

/* ---- the same head on int8 MFMA (v_mfma_i32_16x16x32_i8) ----
 * A work item is 16 vocab rows; the eight waves of a workgroup take one
 * 256-block each.  Operand layout (gfx950): A lane l = row l % 16 with
 * K = 8 (l / 16) + byte, B lane l = input row l % 16 with the same K,
 * D lane l register v = row 4 (l / 16) + v, input row l % 16.  A 32-value
 * run of a half-block is one MFMA K; its two 16-value sub-blocks come apart
 * by running it twice with the B operand zeroed in one half of K, and each
 * sub-block's sum takes its int8 sub-scale in integer.  The -32 offset of
 * the codes enters as 32 x sum_s sc[s] * xsum[s] over a half's 8
 * sub-blocks (two f32 MFMAs of K = 4; integers below 2^24, exact).  So a
 * block's integer sum is exact and its term d * d_x * sum is formed as the
 * reference forms it; the workgroup adds the eight blocks' terms in block
 * order, as the reference's row loop does (dot_q6k_q8, csrc/libtinygiant.c
 * :403-443). */
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int MW = 8;            /* waves: one 256-block each */
constexpr int MT = 64 * MW;

__device__ inline long as_long(u32x2 v) { return (long)(((uint64_t)v.y << 32) | v.x); }
__device__ inline v4i mma_i8(long a, long b) {
    const v4i z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

/* One lane's share of a 16-row item in block w: its A row's codes (both
 * halves), the row's 16 sub-scales and d (the other lanes' D rows take
 * theirs from the lanes that hold them) */
/* The MFMA kernel stages each item (16 vocab rows, 26,880 contiguous,
 * 16-byte-aligned bytes) in LDS through direct-to-LDS copies, 1 KiB an
 * instruction, in the rows' own layout.  Loads of 8 bytes a lane straight
 * from the rows touch 16 rows x 32 bytes an instruction; a timing probe with
 * the same compute and contiguous loads ran 1.4x faster.  A block starts at
 * 210 w within its row, so the fields of the odd 256-blocks lie at 2 mod 4:
 * lds8 / lds16 read the covering dwords and shift (the LDS copies read
 * 16-byte-aligned sources only). */
constexpr int HITEM = 27 * 1024;       /* 16 rows (26,880 B) and the rest of the last copy */
constexpr int HCOP = HITEM / 1024;     /* 27 copies an item */
#ifndef TG_HEAD_NB
#define TG_HEAD_NB 2
#endif
/* LDS item buffers: an item computes while HNB - 1 are in flight.  Two
 * (55 KB with the static arrays' 10 KB: two workgroups a CU) ran 69-72 us,
 * three (93 KB: one workgroup a CU) 84-86 us. */
constexpr int HNB = TG_HEAD_NB;
static_assert(16 * HRB <= HITEM && HITEM - 16 * HRB < 1024, "whole copies");
/* 8 and 16 bytes at LDS offset a of base (a even): the covering dwords from
 * a & ~3, shifted by sh = a & 3 bytes (no branch: the shift is 0 or 2) */
__device__ inline u32x2 lds8(const uint8_t *base, uint32_t a, uint32_t sh) {
    const uint32_t *p = (const uint32_t *)(base + (a & ~3u));
    const uint32_t d0 = p[0], d1 = p[1], d2 = p[2];
    return u32x2{__builtin_amdgcn_alignbyte(d1, d0, sh), __builtin_amdgcn_alignbyte(d2, d1, sh)};
}
__device__ inline u32x4 lds16(const uint8_t *base, uint32_t a, uint32_t sh) {
    const uint32_t *p = (const uint32_t *)(base + (a & ~3u));
    const uint32_t d0 = p[0], d1 = p[1], d2 = p[2], d3 = p[3], d4 = p[4];
    return u32x4{__builtin_amdgcn_alignbyte(d1, d0, sh), __builtin_amdgcn_alignbyte(d2, d1, sh),
                 __builtin_amdgcn_alignbyte(d3, d2, sh), __builtin_amdgcn_alignbyte(d4, d3, sh)};
}
}  // namespace

/* Q6_K head, 2048 columns, k <= 16 input rows: the contract of k_head_q6k. */
__global__ __launch_bounds__(MT) void k_head_q6k_mfma(const uint8_t *__restrict__ W, int nrows, Q8Rows x, int k,
                                                     float *logits, unsigned long long *best, int32_t *idx,
                                                     float *val) {
    __shared__ __attribute__((aligned(16))) float red[2][MW][4][64];   /* the waves' block terms, by item parity */
    __shared__ unsigned long long wb_best[16][16];
    __shared__ int last_wg;
    extern __shared__ __attribute__((aligned(16))) uint8_t hl[];   /* [HNB][HITEM] */
    const int tid = threadIdx.x, lane = tid & 63, c16 = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);

    /* input row c16's operands of block w, for the whole kernel: run m of
     * half h at K slice 8 g .. 8 g + 7, zeroed outside the sub-block each
     * MFMA of a pair keeps; the 16-value sums this lane's K of the offset
     * MFMAs needs; the block scale.  Rows c16 >= k read zeros (the buffers
     * end at row k). */
    long x0[2][4], x1[2][4];
    float s16a[2], s16b[2];
    float xd;
    {
        const Buf qs_b = make_buf(x.qs, (uint32_t)k * NBH * 256u);
        const Buf s16_b = make_buf(x.s16, (uint32_t)k * NBH * 64u);
        const uint32_t qo = ((uint32_t)c16 * NBH + (uint32_t)w) * 256u;
#pragma unroll
        for (int h = 0; h < 2; h++) {
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const long xb = as_long(ld8(qs_b, qo + 128u * h + 32u * m + 8u * (uint32_t)g));   /* 0 past k */
                x0[h][m] = g < 2 ? xb : 0l;
                x1[h][m] = g < 2 ? 0l : xb;
            }
            const uint32_t so = ((uint32_t)c16 * NBH + (uint32_t)w) * 64u + 32u * h;
            s16a[h] = (float)(int)ld4(s16_b, so + 4u * (uint32_t)g);
            s16b[h] = (float)(int)ld4(s16_b, so + 16u + 4u * (uint32_t)g);
        }
        const Buf d_b = make_buf(x.d, (uint32_t)k * NBH * 4u);
        xd = __uint_as_float(ld4(d_b, ((uint32_t)c16 * NBH + (uint32_t)w) * 4u));
    }

    const int nq = (nrows + 15) / 16;
    const u32x4 wd = buf_desc(W, (uint32_t)((size_t)nrows * HRB));   /* rows past nrows read zeros */
    /* the operand loads above complete before any untracked item load goes out */
    __builtin_amdgcn_s_waitcnt(0x0F70);   /* vmcnt(0) */
    /* epilogue thread (tid < 256): D register ev of lane el */
    const int ev = tid >> 6, el = tid & 63, ej = el & 15;
    uint64_t mybest = 0;
    int q = blockIdx.x;
    /* copy j of this wave moves the item's KiB w + 8 j */
    const int ncw = (HCOP - w + 7) / 8;   /* 4 or 3 copies an item */
    uint32_t csrc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) csrc[j] = 1024u * (uint32_t)(w + 8 * j) + 16u * (uint32_t)lane;
    auto issue_item = [&](int qi, int b) {
        const uint32_t base = (uint32_t)qi * 16u * HRB;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (j < ncw) copy_lanes(wd, base + csrc[j], lds_addr(hl + b * HITEM + 1024 * (w + 8 * j)));
    };
    const int G = (int)gridDim.x;
#pragma unroll
    for (int i = 0; i < HNB - 1; i++) issue_item(q + i * G, i);
    /* the epilogue of an item: its 16 rows' logits and argmax keys from the
     * waves' block terms, added in block order (tid < 256) */
    auto epilogue = [&](int qe, const float (&rb)[MW][4][64]) {
        if (tid < 256) {
            const uint32_t row = 16u * (uint32_t)qe + 4u * (uint32_t)(el >> 4) + (uint32_t)ev;
            float s = 0.f;
#pragma unroll
            for (int b = 0; b < MW; b++) s = __fadd_rn(s, rb[b][ev][el]);
            if (ej < k && row < (uint32_t)nrows) {
                if (logits) logits[(size_t)ej * nrows + row] = s;
                const uint64_t key = argmax_key(s, row);
                mybest = key > mybest ? key : mybest;
            }
        }
    };
    /* One barrier an item.  Past it, item q's copies have landed (each wave
     * waited for its own) and every wave has computed the item before: its
     * buffer takes the copies of the item HNB - 1 ahead, and its block terms
     * (in the other half of red) are added up while item q computes. */
    int it = 0;
    for (int bi = 0; q < nq; bi = bi == HNB - 1 ? 0 : bi + 1, it++) {
        /* this item's copies: the later items' (ncw each) stay in flight */
        if (ncw == 4) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * (HNB - 2)) : "memory");
        else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * (HNB - 2)) : "memory");
        bar_lds();
        issue_item(q + (HNB - 1) * G, bi == 0 ? HNB - 1 : bi - 1);
        if (it > 0) epilogue(q - G, red[(it - 1) & 1]);
        const uint8_t *ib = hl + bi * HITEM;
        const uint32_t odd = 2u * (uint32_t)(w & 1);   /* byte shift of block w's fields */
        const uint32_t mb = (uint32_t)c16 * HRB + 210u * (uint32_t)w;   /* this lane's row of block w */
        u32x2 qlv[2][2], qhv[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            qlv[h][0] = lds8(ib, mb + 64u * h + 8u * g, odd);
            qlv[h][1] = lds8(ib, mb + 64u * h + 32u + 8u * g, odd);
            qhv[h] = lds8(ib, mb + 128u + 32u * h + 8u * g, odd);
        }
        const u32x4 sco = lds16(ib, mb + 192u, odd);
        /* the sub-scales and d of D rows 4 g + v */
        u32x4 sc[4];
        float dv[4];
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const uint32_t rv = (uint32_t)(4 * g + v) * HRB + 210u * (uint32_t)w;
            sc[v] = lds16(ib, rv + 192u, odd);
            dv[v] = ref_f16(*(const uint16_t *)(ib + rv + 208u));
        }
        int isum[4] = {0, 0, 0, 0};
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t sw0 = h ? sco.z : sco.x, sw1 = h ? sco.w : sco.y;
            v4f cf = {0.f, 0.f, 0.f, 0.f};
            cf = __builtin_amdgcn_mfma_f32_16x16x4f32((float)(int8_t)(sw0 >> (8 * g)), s16a[h], cf, 0, 0, 0);
            cf = __builtin_amdgcn_mfma_f32_16x16x4f32((float)(int8_t)(sw1 >> (8 * g)), s16b[h], cf, 0, 0, 0);
            int ai[4] = {0, 0, 0, 0};
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const u32x2 ql = qlv[h][m & 1], qh = qhv[h];
                const int sl = 4 * (m >> 1), sh = 2 * m;
                u32x2 c;
                c.x = ((ql.x >> sl) & 0x0F0F0F0Fu) | (((qh.x >> sh) & 0x03030303u) << 4);
                c.y = ((ql.y >> sl) & 0x0F0F0F0Fu) | (((qh.y >> sh) & 0x03030303u) << 4);
                const v4i d0 = mma_i8(as_long(c), x0[h][m]), d1 = mma_i8(as_long(c), x1[h][m]);
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const u32x4 &sv = sc[v];
                    const uint32_t sw = (m >> 1) ? (h ? sv.w : sv.y) : (h ? sv.z : sv.x);
                    const int sc0 = (int)(int8_t)(sw >> (16 * (m & 1))), sc1 = (int)(int8_t)(sw >> (16 * (m & 1) + 8));
                    ai[v] += __mul24(sc0, d0[v]) + __mul24(sc1, d1[v]);   /* |.| < 2^24 per term */
                }
            }
#pragma unroll
            for (int v = 0; v < 4; v++) isum[v] += ai[v] - 32 * (int)cf[v];
        }
        /* the block's term d * d_x * sum, as the reference forms it */
        float (&rb)[MW][4][64] = red[it & 1];   /* added up after the next item's barrier */
#pragma unroll
        for (int v = 0; v < 4; v++) rb[w][v][lane] = __fmul_rn(__fmul_rn(dv[v], xd), (float)isum[v]);
        q += G;
    }
    bar_lds();   /* LDS only: the last item's block terms are in */
    if (it > 0) epilogue(q - G, red[(it - 1) & 1]);
    /* the copies of the items past the end land before the wave ends */
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    /* workgroup best per input row (16 epilogue threads each), then one
     * atomic max each; the last workgroup writes the result */
    if (tid < 256) wb_best[ej][ev * 4 + (el >> 4)] = mybest;
    __syncthreads();
    if (tid < k) {
        uint64_t m = 0;
        for (int i = 0; i < 16; i++) m = wb_best[tid][i] > m ? wb_best[tid][i] : m;
        /* the returned value is stored (to a slot already read), so the max
         * has been performed before this thread reaches the barrier below */
        wb_best[tid][0] = atomicMax(&best[tid], (unsigned long long)m);
    }
    __syncthreads();
    if (tid == 0) last_wg = atomicAdd(&best[16], 1ull) == (unsigned long long)(gridDim.x - 1);
    __syncthreads();
    if (last_wg == 1 && tid < k) {
        const uint64_t key = __hip_atomic_load(&best[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        idx[tid] = (int32_t)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFu));
        if (val) val[tid] = key_value(key);
    }
}

/* argmax of logits [k][nrows] (one workgroup per input row) */
__global__ __launch_bounds__(256) void k_argmax_rows(const float *__restrict__ logits, int nrows,
                                                     unsigned long long *best) {
    __shared__ unsigned long long red[256];
    const int j = blockIdx.x;
    uint64_t m = 0;
    for (int r = threadIdx.x; r < nrows; r += 256) {
        const uint64_t key = argmax_key(logits[(size_t)j * nrows + r], (uint32_t)r);
        m = key > m ? key : m;
    }
    red[threadIdx.x] = m;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s && red[threadIdx.x + s] > red[threadIdx.x]) red[threadIdx.x] = red[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) best[j] = red[0];
}

__global__ void k_argmax_finish(const unsigned long long *best, int k, int32_t *idx, float *val) {
    const int j = threadIdx.x;
    if (j >= k) return;
    const uint64_t key = best[j];
    idx[j] = (int32_t)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFu));
    if (val) val[j] = key_value(key);
}

/* At most 2^20 rows: a head (1.76 GB) and the groups read past its end stay
 * below 2^31 bytes, where the tail lanes' offset points. */
bool head_fast_ok(int fmt, int ncols, int nrows, int k) {
    return fmt == TG_FMT_Q6K && ncols == NBH * 256 && nrows >= 1 && nrows <= (1 << 20) && k >= 1 && k <= 16;
}

/* From this many input rows the int8 MFMA kernel reads the head: its work
 * does not grow with k (151936 x 2048: 68-70 us for every k), the v_dot4
 * kernel's does (61-62 us at k = 5, 72-78 at 8, 76-79 at 9, 102-104 at 12,
 * 121-123 at 16). */
#ifndef TG_HEAD_MFMA_MIN_K
#define TG_HEAD_MFMA_MIN_K 8
#endif
static int g_head_mfma_min_k = TG_HEAD_MFMA_MIN_K;
int set_head_mfma_min_k(int k) {
    const int prev = g_head_mfma_min_k;
    g_head_mfma_min_k = k < 0 ? 0 : k;
    return prev;
}

void launch_head_q6k(const uint8_t *W, int nrows, const Q8Rows &x, int k, float *logits, unsigned long long *best,
                     int32_t *idx, float *val, hipStream_t st) {
    int dev = 0, cus = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (g_head_mfma_min_k > 0 && k >= g_head_mfma_min_k) {
        static int occ = -1;
        const size_t lds = (size_t)HNB * HITEM;
        if (occ < 0 && (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k_head_q6k_mfma, MT, lds) != hipSuccess ||
                        occ < 1))
            occ = 1;
        const int nq = (nrows + 15) / 16;
        const int grid = std::max(1, std::min(std::max(cus, 1) * occ, nq));
        hipLaunchKernelGGL(k_head_q6k_mfma, dim3(grid), dim3(MT), lds, st, W, nrows, x, k, logits, best, idx, val);
        return;
    }
    const int nq = (nrows + RPW - 1) / RPW;
    /* one round of workgroups: each walks its groups with a fixed stride, so
     * a second round would double the time */
    auto launch = [&](const void *fn, int &occ) {
        if (occ < 0 && (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, HT, 0) != hipSuccess || occ < 1)) occ = 1;
        const int grid = std::max(1, std::min(std::max(cus, 1) * occ, (nq + HW - 1) / HW));
        void *args[] = {(void *)&W, (void *)&nrows, (void *)&x, (void *)&k, (void *)&logits, (void *)&best, (void *)&idx,
                        (void *)&val};
        (void)hipLaunchKernel(fn, dim3(grid), dim3(HT), args, 0, st);
    };
/* k is rounded up to an instantiated K; rows j >= k skip their dots */
#define TG_HEAD(KK)                                                                  \
    do {                                                                             \
        static int occ_l = -1, occ_n = -1;                                           \
        if (logits) launch(reinterpret_cast<const void *>(&k_head_q6k<KK, true>), occ_l);  \
        else launch(reinterpret_cast<const void *>(&k_head_q6k<KK, false>), occ_n);        \
    } while (0)
    if (k <= 1) TG_HEAD(1);
    else if (k <= 2) TG_HEAD(2);
    else if (k <= 4) TG_HEAD(4);
    else if (k <= 5) TG_HEAD(5);
    else if (k <= 8) TG_HEAD(8);
    else if (k <= 9) TG_HEAD(9);
    else TG_HEAD(16);
#undef TG_HEAD
}

void launch_argmax_rows(const float *logits, int nrows, int k, unsigned long long *best, hipStream_t st) {
    hipLaunchKernelGGL(k_argmax_rows, dim3(k), dim3(256), 0, st, logits, nrows, best);
}

void launch_argmax_finish(const unsigned long long *best, int k, int32_t *idx, float *val, hipStream_t st) {
    hipLaunchKernelGGL(k_argmax_finish, dim3(1), dim3(64), 0, st, best, k, idx, val);
}

}  // namespace tg
