/*
 * tg_grouped_k.hip -- Q4_K gate/up and Q6_K down expert phases on int8 MFMA
 * for layers whose experts hold many pairs (a prefill, a long verify batch):
 * moe_phase_a / moe_phase_b of csrc/libtinygiant.c:1279-1384 with the
 * per-block dots of dot_q4k_q8 (:223-272) and dot_q6k_q8 (:384-443), the
 * contraction the reference groups four rows at a time (dot_q4k_q8_x4
 * :276-337, dot_q6k_q8_x4 :445-487) done sixteen pairs at a time.
 *
 * Arithmetic.  v_mfma_i32_16x16x32_i8 sums 32 int8 products exactly.  A
 * Q4_K sub-block is 32 values under one 6-bit scale and min, so one MFMA per
 * sub-block gives the reference's integer sums idot for 16 weight rows x 16
 * pairs, and the scale work is the reference's per group g of two
 * sub-blocks, summed here over the block: d * sum_s sc_s idot_s - dmin *
 * sum_s m_s bs_s, both sums exact (int32, and the min sums, a 16 x 16
 * product of 8-long integer vectors, on two f32 MFMAs of K = 4 whose
 * products and sums stay integers below 2^24).  A Q6_K sub-block is 16
 * values under one int8 scale: each 32-value chunk of a half-block runs
 * twice, the pair operand zero in one half of K each time, so the two
 * sub-block sums come out apart; the 6-bit codes enter unshifted and the
 * -32 offset is folded in with the pair's 16-value sums (sum (c - 32) x sc =
 * sum c x sc - 32 sum sc sum x, the last on two f32 MFMAs), exact in int32
 * per half-block.  Only the f32 additions (per block or half-block, then
 * across waves) are associated differently from the reference's
 * sub-block-by-sub-block sum.
 *
 * Operand layout of v_mfma_i32_16x16x32_i8 (measured on gfx950): A lane l =
 * row l % 16 of A, K = 8 (l / 16) + byte; B lane l = column l % 16, the same
 * K; D lane l, register v = A row 4 (l / 16) + v, B column l % 16.  The pairs'
 * q8 operands go in as A and the weight rows as B, so the four sums of a lane
 * share one weight row (lane % 16) and its scales.
 *
 * Work: one workgroup per (16-row slab, active expert).  The slab is staged
 * in LDS (Q6_K blocks re-spaced to 224 bytes so every field is aligned, each
 * load inside its block, since a buffer load that runs past the matrix end
 * reads zero as a whole); the
 * four waves split the row's blocks (Q4_K) or half-blocks (Q6_K); each pass
 * runs 16 pairs of the expert against the resident slab, their q8 operands
 * read from the q8 rows in global memory; 256 threads add the waves' partial
 * sums in wave order and write one result each.  HBM sees each weight byte
 * once however many pairs the expert holds.
 */
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "tg_device.hpp"
#include "tg_kernels.h"
#include "tg_xchg.hpp"

namespace tg {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

/* four waves a workgroup: three workgroups (twelve waves, three slabs in
 * flight) share a CU, within its LDS; eight waves a workgroup measured 16%
 * slower (two workgroups a CU) */
constexpr int NW = 4;                    /* waves per workgroup */
constexpr int NT = 64 * NW;
constexpr uint32_t OOB = 0x80000000u;    /* past every buffer: the load reads zero */
constexpr uint32_t Q4B = 144, Q6B = 210; /* bytes per 256-value block */
constexpr uint32_t Q6S = 224;            /* LDS stride of a staged Q6_K block */
/* A gate/up wave's q8 operands of a pass are loaded at once: QA_WB Q4_K
 * blocks of a row (D <= 256 NW QA_WB), in a form for Qwen3's 8 blocks of D
 * (fewer registers) and one for longer rows. */
constexpr int QA_WB_MAX = 3;

__device__ inline long as_long(u32x2 v) { return (long)(((uint64_t)v.y << 32) | v.x); }

/* a wave-uniform read of a read-only table through the constant address
 * space: a scalar load, counted apart from the vector loads */
template <class T>
__device__ inline T ldc(const T *p, size_t i) {
    return ((const __attribute__((address_space(4))) T *)(uintptr_t)p)[i];
}

__device__ inline v4i mma(long a, long b) {
    const v4i z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

/* LDS bytes: the gate and up slabs (rows 16 bytes apart more than their
 * length, so the 16 lanes reading one sub-block of 16 rows hit distinct
 * banks; each slab rounded up to whole 1 KiB copies), then the waves'
 * partial sums.  Q6_K slabs likewise pad each row of blocks by 16 bytes. */
__host__ __device__ inline uint32_t qa_row_stride(int D) { return (uint32_t)(D / 256) * Q4B + 16u; }
__host__ __device__ inline uint32_t qa_slab_region(int D) { return (16u * qa_row_stride(D) + 1023u) & ~1023u; }
__host__ __device__ inline uint32_t qb_row_stride(int I) { return (uint32_t)(I / 256) * Q6S + 16u; }
__host__ __device__ inline size_t qa_lds_bytes(int D) {
    return 2u * (size_t)qa_slab_region(D) + (size_t)NW * 2 * 4 * 64 * 4;
}
__host__ __device__ inline size_t qb_lds_bytes(int I) { return 64u * (size_t)qb_row_stride(I); }

/* 6-bit scales and mins of a Q4_K block header (get_scale_min_k4,
 * csrc/libtinygiant.c:146-155), four bytes at a time: sc of sub-blocks 0-3,
 * 4-7, then the mins */
struct Q4Hdr {
    float d, dmin;
    uint32_t scl, sch, mnl, mnh;
};
__device__ inline Q4Hdr q4_hdr(u32x4 h) {
    Q4Hdr r;
    const uint32_t m4 = 0x0F0F0F0Fu;
    r.d = ref_f16(h.x & 0xFFFFu);
    r.dmin = ref_f16(h.x >> 16);
    r.scl = h.y & 0x3F3F3F3Fu;
    r.mnl = h.z & 0x3F3F3F3Fu;
    r.sch = (h.w & m4) | ((h.y >> 2) & 0x30303030u);
    r.mnh = ((h.w >> 4) & m4) | ((h.z >> 2) & 0x30303030u);
    return r;
}
__device__ inline int byte_of(uint32_t w, int i) { return (int)((w >> (8 * i)) & 0xFFu); }

/* copy_lanes with the nontemporal hint: each slab byte is read once per
 * call (64- and 128-token Qwen3 prefills measured 5% faster with it); the
 * same 5 wait states before the load */
__device__ inline void copy_lanes_nt(const u32x4 &desc, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 3\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
                 :
                 : "s"(lds), "v"(voff), "s"(desc)
                 : "memory");
}

}  // namespace

/* Phase A: hidden[p][r] = act(gate_r . xq_p + bg[r], up_r . xq_p + bu[r])
 * for rows r of slab blockIdx.x and every pair p of active expert
 * a.ed[blockIdx.y]; Q4_K gate and up matrices of D = 256 nb columns.  The
 * slabs arrive by direct-to-LDS copies, while the first pass's q8 operands
 * load into registers. */
template <int QA_WB>
__global__ __launch_bounds__(NT) void k_moe_qa(MoeArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const ExpDesc &ex = a.ed[blockIdx.y];
    const int e = ex.e, p0 = ex.p0, np = ex.np;
    const int nb = a.D / 256;
    const uint32_t rb = (uint32_t)nb * Q4B, rs = qa_row_stride(a.D), sreg = qa_slab_region(a.D);
    float *red = (float *)(lds + 2 * sreg);   /* [NW][2][4][64] */
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, c16 = lane & 15;
    const int r0 = blockIdx.x * 16;

    /* the slabs, 1 KiB of LDS a copy: lane l of copy k fills LDS bytes
     * 1024 k + 16 l, i.e. row (1024 k + 16 l) / rs at that column (the row
     * padding and rows past 16 or past I read zero) */
    {
        const uint32_t mbytes = (uint32_t)a.I * rb, base = (uint32_t)r0 * rb, nins = sreg / 1024u;
        const u32x4 gd = buf_desc((const void *)(uintptr_t)ex.gate, mbytes);
        const u32x4 ud = buf_desc((const void *)(uintptr_t)ex.up, mbytes);
        for (uint32_t k = (uint32_t)w; k < nins; k += NW) {
            const uint32_t P = 1024u * k + 16u * (uint32_t)lane, row = P / rs, col = P - row * rs;
            const uint32_t src = row < 16u && col < rb ? base + row * rb + col : OOB;
            copy_lanes_nt(gd, src, lds_addr(lds + 1024u * k));
            copy_lanes_nt(ud, src, lds_addr(lds + sreg + 1024u * k));
        }
    }
    const Q8Rows &q = a.xq;
    const Buf qs_b = make_buf(q.qs, (uint32_t)((size_t)a.k * nb * 256));
    const Buf s32_b = make_buf(q.s32, (uint32_t)((size_t)a.k * nb * 32));
    const Buf d_b = make_buf(q.d, (uint32_t)((size_t)a.k * nb * 4));
    /* the input row of pair t + c16 (0 past the expert's pairs): the 16 rows
     * come through the scalar path, so waiting for them does not wait for
     * the slab copies queued on the vector path */
    auto pair_row = [&](int t) {
        uint32_t rj[16];
#pragma unroll
        for (int j = 0; j < 16; j++) rj[j] = (uint32_t)ldc(a.p_row, (size_t)min(p0 + t + j, a.P - 1));
        uint32_t r = 0u;
#pragma unroll
        for (int j = 0; j < 16; j++) r = c16 == j && t + j < np ? rj[j] : r;
        return r;
    };
    const float *gbias = a.gbias ? (const float *)(uintptr_t)a.gbias[e] : nullptr;
    const float *ubias = a.ubias ? (const float *)(uintptr_t)a.ubias[e] : nullptr;

    /* pair c16's q8 operands of the wave's blocks b = w + NW i of a pass,
     * all loaded at once: sub-block s = 2 jg + half covers x[64 jg + 32 half
     * ...], this lane's K slice 8 g .. 8 g + 7 */
    long xb[QA_WB][8];
    float bsg0[QA_WB], bsg1[QA_WB];   /* the pair's 32-value sums of sub-blocks g and 4 + g */
    float xd[QA_WB];
    auto load_x = [&](uint32_t prow, bool pv) {
#pragma unroll
        for (int i = 0; i < QA_WB; i++) {
            const int b = w + NW * i;
            const bool v = pv && b < nb;
            const uint32_t qb = prow * (uint32_t)nb + (uint32_t)b;
#pragma unroll
            for (int s = 0; s < 8; s++)
                xb[i][s] = as_long(ld8(qs_b, v ? qb * 256u + 64u * (s >> 1) + 32u * (s & 1) + 8u * g : OOB));
            bsg0[i] = (float)(int)ld4(s32_b, v ? qb * 32u + 4u * g : OOB);
            bsg1[i] = (float)(int)ld4(s32_b, v ? qb * 32u + 16u + 4u * g : OOB);
            xd[i] = __uint_as_float(ld4(d_b, v ? qb * 4u : OOB));
        }
    };
    int t0 = 0;
    bool pv = c16 < np;
    uint32_t prow = pair_row(0);
    load_x(prow, pv);
    wait_copies();
    __syncthreads();

    for (;;) {
        float acc[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int i = 0; i < QA_WB; i++) {
            const int b = w + NW * i;
            if (b >= nb) break;   /* uniform per wave */
#pragma unroll 1
            for (int m = 0; m < 2; m++) {
                const uint8_t *sb = lds + m * sreg;
                /* the pairs' q8 operands are the MFMA's A side and the weight
                 * rows its B side, so a lane's four sums belong to one row
                 * (c16) and four pairs (4 g + v): one header a lane */
                const Q4Hdr hr = q4_hdr(*(const u32x4 *)(sb + c16 * rs + b * Q4B));
                float xdv[4];
#pragma unroll
                for (int v = 0; v < 4; v++) xdv[v] = __shfl(xd[i], 4 * g + v, 64);
                /* the min terms sum_s bs[pair][s] m[row][s] of the 16 pairs x 16
                 * rows: two f32 MFMAs of K = 4 (sub-blocks g and 4 + g of this
                 * lane group; products and sums are integers below 2^24, exact) */
                v4f im = {0.f, 0.f, 0.f, 0.f};
                im = __builtin_amdgcn_mfma_f32_16x16x4f32(bsg0[i], (float)byte_of(hr.mnl, g), im, 0, 0, 0);
                im = __builtin_amdgcn_mfma_f32_16x16x4f32(bsg1[i], (float)byte_of(hr.mnh, g), im, 0, 0, 0);
                /* the scale terms sum_s sc[row][s] idot[pair][row][s]: one int8
                 * MFMA per sub-block, summed exactly in int32 */
                const uint8_t *ab = sb + c16 * rs + b * Q4B + 16 + 8 * g;   /* row c16's codes */
                int isc[4] = {0, 0, 0, 0};
#pragma unroll
                for (int jg = 0; jg < 4; jg++) {
                    const u32x2 qq = *(const u32x2 *)(ab + 32 * jg);
                    u32x2 lo, hi;
                    lo.x = qq.x & 0x0F0F0F0Fu;
                    lo.y = qq.y & 0x0F0F0F0Fu;
                    hi.x = (qq.x >> 4) & 0x0F0F0F0Fu;
                    hi.y = (qq.y >> 4) & 0x0F0F0F0Fu;
                    const v4i dl = mma(xb[i][2 * jg], as_long(lo));
                    const v4i dh = mma(xb[i][2 * jg + 1], as_long(hi));
                    const uint32_t scw = jg < 2 ? hr.scl : hr.sch;
                    const int s0 = byte_of(scw, 2 * (jg & 1)), s1 = byte_of(scw, 2 * (jg & 1) + 1);
#pragma unroll
                    for (int v = 0; v < 4; v++) isc[v] += __mul24(s0, dl[v]) + __mul24(s1, dh[v]);
                }
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    /* acc indexed with constants only (m is a loop variable) */
                    const float t = xdv[v] * (hr.d * (float)isc[v] - hr.dmin * im[v]);
                    if (m == 0) acc[0][v] += t;
                    else acc[1][v] += t;
                }
            }
        }
        /* the waves' partial sums (block order), then one result per thread */
#pragma unroll
        for (int m = 0; m < 2; m++)
#pragma unroll
            for (int v = 0; v < 4; v++) red[((w * 2 + m) * 4 + v) * 64 + lane] = acc[m][v];
        /* the next pass's q8 operands load while this one is written out */
        const int t1 = t0 + 16;
        if (t1 < np) {
            pv = t1 + c16 < np;
            prow = pair_row(t1);
            load_x(prow, pv);
        }
        __syncthreads();
        if (tid < 256) {
            /* register ev of D lane el: pair 4 (el / 16) + ev, slab row el % 16 */
            const int ev = tid >> 6, el = tid & 63;
            const int jj = t0 + 4 * (el >> 4) + ev, r = r0 + (el & 15);
            if (jj < np && r < a.I) {
                float gv = 0.f, uv = 0.f;
#pragma unroll
                for (int ww = 0; ww < NW; ww++) {
                    gv += red[((ww * 2 + 0) * 4 + ev) * 64 + el];
                    uv += red[((ww * 2 + 1) * 4 + ev) * 64 + el];
                }
                if (gbias) gv += gbias[r];
                if (ubias) uv += ubias[r];
                a.hidden[(size_t)(p0 + jj) * a.I + r] = act_fn(a.act, gv, uv);
            }
        }
        if (t1 >= np) break;
        t0 = t1;
        __syncthreads();   /* red is rewritten by the next pass */
    }
}

/* Phase A, persistent, for Q4_K gate/up rows of D = 2048 (8 blocks): one
 * workgroup a compute unit walks its list of items (active expert, 16-row
 * slab, pass of 16 pairs), the slabs streaming through a ring of four LDS
 * slots three items ahead of the item computed, so a compute unit always
 * has weight bytes in flight.
 *
 * Eight compute waves: wave c takes matrix c / 4 (gate, up) and blocks
 * c % 4 and c % 4 + 4 of it, so the partial sums of a block pair meet in
 * LDS in the order of the expert-major kernel (wave order).  They hold the
 * q8 operands of a run of items with the same expert and pass, loaded once
 * a run (a compute unit returns its loads in issue order, so operands loaded
 * per item would wait behind the slabs in flight each time); a workgroup's
 * list is a contiguous stretch of the layer's items ordered expert, pass,
 * slab, so it holds a few runs.  Two copy waves issue the slab copies
 * (direct-to-LDS, one matrix each) and nothing else, so each waits for its
 * own with exact counts; two finishing waves finish the previous item (its
 * partial sums, double-buffered in LDS, the activation, the hidden values)
 * while the compute waves work on the current one, one barrier an item.
 *
 * A slab's LDS image swizzles each row's 16-byte units within aligned
 * groups of eight (unit u of row r at 72 r + (u ^ ((r >> 1) & 7))): the 16
 * rows a lane group reads at one column then fall on distinct banks. */
constexpr int RG_NB = 8;                              /* Q4_K blocks of a row */
constexpr int RG_UNITS = RG_NB * 9;                   /* 16-byte units of a 1152-byte row */
constexpr int RG_SLAB = 16 * RG_UNITS * 16;           /* 18,432 bytes: one matrix's 16 rows */
constexpr int RG_COPIES = RG_SLAB / 1024;             /* 18 copies of 1 KiB */
constexpr int RG_SLOTS = 4;
constexpr int RG_CW = 8, RG_YW = 2, RG_FW = 2;        /* compute, copy and finishing waves */
constexpr int RG_LC = RG_COPIES;                      /* copies a copy wave issues per item (its matrix's slab) */
constexpr int RG_NT = 64 * (RG_CW + RG_YW + RG_FW);
constexpr int RG_FO = 16 * 16 / (64 * RG_FW);         /* (pair, row) results a finishing thread writes */
static_assert(2 * RG_LC <= 63, "a vmcnt count");
static_assert(RG_SLAB % 1024 == 0, "whole copies");
static_assert(RG_UNITS % 8 == 0, "the swizzle stays inside a row");

__device__ inline uint32_t rg_unit(int r, int u) { return (uint32_t)(RG_UNITS * r + (u ^ ((r >> 1) & 7))); }

struct RgX {   /* a compute lane's q8 operands of one run, blocks c % 4 and c % 4 + 4 */
    long xb[2][8];
    uint32_t bs0[2], bs1[2], xd[2];
    float xdv[2][4];   /* the scales of pairs 4 g .. 4 g + 3, set once the run starts */
};

__global__ __launch_bounds__(RG_NT) void k_moe_qa_ring(MoeArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t ring[RG_SLOTS][2][RG_SLAB];
    __shared__ __attribute__((aligned(16))) float red[2][RG_CW][4][64];   /* by item parity */
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, g = lane >> 4,
              c16 = lane & 15;
    const bool loader = w >= RG_CW, copier = loader && w < RG_CW + RG_YW;
    const int i0 = ldc(a.rg_off, blockIdx.x), n = ldc(a.rg_off, blockIdx.x + 1) - i0;
    if (n <= 0) return;   /* uniform */
    const uint32_t mbytes = (uint32_t)a.I * (RG_NB * Q4B);
    const Q8Rows &q = a.xq;
    const Buf qs_b = make_buf(q.qs, (uint32_t)((size_t)a.k * RG_NB * 256));
    const Buf s32_b = make_buf(q.s32, (uint32_t)((size_t)a.k * RG_NB * 32));
    const Buf d_b = make_buf(q.d, (uint32_t)((size_t)a.k * RG_NB * 4));
    const int mw = (w >> 2) & 1, bw = w & 3;   /* a compute wave's matrix and first block */

    /* item j of the list (j < n): expert index, slab, pass */
    auto item = [&](int j) { return ldc(a.rg_items, (size_t)(i0 + j)); };
    /* What the copy and finishing waves need of an item comes through the
     * scalar path in stages, each from loads issued an item earlier (an item
     * code, then its expert's entries, then the biases): a chain of dependent
     * scalar loads in one item's step would stall the wave for each round
     * trip, and the barrier with it. */
    struct Info {   /* a copy wave's: its matrix (gate for wave RG_CW, up for the next) and slab */
        uint64_t base;
        int s;
    };
    auto info_code = [&](int it) __attribute__((always_inline)) {
        Info f;
        f.base = w - RG_CW ? ldc(&a.ed[it >> 16].up, 0) : ldc(&a.ed[it >> 16].gate, 0);
        f.s = (it >> 8) & 255;
        return f;
    };
    struct Fin {   /* a finishing wave's: slab, pairs, biases */
        int s, tp, p0, np, e;
        const float *gb, *ub;
    };
    auto fin_head = [&](int it) __attribute__((always_inline)) {
        Fin f;
        f.s = (it >> 8) & 255;
        f.tp = 16 * (it & 255);
        f.p0 = ldc(&a.ed[it >> 16].p0, 0);
        f.np = ldc(&a.ed[it >> 16].np, 0);
        f.e = ldc(&a.ed[it >> 16].e, 0);
        return f;
    };
    auto fin_bias = [&](Fin &f) __attribute__((always_inline)) {
        f.gb = a.gbias ? (const float *)(uintptr_t)ldc(a.gbias, f.e) : nullptr;
        f.ub = a.ubias ? (const float *)(uintptr_t)ldc(a.ubias, f.e) : nullptr;
    };
    /* the copy wave's matrix slab of item j, 18 KiB */
    auto issue_copies = [&](int j, const Info &f) __attribute__((always_inline)) {
        const int s = f.s, m = w - RG_CW;
        const u32x4 desc = buf_desc((const void *)(uintptr_t)f.base, mbytes);
        uint8_t *dst = &ring[j % RG_SLOTS][m][0];
#pragma unroll
        for (int k = 0; k < RG_LC; k++) {
            const int P = 64 * k + lane, r = P / RG_UNITS, u = (P % RG_UNITS) ^ ((r >> 1) & 7);
            copy_lanes_nt(desc, (uint32_t)(s * 16 + r) * (RG_NB * Q4B) + 16u * (uint32_t)u, lds_addr(dst + 1024 * k));
        }
    };
    /* the loader wave waits for item j's copies, k items' copies issued after them */
    auto wait_copies_behind = [&](int k) __attribute__((always_inline)) {
        if (k >= 2) wait_copies_but<2 * RG_LC>();
        else if (k == 1) wait_copies_but<RG_LC>();
        else wait_copies_but<0>();
    };
    static_assert(RG_SLOTS - 2 == 2, "wait_copies_behind covers the items in flight");
    /* the compute lane's operands of run r: its pair c16, whose input row the
     * run's record holds (one round trip of scalar loads) */
    auto load_x = [&](int r, RgX &x) __attribute__((always_inline)) {
        const int *rc = a.rg_runs + (size_t)RING_REC * r;
        const int nv = ldc(rc, 1);
        uint32_t rj[16];
#pragma unroll
        for (int jj = 0; jj < 16; jj++) rj[jj] = (uint32_t)ldc(rc, 2 + jj);
        uint32_t prow = 0u;
#pragma unroll
        for (int jj = 0; jj < 16; jj++) prow = c16 == jj ? rj[jj] : prow;
        const bool pv = c16 < nv;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t qb = prow * RG_NB + (uint32_t)(bw + 4 * h);
#pragma unroll
            for (int s = 0; s < 8; s++)
                x.xb[h][s] = as_long(ld8(qs_b, pv ? qb * 256u + 64u * (s >> 1) + 32u * (s & 1) + 8u * g : OOB));
            x.bs0[h] = ld4(s32_b, pv ? qb * 32u + 4u * g : OOB);
            x.bs1[h] = ld4(s32_b, pv ? qb * 32u + 16u + 4u * g : OOB);
            x.xd[h] = ld4(d_b, pv ? qb * 4u : OOB);
        }
    };
    /* compute item j from its slot with operands x: the wave's two blocks of
     * its matrix, their sums to red */
    auto compute = [&](int j, const RgX &x) __attribute__((always_inline)) {
        const uint8_t *sb = &ring[j % RG_SLOTS][mw][0];
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int b = bw + 4 * h;
            const float *xdv = x.xdv[h];
            const Q4Hdr hr = q4_hdr(*(const u32x4 *)(sb + 16 * rg_unit(c16, 9 * b)));
            v4f im = {0.f, 0.f, 0.f, 0.f};
            im = __builtin_amdgcn_mfma_f32_16x16x4f32((float)(int)x.bs0[h], (float)byte_of(hr.mnl, g), im, 0, 0, 0);
            im = __builtin_amdgcn_mfma_f32_16x16x4f32((float)(int)x.bs1[h], (float)byte_of(hr.mnh, g), im, 0, 0, 0);
            int isc[4] = {0, 0, 0, 0};
#pragma unroll
            for (int jg = 0; jg < 4; jg++) {
                const u32x2 qq = *(const u32x2 *)(sb + 16 * rg_unit(c16, 9 * b + 1 + 2 * jg + (g >> 1)) + 8 * (g & 1));
                u32x2 lo, hi;
                lo.x = qq.x & 0x0F0F0F0Fu;
                lo.y = qq.y & 0x0F0F0F0Fu;
                hi.x = (qq.x >> 4) & 0x0F0F0F0Fu;
                hi.y = (qq.y >> 4) & 0x0F0F0F0Fu;
                const v4i dl = mma(x.xb[h][2 * jg], as_long(lo));
                const v4i dh = mma(x.xb[h][2 * jg + 1], as_long(hi));
                const uint32_t scw = jg < 2 ? hr.scl : hr.sch;
                const int s0 = byte_of(scw, 2 * (jg & 1)), s1 = byte_of(scw, 2 * (jg & 1) + 1);
#pragma unroll
                for (int v = 0; v < 4; v++) isc[v] += __mul24(s0, dl[v]) + __mul24(s1, dh[v]);
            }
#pragma unroll
            for (int v = 0; v < 4; v++) acc[v] += xdv[v] * (hr.d * (float)isc[v] - hr.dmin * im[v]);
        }
#pragma unroll
        for (int v = 0; v < 4; v++) red[j & 1][w][v][lane] = acc[v];
    };
    /* the finishing threads, RG_FO (pair, row) results each: the gate and
     * up waves' sums in wave order, the activation, the hidden values of item
     * j; the sums of pair 4 g + v and row c16 sit in lane 16 g + c16,
     * register v */
    auto finish = [&](int j, const Fin &fi) __attribute__((always_inline)) {
        const int s = fi.s, tp = fi.tp, p0 = fi.p0, np = fi.np;
        const float *gb = fi.gb, *ub = fi.ub;
#pragma unroll
        for (int o = tid - 64 * (RG_CW + RG_YW), u = 0; u < RG_FO; u++, o += 64 * RG_FW) {
            const int jj = o >> 4, rr = o & 15, ln = 16 * (jj >> 2) + rr, v = jj & 3;
            float gv = 0.f, uv = 0.f;
#pragma unroll
            for (int ww = 0; ww < 4; ww++) {
                gv += red[j & 1][ww][v][ln];
                uv += red[j & 1][4 + ww][v][ln];
            }
            const int r = 16 * s + rr;
            if (gb) gv += gb[r];
            if (ub) uv += ub[r];
            if (tp + jj < np) a.hidden[(size_t)(p0 + tp + jj) * a.I + r] = act_fn(a.act, gv, uv);
        }
    };
    /* a run: items of one expert and pass */
    auto run_end = [&](int s) { return min(ldc(a.rg_rend, (size_t)(i0 + s)), i0 + n) - i0; };

    /* The three roles run loops of their own (so the compiler's waits for
     * the compute waves' operand loads never land in the others' code),
     * meeting at one barrier an item.  Between the barriers of items i and
     * i + 1 the compute waves compute item i (reading slot i % 4, writing
     * red[i % 2]) while the copy waves copy item i + 3 into item i - 1's slot
     * and the finishing waves finish item i - 1 (reading red[(i - 1) % 2]):
     * each wave reaches the next barrier only after its part. */
    if (copier) {
        for (int j = 0; j < RG_SLOTS - 1 && j < n; j++) issue_copies(j, info_code(item(j)));
        Info fc = info_code(item(min(RG_SLOTS - 1, n - 1)));   /* item i + 3 */
        int code = item(min(RG_SLOTS, n - 1));                  /* item i + 4 */
        for (int i = 0; i < n; i++) {
            wait_copies_behind(min(RG_SLOTS - 2, n - 1 - i));
            /* a copy wave writes no LDS itself: its barrier leaves the scalar
             * reads of the next items' info in flight */
            asm volatile("s_barrier" ::: "memory");
            if (i + RG_SLOTS - 1 < n) issue_copies(i + RG_SLOTS - 1, fc);
            fc = info_code(code);
            code = item(min(i + RG_SLOTS + 1, n - 1));
        }
        asm volatile("s_barrier" ::: "memory");
        wait_copies();   /* no copy outlives the workgroup */
        return;
    }
    if (loader) {
        Fin ff = fin_head(item(0));                /* item i - 1, biases too */
        fin_bias(ff);
        Fin fh = fin_head(item(min(1, n - 1)));    /* item i */
        int code = item(min(2, n - 1));            /* item i + 1 */
        for (int i = 0; i < n; i++) {
            asm volatile("s_barrier" ::: "memory");   /* a finishing wave writes no LDS */
            if (i > 0) {
                finish(i - 1, ff);
                ff = fh;
                fin_bias(ff);
                fh = fin_head(code);
                code = item(min(i + 2, n - 1));
            }
        }
        asm volatile("s_barrier" ::: "memory");   /* item n - 1's sums are in LDS */
        finish(n - 1, ff);
        return;
    }
    /* A run's operands are loaded into a staging set while the run before is
     * computed, three items before its end (ahead of the copies of the next
     * run's first items, which they would otherwise wait behind), and taken
     * as the values of an empty asm statement when the run starts: the
     * compiler waits for the loads there and not at their uses, and the set
     * in use never has loads in flight. */
    auto settle = [&](RgX &x) __attribute__((always_inline)) {
#pragma unroll
        for (int h = 0; h < 2; h++)
            asm volatile(""
                         : "+v"(x.xb[h][0]), "+v"(x.xb[h][1]), "+v"(x.xb[h][2]), "+v"(x.xb[h][3]), "+v"(x.xb[h][4]),
                           "+v"(x.xb[h][5]), "+v"(x.xb[h][6]), "+v"(x.xb[h][7]), "+v"(x.bs0[h]), "+v"(x.bs1[h]),
                           "+v"(x.xd[h]));
    };
    /* the scale of each of the lane's four result pairs, shuffled once a run */
    auto prep = [&](RgX &x) __attribute__((always_inline)) {
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int v = 0; v < 4; v++) x.xdv[h][v] = __uint_as_float(__shfl(x.xd[h], 4 * g + v, 64));
    };
    RgX cur, stage;
    int run = ldc(a.rg_run0, blockIdx.x);   /* the run of item 0; the runs follow in order */
    load_x(run, cur);
    settle(cur);
    prep(cur);
    int re = run_end(0);
    for (int i = 0; i < n;) {
        const int pf = max(i, re - 3);
        for (; i < re; i++) {
            if (i == pf && re < n) load_x(run + 1, stage);
            bar_lds();   /* item i's slab has landed, item i - 1's sums are read */
            compute(i, cur);
        }
        if (i < n) {
            re = run_end(i);
            settle(stage);
            cur = stage;
            prep(cur);
            run++;
        }
    }
    bar_lds();   /* item n - 1's sums are in LDS */
}

/* Phase B: part[p][r] = w_p * (down_r . hq_p + bd[r]) for the 64 rows r of
 * slab blockIdx.x and every pair p of active expert a.ed[blockIdx.y]; Q6_K
 * down matrix of I = 256 nbi columns.  Wave w owns rows 16 w .. 16 w + 15 of
 * the slab over the whole row, so its MFMA sums are the rows' results and no
 * partial sums cross waves.  The slab's loads go out first, then the first
 * pass's q8 operands, then the slab is stored to LDS. */
constexpr int QB_ROWS = 64;                 /* rows of a down slab: one 16-row tile a wave */
constexpr int QB_PIECES = 13;               /* 16-byte pieces of a block's bytes 0-207 */
constexpr int QB_NPC = 10;                  /* pieces per thread in flight while the slab is staged */
constexpr int QB_CH = 6;                    /* half-blocks whose q8 operands a wave holds at once */
template <int>
__global__ __launch_bounds__(NT) void k_moe_qb(MoeArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const ExpDesc &ex = a.ed[blockIdx.y];
    const int e = ex.e, p0 = ex.p0, np = ex.np;
    const int nbi = a.I / 256, nhb = 2 * nbi;
    /* n / nbi for the slab's block indices n < 64 * 12 as (n * inv) >> 16:
     * inv exceeds 2^16 / nbi by less than 1, so the product's error stays
     * below 768 / 2^16 < 1 / nbi */
    const uint32_t inv = (65536u + (uint32_t)nbi - 1u) / (uint32_t)nbi;
    auto div_nbi = [&](int n) { return (int)(((uint32_t)n * inv) >> 16); };
    const uint32_t rb = (uint32_t)nbi * Q6B, rs = qb_row_stride(a.I);
    /* LDS offset of block blk of slab row row */
    auto blk_at = [&](int row, int blk) { return (uint32_t)row * rs + (uint32_t)blk * Q6S; };
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, g = lane >> 4,
              c16 = lane & 15;
    const int r0 = blockIdx.x * QB_ROWS;

    /* the slab, each block at a 224-byte stride: bytes 0-207 as 13 pieces,
     * then d at 208 (a load that ran past byte 209 would read zero in the
     * matrix's last block; rows past D read zero) */
    const Buf dw = make_buf_uniform((const void *)(uintptr_t)ex.down, (uint32_t)a.D * rb);
    const int nch = QB_ROWS * nbi * QB_PIECES;
    auto piece_src = [&](int c) {
        const int piece = c % QB_PIECES, rbk = c / QB_PIECES, row = div_nbi(rbk), blk = rbk - row * nbi;
        return (uint32_t)(r0 + row) * rb + (uint32_t)blk * Q6B + 16u * piece;
    };
    auto piece_dst = [&](int c) {
        const int rbk = c / QB_PIECES, row = div_nbi(rbk);
        return blk_at(row, rbk - row * nbi) + 16 * (c % QB_PIECES);
    };
    u32x4 pc[QB_NPC];
#pragma unroll
    for (int i = 0; i < QB_NPC; i++) {
        const int c = tid + NT * i;
        pc[i] = ld16(dw, c < nch ? piece_src(c) : OOB);
    }
    uint32_t dd[(QB_ROWS * 12 + NT - 1) / NT];   /* d of the slab's blocks (I <= 3072) */
#pragma unroll
    for (int i = 0; i < (QB_ROWS * 12 + NT - 1) / NT; i++) {
        const int rbk = tid + NT * i;
        const int row = div_nbi(rbk);
        dd[i] = rbk < QB_ROWS * nbi ? ld2(dw, (uint32_t)(r0 + row) * rb + (uint32_t)(rbk - row * nbi) * Q6B + 208u) : 0u;
    }

    const Q8Rows &q = a.hq;
    const Buf qs_b = make_buf(q.qs, (uint32_t)((size_t)a.P * nbi * 256));
    const Buf s16_b = make_buf(q.s16, (uint32_t)((size_t)a.P * nbi * 64));
    const Buf d_b = make_buf(q.d, (uint32_t)((size_t)a.P * nbi * 4));
    const Buf pw_b = make_buf(a.p_w, (uint32_t)a.P * 4u);
    const float *dbias = a.dbias ? (const float *)(uintptr_t)a.dbias[e] : nullptr;
    /* pair c16's q8 operands of half-blocks c0 .. c0 + QB_CH - 1: chunk m of
     * half h of block bi covers x[128 h + 32 m ...], this lane's K slice
     * 8 g .. 8 g + 7; the 16-value sums of sub-blocks 8 h + g and 8 h + 4 + g */
    long xb[QB_CH][4];
    int s16g[QB_CH][2];
    float xd[QB_CH];
    auto load_x = [&](uint32_t prow, bool pv, int c0) {
#pragma unroll
        for (int i = 0; i < QB_CH; i++) {
            const int hb = c0 + i;
            const bool v = pv && hb < nhb;
            const int bi = hb >> 1, h = hb & 1;
            const uint32_t qb = prow * (uint32_t)nbi + (uint32_t)bi;
#pragma unroll
            for (int m = 0; m < 4; m++)
                xb[i][m] = as_long(ld8(qs_b, v ? qb * 256u + 128u * h + 32u * m + 8u * g : OOB));
            /* each its own load: a select among loaded words would wait for the load */
            s16g[i][0] = (int)ld4(s16_b, v ? qb * 64u + 32u * h + 4u * g : OOB);
            s16g[i][1] = (int)ld4(s16_b, v ? qb * 64u + 32u * h + 16u + 4u * g : OOB);
            xd[i] = __uint_as_float(ld4(d_b, v ? qb * 4u : OOB));
        }
    };
    int t0 = 0;
    bool pv = c16 < np;
    uint32_t prow = (uint32_t)(pv ? p0 + c16 : 0);
    load_x(prow, pv, 0);
#pragma unroll
    for (int i = 0; i < QB_NPC; i++) {
        const int c = tid + NT * i;
        if (c < nch) *(u32x4 *)(lds + piece_dst(c)) = pc[i];
    }
    for (int c = tid + NT * QB_NPC; c < nch; c += NT)   /* rows of more than 3 blocks */
        *(u32x4 *)(lds + piece_dst(c)) = ld16(dw, piece_src(c));
#pragma unroll
    for (int i = 0; i < (QB_ROWS * 12 + NT - 1) / NT; i++) {
        const int rbk = tid + NT * i;
        const int row = div_nbi(rbk);
        if (rbk < QB_ROWS * nbi) *(uint32_t *)(lds + blk_at(row, rbk - row * nbi) + 208) = dd[i];
    }
    __syncthreads();

    const int tr = 16 * w;   /* the wave's first slab row */
    for (;;) {
        /* the weights of the lane's four pairs, waited for only at the end */
        float pwv[4];
#pragma unroll
        for (int v = 0; v < 4; v++)
            pwv[v] = __uint_as_float(ld4(pw_b, t0 + 4 * g + v < np ? (uint32_t)(p0 + t0 + 4 * g + v) * 4u : OOB));
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        for (int c0 = 0; c0 < nhb; c0 += QB_CH) {
            if (c0 > 0) load_x(prow, pv, c0);   /* rows of more than 3 blocks */
#pragma unroll
            for (int i = 0; i < QB_CH; i++) {
                const int hb = c0 + i;
                if (hb >= nhb) break;   /* uniform */
                const int bi = hb >> 1, h = hb & 1;
                /* row c16's codes: ql bytes 64 h + 32 (m & 1) + 8 g, qh bytes 32 h + 8 g */
                const uint8_t *ab = lds + blk_at(tr + c16, bi);
                const u32x2 ql0 = *(const u32x2 *)(ab + 64 * h + 8 * g);
                const u32x2 ql1 = *(const u32x2 *)(ab + 64 * h + 32 + 8 * g);
                const u32x2 qh = *(const u32x2 *)(ab + 128 + 32 * h + 8 * g);
                /* the pairs' q8 operands are the MFMA's A side and the weight
                 * rows its B side, so a lane's four sums belong to row c16
                 * and pairs 4 g + v: its scales are row c16's */
                const u32x2 scr = *(const u32x2 *)(ab + 192 + 8 * h);   /* sub-block scales 8 h .. 8 h + 7 */
                const float dv = ref_f16(*(const uint32_t *)(ab + 208) & 0xFFFFu);
                float xdv[4];
#pragma unroll
                for (int v = 0; v < 4; v++) xdv[v] = __shfl(xd[i], 4 * g + v, 64);
                /* the -32 offset terms sum_s s16[pair][s] sc[row][s] over the
                 * half's 8 sub-blocks: two f32 MFMAs of K = 4 (sub-blocks g
                 * and 4 + g; integers below 2^24, exact) */
                v4f cf = {0.f, 0.f, 0.f, 0.f};
                cf = __builtin_amdgcn_mfma_f32_16x16x4f32((float)s16g[i][0], (float)(int8_t)(scr.x >> (8 * g)), cf, 0,
                                                          0, 0);
                cf = __builtin_amdgcn_mfma_f32_16x16x4f32((float)s16g[i][1], (float)(int8_t)(scr.y >> (8 * g)), cf, 0,
                                                          0, 0);
                int ai[4] = {0, 0, 0, 0};
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    const u32x2 ql = (m & 1) ? ql1 : ql0;
                    const int sl = 4 * (m >> 1), sh = 2 * m;
                    u32x2 c;
                    c.x = ((ql.x >> sl) & 0x0F0F0F0Fu) | (((qh.x >> sh) & 0x03030303u) << 4);
                    c.y = ((ql.y >> sl) & 0x0F0F0F0Fu) | (((qh.y >> sh) & 0x03030303u) << 4);
                    /* K slots 0-15 (lane groups 0, 1) are sub-block 2 m, 16-31 sub-block 2 m + 1 */
                    const long x0 = g < 2 ? xb[i][m] : 0l, x1 = g < 2 ? 0l : xb[i][m];
                    const v4i d0 = mma(x0, as_long(c)), d1 = mma(x1, as_long(c));
                    const uint32_t sw = m < 2 ? scr.x : scr.y;
                    const int sc0 = (int)(int8_t)(sw >> (16 * (m & 1))), sc1 = (int)(int8_t)(sw >> (16 * (m & 1) + 8));
#pragma unroll
                    for (int v = 0; v < 4; v++) ai[v] += __mul24(sc0, d0[v]) + __mul24(sc1, d1[v]);   /* |.| < 2^24 */
                }
                /* sum (c - 32) x sc, exact in int32 */
#pragma unroll
                for (int v = 0; v < 4; v++) acc[v] += dv * xdv[v] * (float)(ai[v] - 32 * (int)cf[v]);
            }
        }
        /* row r0 + tr + c16 of pairs t0 + 4 g + v, in the half-blocks' order */
        const int r = r0 + tr + c16;
        if (r < a.D) {
            const float bias = dbias ? dbias[r] : 0.f;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int jj = t0 + 4 * g + v;
                if (jj < np) a.part[(size_t)(p0 + jj) * a.D + r] = pwv[v] * (acc[v] + bias);
            }
        }
        t0 += 16;
        if (t0 >= np) break;
        pv = t0 + c16 < np;
        prow = (uint32_t)(pv ? p0 + t0 + c16 : 0);
        load_x(prow, pv, 0);
    }
}

/* Phase B, persistent, for Q6_K down rows of I = 768 (3 blocks, 630 bytes
 * a row) without a down bias: one workgroup a compute unit walks its list
 * of items (active expert, 32-row slab, pass of 16 pairs), the slabs
 * (20,160 contiguous bytes) streaming through a ring of six LDS slots five
 * items ahead, as the gate/up ring does.  Twelve compute waves take one
 * 128-value half-block of one 16-row tile each (wave c: half-block c % 6,
 * block c % 6 / 2, tile c / 6; three a SIMD), with k_moe_qb's arithmetic,
 * and leave each
 * half-block's term d x d_x x (sum - 32 x offsets) in LDS.  Two copy waves
 * issue the slab copies and wait for them with exact counts (they issue no
 * other memory operation, which would enter the counts); two finishing
 * waves finish the previous item: the six terms added in half-block order
 * (k_moe_qb's order), times the pair's weight.  The slab
 * keeps the matrix's layout in LDS (the copies read 16-byte-aligned sources
 * only), so fields of odd rows and odd blocks lie at 2 mod 4 and are read
 * as covering dwords, shifted. */
constexpr int DR_NB = 3;                                  /* Q6_K blocks of a 768-value row */
constexpr int DR_RB = DR_NB * (int)Q6B;                   /* 630 bytes a row */
constexpr int DR_ROWS = 32;
constexpr int DR_SLAB = DR_ROWS * DR_RB;                  /* 20,160 bytes */
constexpr int DR_COPIES = (DR_SLAB + 1023) / 1024;        /* 20 copies, the last of DR_LAST lanes */
constexpr int DR_LAST = (DR_SLAB - 1024 * (DR_COPIES - 1)) / 16;
constexpr int DR_SLOTS = 6;
constexpr int DR_HB = 2 * DR_NB;                        /* half-blocks of a row */
constexpr int DR_CW = 2 * DR_HB, DR_YW = 2, DR_FW = 2;  /* compute, copy and finishing waves */
constexpr int DR_LC = DR_COPIES / DR_YW;                  /* copies a copy wave issues per item */
constexpr int DR_NT = 64 * (DR_CW + DR_YW + DR_FW);
constexpr int DR_FO = 2 * 16 * 16 / (64 * DR_FW);         /* (pair, row) results a finishing thread writes */
static_assert(DR_SLAB % 16 == 0 && DR_LAST > 0 && DR_LAST <= 64, "whole 16-byte pieces");
static_assert(DR_COPIES % DR_YW == 0, "equal copy counts per copy wave");
static_assert((DR_SLOTS - 2) * DR_LC <= 63, "a vmcnt count");

/* 8 bytes at LDS offset o (o even) of base: the covering dwords, shifted */
__device__ inline u32x2 dr_ld8(const uint8_t *base, uint32_t o) {
    const uint32_t *p = (const uint32_t *)(base + (o & ~3u));
    const uint32_t sh = o & 3u;
    const uint32_t d0 = p[0], d1 = p[1], d2 = p[2];
    return u32x2{__builtin_amdgcn_alignbyte(d1, d0, sh), __builtin_amdgcn_alignbyte(d2, d1, sh)};
}

struct DrX {   /* a compute lane's q8 operands of one run: pair c16, its wave's half-block */
    long x0[4], x1[4];   /* K slice 8 g of chunk m, zero in the half of K the other sub-block takes */
    float s16a, s16b, xd;
    float xdv[4];        /* the scales of pairs 4 g .. 4 g + 3, set once the run starts */
};

__global__ __launch_bounds__(DR_NT) void k_moe_qb_ring(MoeArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t ring[DR_SLOTS][DR_SLAB];
    __shared__ __attribute__((aligned(16))) float red[2][DR_HB][2][4][64];   /* by item parity */
    __shared__ float pwl[DR_FW][16];                                          /* a finishing wave's pair weights */
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, g = lane >> 4,
              c16 = lane & 15;
    const bool loader = w >= DR_CW, copier = loader && w < DR_CW + DR_YW;
    const int i0 = ldc(a.rb_off, blockIdx.x), n = ldc(a.rb_off, blockIdx.x + 1) - i0;
    if (n <= 0) return;   /* uniform */
    const uint32_t mbytes = (uint32_t)a.D * DR_RB;
    const Q8Rows &q = a.hq;
    const Buf qs_b = make_buf(q.qs, (uint32_t)((size_t)a.P * DR_NB * 256));
    const Buf s16_b = make_buf(q.s16, (uint32_t)((size_t)a.P * DR_NB * 64));
    const Buf d_b = make_buf(q.d, (uint32_t)((size_t)a.P * DR_NB * 4));
    const int hbw = w % DR_HB, bi = hbw >> 1, h = hbw & 1, tw = w / DR_HB;   /* a compute wave's half-block, tile */

    auto item = [&](int j) { return ldc(a.rb_items, (size_t)(i0 + j)); };
    /* What the copy and finishing waves need of an item comes through the
     * scalar path in stages, each from loads issued an item earlier: an item
     * code, then its expert's table entries, then the pair weights.  A chain
     * of dependent scalar loads in one item's step would stall the wave for
     * each load's round trip (about a microsecond under the weight stream)
     * and the barrier with it. */
    struct Info {   /* a copy wave's: the matrix and slab */
        uint64_t base;
        int s;
    };
    auto info_code = [&](int it) __attribute__((always_inline)) {
        Info f;
        f.base = ldc(&a.ed[it >> 16].down, 0);
        f.s = (it >> 8) & 255;
        return f;
    };
    struct Fin {   /* a finishing wave's: slab, pairs and their weights */
        int s, tp, p0, np;
        float pw[16];
    };
    auto fin_head = [&](int it) __attribute__((always_inline)) {
        Fin f;
        f.s = (it >> 8) & 255;
        f.tp = 16 * (it & 255);
        f.p0 = ldc(&a.ed[it >> 16].p0, 0);
        f.np = ldc(&a.ed[it >> 16].np, 0);
        return f;
    };
    auto fin_pw = [&](Fin &f) __attribute__((always_inline)) {
#pragma unroll
        for (int v = 0; v < 16; v++) f.pw[v] = ldc(a.p_w, (size_t)min(f.p0 + f.tp + v, a.P - 1));
    };
    /* the copy wave's share of item j's copies */
    auto issue_copies = [&](int j, const Info &f) __attribute__((always_inline)) {
        const u32x4 desc = buf_desc((const void *)(uintptr_t)f.base, mbytes);
        uint8_t *dst = &ring[j % DR_SLOTS][0];
        const uint32_t src = (uint32_t)f.s * DR_SLAB + 16u * (uint32_t)lane;
#pragma unroll
        for (int kk = 0; kk < DR_LC; kk++) {
            const int k = DR_LC * (w - DR_CW) + kk;
            if (k < DR_COPIES - 1 || lane < DR_LAST) copy_lanes_nt(desc, src + 1024u * k, lds_addr(dst + 1024 * k));
        }
    };
    auto wait_copies_behind = [&](int k) __attribute__((always_inline)) {
        if (k >= 4) wait_copies_but<4 * DR_LC>();
        else if (k == 3) wait_copies_but<3 * DR_LC>();
        else if (k == 2) wait_copies_but<2 * DR_LC>();
        else if (k == 1) wait_copies_but<DR_LC>();
        else wait_copies_but<0>();
    };
    static_assert(DR_SLOTS - 2 == 4, "wait_copies_behind covers the items in flight");
    /* the compute lane's operands of run r: its pair c16 (the run's first
     * pair and count from its record, one round trip of scalar loads) */
    auto load_x = [&](int r, DrX &x) __attribute__((always_inline)) {
        const int *rc = a.rb_runs + (size_t)RING_REC * r;
        const int pf = ldc(rc, 0), nv = ldc(rc, 1);
        const bool pv = c16 < nv;
        const uint32_t qb = (uint32_t)(pf + c16) * DR_NB + (uint32_t)bi;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const long xb = as_long(ld8(qs_b, pv ? qb * 256u + 128u * h + 32u * m + 8u * g : OOB));
            x.x0[m] = g < 2 ? xb : 0l;
            x.x1[m] = g < 2 ? 0l : xb;
        }
        x.s16a = (float)(int)ld4(s16_b, pv ? qb * 64u + 32u * h + 4u * g : OOB);
        x.s16b = (float)(int)ld4(s16_b, pv ? qb * 64u + 32u * h + 16u + 4u * g : OOB);
        x.xd = __uint_as_float(ld4(d_b, pv ? qb * 4u : OOB));
    };
    /* compute item j from its slot: the wave's half-block of its tile */
    auto compute = [&](int j, const DrX &x) __attribute__((always_inline)) {
        const uint8_t *sb = &ring[j % DR_SLOTS][0];
        const float *xdv = x.xdv;
        {
            const int tq = tw;
            const uint32_t rb = (uint32_t)(16 * tq + c16) * DR_RB + (uint32_t)bi * Q6B;   /* row c16's block */
            const u32x2 ql0 = dr_ld8(sb, rb + 64u * h + 8u * g);
            const u32x2 ql1 = dr_ld8(sb, rb + 64u * h + 32u + 8u * g);
            const u32x2 qh = dr_ld8(sb, rb + 128u + 32u * h + 8u * g);
            const u32x2 scr = dr_ld8(sb, rb + 192u + 8u * h);
            const uint32_t dw = *(const uint32_t *)(sb + ((rb + 208u) & ~3u));
            const float dv = ref_f16((rb & 2u) ? (dw >> 16) : (dw & 0xFFFFu));
            v4f cf = {0.f, 0.f, 0.f, 0.f};
            cf = __builtin_amdgcn_mfma_f32_16x16x4f32(x.s16a, (float)(int8_t)(scr.x >> (8 * g)), cf, 0, 0, 0);
            cf = __builtin_amdgcn_mfma_f32_16x16x4f32(x.s16b, (float)(int8_t)(scr.y >> (8 * g)), cf, 0, 0, 0);
            int ai[4] = {0, 0, 0, 0};
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const u32x2 ql = (m & 1) ? ql1 : ql0;
                const int sl = 4 * (m >> 1), sh = 2 * m;
                u32x2 c;
                c.x = ((ql.x >> sl) & 0x0F0F0F0Fu) | (((qh.x >> sh) & 0x03030303u) << 4);
                c.y = ((ql.y >> sl) & 0x0F0F0F0Fu) | (((qh.y >> sh) & 0x03030303u) << 4);
                const v4i d0 = mma(x.x0[m], as_long(c)), d1 = mma(x.x1[m], as_long(c));
                const uint32_t sw = m < 2 ? scr.x : scr.y;
                const int sc0 = (int)(int8_t)(sw >> (16 * (m & 1))), sc1 = (int)(int8_t)(sw >> (16 * (m & 1) + 8));
#pragma unroll
                for (int v = 0; v < 4; v++) ai[v] += __mul24(sc0, d0[v]) + __mul24(sc1, d1[v]);   /* |.| < 2^24 */
            }
#pragma unroll
            for (int v = 0; v < 4; v++) red[j & 1][hbw][tq][v][lane] = dv * xdv[v] * (float)(ai[v] - 32 * (int)cf[v]);
        }
    };
    /* the finishing threads, DR_FO (pair, row) results each: the six
     * half-block terms in order, times the pair's weight; the term of pair
     * 4 g + v and row c16 of tile tq sits in lane 16 g + c16, register v */
    auto finish = [&](int j, const Fin &fi) __attribute__((always_inline)) {
        /* the weights (scalars) through the wave's own LDS words: a per-lane
         * select among them became a lookup through scratch memory */
        float *pl = pwl[w - DR_CW - DR_YW];
        if (lane == 0) {
#pragma unroll
            for (int v = 0; v < 16; v++) pl[v] = fi.pw[v];
        }
        const int f = tid - 64 * (DR_CW + DR_YW);
#pragma unroll
        for (int u = 0; u < DR_FO; u++) {
            const int o = f + 64 * DR_FW * u, tq = o >> 8, jj = (o >> 4) & 15, rr = o & 15;
            const int ln = 16 * (jj >> 2) + rr, v = jj & 3;
            if (fi.tp + jj < fi.np) {
                float acc = 0.f;
#pragma unroll
                for (int c = 0; c < DR_HB; c++) acc += red[j & 1][c][tq][v][ln];
                const int r = DR_ROWS * fi.s + 16 * tq + rr;
                a.part[(size_t)(fi.p0 + fi.tp + jj) * a.D + r] = pl[jj] * (acc + 0.f);
            }
        }
    };
    auto run_end = [&](int s0) { return min(ldc(a.rb_rend, (size_t)(i0 + s0)), i0 + n) - i0; };

    /* as in the gate/up ring: between the barriers of items i and i + 1 the
     * compute waves compute item i (slot i % DR_SLOTS, red[i % 2]) while the
     * copy waves copy item i + DR_SLOTS - 1 into item i - 1's slot and the
     * finishing waves finish item i - 1 (red[(i - 1) % 2]) */
    if (copier) {
        for (int j = 0; j < DR_SLOTS - 1 && j < n; j++) issue_copies(j, info_code(item(j)));
        Info fc = info_code(item(min(DR_SLOTS - 1, n - 1)));   /* item i + DR_SLOTS - 1 */
        int code = item(min(DR_SLOTS, n - 1));                  /* item i + DR_SLOTS */
        for (int i = 0; i < n; i++) {
            wait_copies_behind(min(DR_SLOTS - 2, n - 1 - i));
            asm volatile("s_barrier" ::: "memory");   /* a copy wave writes no LDS itself */
            if (i + DR_SLOTS - 1 < n) issue_copies(i + DR_SLOTS - 1, fc);
            fc = info_code(code);
            code = item(min(i + DR_SLOTS + 1, n - 1));
        }
        asm volatile("s_barrier" ::: "memory");
        wait_copies();   /* no copy outlives the workgroup */
        return;
    }
    if (loader) {
        Fin ff = fin_head(item(0));                /* item i - 1, weights too */
        fin_pw(ff);
        Fin fh = fin_head(item(min(1, n - 1)));    /* item i */
        int code = item(min(2, n - 1));            /* item i + 1 */
        for (int i = 0; i < n; i++) {
            bar_lds();   /* its own weight words are written and read in order */
            if (i > 0) {
                finish(i - 1, ff);
                ff = fh;
                fin_pw(ff);
                fh = fin_head(code);
                code = item(min(i + 2, n - 1));
            }
        }
        bar_lds();   /* item n - 1's terms are in LDS */
        finish(n - 1, ff);
        return;
    }
    auto settle = [&](DrX &x) __attribute__((always_inline)) {
        asm volatile(""
                     : "+v"(x.x0[0]), "+v"(x.x0[1]), "+v"(x.x0[2]), "+v"(x.x0[3]), "+v"(x.x1[0]), "+v"(x.x1[1]),
                       "+v"(x.x1[2]), "+v"(x.x1[3]), "+v"(x.s16a), "+v"(x.s16b), "+v"(x.xd));
    };
    auto prep = [&](DrX &x) __attribute__((always_inline)) {
#pragma unroll
        for (int v = 0; v < 4; v++) x.xdv[v] = __shfl(x.xd, 4 * g + v, 64);
    };
    DrX cur, stage;
    int run = ldc(a.rb_run0, blockIdx.x);   /* the run of item 0; the runs follow in order */
    load_x(run, cur);
    settle(cur);
    prep(cur);
    int re = run_end(0);
    for (int i = 0; i < n;) {
        const int pf = max(i, re - (DR_SLOTS - 1));
        for (; i < re; i++) {
            if (i == pf && re < n) load_x(run + 1, stage);
            bar_lds();   /* item i's slab has landed, item i - 1's terms are read */
            compute(i, cur);
        }
        if (i < n) {
            re = run_end(i);
            settle(stage);
            cur = stage;
            prep(cur);
            run++;
        }
    }
    bar_lds();   /* item n - 1's terms are in LDS */
}

bool qb_ring_shape(int I, int D) { return I == DR_NB * 256 && D % DR_ROWS == 0 && D / DR_ROWS <= 256; }

/* The MFMA phases need Q4_K gate/up and Q6_K down matrices of whole blocks,
 * slabs within the device's LDS, and 31-bit buffer ranges. */
bool qk_grouped_fits(const MoeArgs &a) {
    static int max_lds = -1;
    if (max_lds < 0) {
        int dev = 0;
        max_lds = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
            max_lds = 0;
    }
    if (a.gate_fmt != TG_FMT_Q4K || a.D % 256 || a.I % 256 || a.n_act_a <= 0) return false;
    if (a.D > 256 * NW * QA_WB_MAX || a.I > 3072) return false;   /* a pass's operands and the slab's d in registers */
    const uint64_t lim = 1ull << 31;
    return qa_lds_bytes(a.D) <= (size_t)max_lds && qb_lds_bytes(a.I) <= (size_t)max_lds &&
           (uint64_t)a.I * (a.D / 256) * Q4B < lim && (uint64_t)a.D * (a.I / 256) * Q6B < lim &&
           (uint64_t)a.P * a.I < lim && (uint64_t)a.k * a.D < lim && (uint64_t)a.P * (a.I / 256) * 64 < lim;
}

bool qa_ring_shape(int gate_fmt, int D, int I) { return gate_fmt == TG_FMT_Q4K && D == 256 * RG_NB && I % 16 == 0 && I <= 4096; }

/* Items in the order expert (busiest first), pass, slab, cut into G
 * contiguous stretches of equal length: each workgroup's stretch is a few
 * runs of one (expert, pass), and the passes of an expert run at about the
 * same time on neighbouring workgroups, so their slabs' second reads come
 * from the caches.  rend[i] is the end of item i's run (the items of its
 * expert and pass): a workgroup finds where its run ends with one load, not
 * by scanning the items that follow.  runs holds each run's record (first
 * pair, pair count, the input rows of its first 16 pairs) in list order and
 * run0[w] the run of workgroup w's first item, so a compute wave reaches a
 * run's operands with one round trip of scalar loads. */
void ring_items(const ExpDesc *ed, int n_act, int slabs, int G, const int *p_row, int P, RingLists &r) {
    r.items.clear();
    r.rend.clear();
    r.runs.clear();
    std::vector<int> run_of;
    for (int ei = 0; ei < n_act; ei++)
        for (int t = 0; t < std::max(1, (ed[ei].np + 15) / 16); t++) {
            const int run = (int)(r.runs.size() / RING_REC), pf = ed[ei].p0 + 16 * t;
            r.runs.push_back(pf);
            r.runs.push_back(ed[ei].np - 16 * t);
            for (int j = 0; j < 16; j++) r.runs.push_back(p_row[std::min(pf + j, P - 1)]);
            r.runs.resize((size_t)(run + 1) * RING_REC, 0);
            for (int s = 0; s < slabs; s++) r.items.push_back(ei << 16 | s << 8 | t);
            r.rend.resize(r.items.size(), (int)r.items.size());
            run_of.resize(r.items.size(), run);
        }
    r.off.resize(G + 1);
    r.run0.resize(G + 1);
    for (int w = 0; w <= G; w++) {
        r.off[w] = (int)((int64_t)r.items.size() * w / G);
        r.run0[w] = r.off[w] < (int)run_of.size() ? run_of[r.off[w]] : 0;
    }
}

void launch_moe_a_qk(const MoeArgs &a, hipStream_t st) {
    if (a.rg_items && qa_ring_shape(a.gate_fmt, a.D, a.I)) {
        hipLaunchKernelGGL(k_moe_qa_ring, dim3(a.rg_n), dim3(RG_NT), 0, st, a);
        return;
    }
    const dim3 grid((a.I + 15) / 16, a.n_act_a);
    if (a.D <= 256 * NW * 2) hipLaunchKernelGGL(k_moe_qa<2>, grid, dim3(NT), qa_lds_bytes(a.D), st, a);
    else hipLaunchKernelGGL(k_moe_qa<QA_WB_MAX>, grid, dim3(NT), qa_lds_bytes(a.D), st, a);
}

void launch_moe_b_qk(const MoeArgs &a, hipStream_t st) {
    if (a.rb_items && !a.dbias && qb_ring_shape(a.I, a.D)) {
        hipLaunchKernelGGL(k_moe_qb_ring, dim3(a.rb_n), dim3(DR_NT), 0, st, a);
        return;
    }
    hipLaunchKernelGGL(k_moe_qb<0>, dim3((a.D + QB_ROWS - 1) / QB_ROWS, a.n_act_a), dim3(NT), qb_lds_bytes(a.I), st,
                       a);
}

}  // namespace tg
