/*
 * tg_decode.hip -- persistent single-launch expert decode step for one token.
 *
 * One cooperative launch runs every layer of the step
 *     h <- h + sum_e w_e * down_e( q8( act(gate_e . q8(RMSNorm h), up_e . q8(RMSNorm h)) ) )
 * (tinygiant/engine.py:281-282,335-341 per layer; the expert math is
 * moe_phase_a / moe_phase_b of csrc/libtinygiant.c:1279-1384 for k = 1).
 *
 * Placement.  One workgroup per CU, 256 workgroups; the dispatcher places
 * workgroup g on XCD g % 8, so workgroup g = x + 8 j is rank j (of 32) on
 * XCD x.  XCD x owns the layer's x-th active expert: its 32 workgroups split
 * that expert's gate/up rows (24 each) and down rows (64 each), so the
 * hidden vector an expert produces never leaves its XCD.  Per layer:
 *   1  gather h: the 32 ranks of an XCD all-gather their 64-row slices of h
 *   2  RMSNorm + q8 of h, in LDS, on every workgroup (8 blocks, one per wave)
 *   3  gate/up rows of the workgroup's expert -> SwiGLU -> 24 hidden values
 *   4  the XCD all-gathers its expert's 768 hidden values
 *   5  q8 of the hidden vector (3 blocks)
 *   6  down rows [64 j, 64 j + 64) of the expert
 *   7  cross-XCD hop: rank j of every XCD exchanges its 64 down values, so
 *      each holds all 8 experts' outputs for rows [64 j, 64 j + 64)
 *   8  h[r] += w_e * out_e[r] in expert order (the reference's combine order,
 *      csrc/libtinygiant.c:1428-1434); all 8 XCDs compute the same bits for
 *      the slice and publish it for step 1 of the next layer.
 * Only step 7 crosses XCDs; the placement the intra-XCD exchanges rely on
 * is recorded by every launch (HW_REG_XCC_ID of each workgroup) for the host
 * to check, and a launch with pol = 1 stores every slot device-coherently,
 * which is correct wherever the workgroups run.
 *
 * Weights stream through LDS.  A CU returns the data of its vector loads in
 * the order it issued them, so an exchange poll waits behind every weight
 * load its CU issued before it.  The weights are therefore copied into LDS
 * by direct-to-LDS loads (no registers) in four batches per layer, each
 * issued right after an exchange or a phase that frees its region, and
 * needed only after a later exchange:
 *   D  this layer's down rows            at the start of RMSNorm (every wave)
 *   N  the next layer's RMSNorm weight   at the start of gate/up (the
 *                                        communication waves, idle there)
 *   A  the first 24 KiB of the next      at the start of q8(hidden) (every
 *      layer's gate/up rows              wave)
 *   B  the rest of its gate/up rows      at the start of the down dots (the
 *                                        communication waves)
 * so the exchange polls wait for little that is not needed anyway, and the
 * weight stream runs while the chain of exchanges and dots runs (an issuing
 * wave stalls once its CU's memory queue is full, so each batch is spread
 * over waves that have time).  Each lane then reads its Q4_K block
 * (gate/up) or Q6_K half-block (down) from LDS.
 *
 * Down matrices arrive in a row-group layout made once when the step is
 * created (tg_api.hip): every 8 rows' Q6_K blocks become field-major
 * {ql[24][128] | qh[24][64] | sc[24][16] | d[24]} (5040 bytes, the same
 * bytes), so every field a lane reads is aligned in LDS.
 *
 * Exchanges use epoch-tagged 16-byte slots {tag, v0, v1, v2}, written and
 * polled as one vector access so the tag and its values arrive together.
 * Two communication waves per workgroup publish; the two intra-XCD gathers
 * are polled by all eight waves (one or two slots a lane, so a round is one
 * load latency), the cross-XCD hop by the communication waves alone.
 * Every wait is bounded; a timed-out wait raises an abort flag that
 * releases every other waiter, so the grid always drains.
 */
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "tg_common.h"
#include "tg_decode.h"
#include "tg_device.hpp"
#include "tg_xchg.hpp"

namespace tg {

namespace {

constexpr int NW = 6;                 /* compute waves per workgroup */
constexpr int NC = 2;                 /* communication waves per workgroup */
constexpr int NA = NW + NC;           /* all waves (RMSNorm / q8 use every wave) */
constexpr int NT = NA * 64;
constexpr int CL = NC * 64;           /* communication lanes */
constexpr int D = 2048, I = 768;      /* Qwen3-30B-A3B expert shape */
constexpr int NBD = D / 256, NBI = I / 256;
constexpr int GATE_RB = NBD * 144;    /* Q4_K row of D values */
constexpr int DOWN_RB = NBI * 210;    /* Q6_K row of I values */
constexpr int NE = DECODE_MAXE;       /* active experts per layer (top-8 at k = 1) */
constexpr int NWG = DECODE_GRID;      /* workgroups: one per CU */
constexpr int NX = 8;                 /* XCDs; workgroup g runs on XCD g % NX */
constexpr int NR = NWG / NX;          /* ranks (workgroups) per XCD */
constexpr int RA = I / NR;            /* gate/up rows per workgroup: 24 */
constexpr int RB = D / NR;            /* down rows (and h rows) per workgroup: 64 */
constexpr int HB = 2 * NBI;           /* Q6_K half-blocks per down row: 6 */
constexpr int XST = 272;              /* LDS stride of a q8(x) 256-block (bank-conflict padding) */
constexpr int HST = 144;              /* LDS stride of a q8(hidden) 128-value half-block */
constexpr int VPS = 3;                /* values per slot */
constexpr int GS = RA / VPS;          /* hidden slots per workgroup: 8 */
constexpr int PS = (RB + VPS - 1) / VPS;   /* slots per 64-row slice: 22 */
constexpr int MAX_LAYERS = 64;        /* layer descriptors staged in LDS */
constexpr int NTS = 24;               /* timing words per layer */
/* LDS weight regions and their direct-to-LDS copies (1 KiB an instruction) */
constexpr int SEG = RA * GATE_RB;     /* one matrix's 24-row slice: 27,648 bytes */
constexpr int WGB = 2 * SEG;          /* gate rows, then up rows */
constexpr int G_INS = WGB / 1024;     /* 54 */
constexpr int DGRP = 8 * DOWN_RB;     /* one 8-row group of the row-group layout: 5040 bytes */
constexpr int WDB = RB / 8 * DGRP;    /* the 64-row down slice: 40,320 bytes */
constexpr int D_INS = (WDB + 1023) / 1024;   /* 40 (the last one runs past the slice) */
constexpr int N_INS = D * 4 / 1024;   /* RMSNorm weight: 8 */
#ifndef TG_DECODE_G_SPLIT
#define TG_DECODE_G_SPLIT 24
#endif
#ifndef TG_DECODE_B_AT_DOWN
#define TG_DECODE_B_AT_DOWN 1
#endif
/* Copy batches (each wave issues its share; a wave that issues more than
 * its CU's memory queue takes stalls until the queue drains):
 *   D  this layer's down rows     every wave, at the start of RMSNorm
 *      (after the h gather)       (done before the hidden gather ends)
 *   N  the next layer's RMSNorm   the communication waves, at the start of
 *      weight (8 KiB)             gate/up (the region is free after RMSNorm;
 *                                 done before the hidden gather ends)
 *   A  the first G_SPLIT gate/up  every wave, at the start of q8(hidden)
 *      KiB of the next layer      (after the hidden gather)
 *   B  the other gate/up KiB      the communication waves at the start of
 *                                 the down dots (they are idle there), or
 *                                 every wave after the hop
 * A and B are done before the next h gather ends.  The copies that drain
 * between the hidden gather and the hop (A, B) set how long the hop's polls
 * wait, so N moves what it can into the gap before the hidden gather. */
constexpr int G_SPLIT = TG_DECODE_G_SPLIT;
constexpr bool B_AT_DOWN = TG_DECODE_B_AT_DOWN != 0;

static_assert(NE == NX, "one expert per XCD");
static_assert(NR * RA == I && NR * RB == D && RA % VPS == 0, "row split");
static_assert(2 * RA * NBD == NW * 64, "gate/up: one Q4_K block per compute lane");
static_assert(RB * HB == NW * 64, "down: one Q6_K half-block per compute lane");
static_assert((NR - 1) * PS <= 6 * CL && (NR - 1) * GS <= 2 * CL && (NX - 1) * PS <= 2 * CL, "poll shares");
static_assert(NBI <= NA && NBD == NA, "q8 blocks per wave");
static_assert(RB == VPS * (PS - 1) + 1, "the last slice slot holds one row and the slice's sum of h^2");
static_assert(NR % NA == 0, "layer-0 slice sums: whole slices per wave");
static_assert(WGB % 1024 == 0 && SEG % 1024 == 0 && DGRP % 16 == 0 && RB % 8 == 0, "copy granules");
static_assert(G_SPLIT <= G_INS, "copy split");
static_assert(G_SPLIT <= G_INS, "batch split");

/* Slot policies: slots read only inside the writer's XCD are stored plainly
 * (the line stays in that XCD's L2) and loaded with sc1, which bypasses the
 * CU's L1 and reads the L2 line; cross-XCD slots are stored with sc1 (write
 * through to memory) and loaded with sc1 (no stale line from the reader's
 * L2).  With pol = 1 every slot is stored with sc1. */
/* slot regions (u32x4 index), each double buffered by layer parity:
 *   h slices  [2][NWG][PS]   rows [64 j, 64 j + 64) of the layer output
 *   hidden    [2][NWG][GS]   the workgroup's 24 hidden values
 *   partials  [2][NWG][PS]   the workgroup's 64 down values (unweighted) */
constexpr uint32_t HSL = 0, GSL = 2u * NWG * PS, PSL = GSL + 2u * NWG * GS, NSLOTS = PSL + 2u * NWG * PS;

/* ---- LDS images of q8 rows (blocks padded so the lanes of a wave reading
 * different blocks hit different banks) ---- */
struct __attribute__((aligned(16))) LdsX {   /* q8(RMSNorm(h)) : D values, block b at b * XST */
    int8_t qs[NBD * XST];
    float d[NBD];
    int32_t s32[NBD * 8];
};
struct __attribute__((aligned(16))) LdsH {   /* q8(hidden) of this XCD's expert : I values, */
    int8_t qs[HB * HST];                     /* half-block hb = 2 b + h at hb * HST */
    float d[NBI];
    int32_t s16[NBI * 16];
};

/* One lane's Q4_K block (144 bytes: d, dmin, scales[12], qs[128]). */
struct Q4Blk {
    u32x4 w[9];
};
__device__ inline Q4Blk lds_q4blk(const uint8_t *p) {
    Q4Blk r;
#pragma unroll
    for (int i = 0; i < 9; i++) r.w[i] = *reinterpret_cast<const u32x4 *>(p + 16 * i);
    return r;
}
/* dot_q4k_q8 of one block (csrc/libtinygiant.c:223-272): integer sums per
 * 32-value sub-block are exact; per group g the float combine is
 * d*(sc_lo*lo + sc_hi*hi) - dmin*(m_lo*bs_lo + m_hi*bs_hi) (both brackets
 * below 2^24), scaled by the q8 block scale.  Scales and mins are the
 * get_scale_min_k4 unpack (:146-155) done four bytes at a time. */
__device__ inline float dot_q4blk(const Q4Blk &q, const int8_t *xq, const int32_t *s32, float xd) {
    const uint32_t m4 = 0x0F0F0F0Fu;
    const float d = ref_f16(q.w[0].x & 0xFFFFu), dmin = ref_f16(q.w[0].x >> 16);
    const uint32_t s0 = q.w[0].y, s1 = q.w[0].z, s2 = q.w[0].w;
    const uint32_t scl = s0 & 0x3F3F3F3Fu, mnl = s1 & 0x3F3F3F3Fu;
    const uint32_t sch = (s2 & m4) | ((s0 >> 2) & 0x30303030u);
    const uint32_t mnh = ((s2 >> 4) & m4) | ((s1 >> 2) & 0x30303030u);
    const u32x4 bs0 = *reinterpret_cast<const u32x4 *>(s32), bs1 = *reinterpret_cast<const u32x4 *>(s32 + 4);
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const u32x4 *xp = reinterpret_cast<const u32x4 *>(xq + 64 * g);
        const u32x4 xa0 = xp[0], xa1 = xp[1], xb0 = xp[2], xb1 = xp[3];
        const u32x4 qa = q.w[1 + 2 * g], qb = q.w[2 + 2 * g];
        int lo = 0, hi = 0;
        lo = dot4(qa.x & m4, xa0.x, lo); lo = dot4(qa.y & m4, xa0.y, lo);
        lo = dot4(qa.z & m4, xa0.z, lo); lo = dot4(qa.w & m4, xa0.w, lo);
        lo = dot4(qb.x & m4, xa1.x, lo); lo = dot4(qb.y & m4, xa1.y, lo);
        lo = dot4(qb.z & m4, xa1.z, lo); lo = dot4(qb.w & m4, xa1.w, lo);
        hi = dot4((qa.x >> 4) & m4, xb0.x, hi); hi = dot4((qa.y >> 4) & m4, xb0.y, hi);
        hi = dot4((qa.z >> 4) & m4, xb0.z, hi); hi = dot4((qa.w >> 4) & m4, xb0.w, hi);
        hi = dot4((qb.x >> 4) & m4, xb1.x, hi); hi = dot4((qb.y >> 4) & m4, xb1.y, hi);
        hi = dot4((qb.z >> 4) & m4, xb1.z, hi); hi = dot4((qb.w >> 4) & m4, xb1.w, hi);
        const uint32_t scw = g < 2 ? scl : sch, mnw = g < 2 ? mnl : mnh;
        const int sh0 = 16 * (g & 1);
        const int sc_lo = (int)((scw >> sh0) & 0xFFu), sc_hi = (int)((scw >> (sh0 + 8)) & 0xFFu);
        const int m_lo = (int)((mnw >> sh0) & 0xFFu), m_hi = (int)((mnw >> (sh0 + 8)) & 0xFFu);
        const int bs_lo = (int)(g < 2 ? (g == 0 ? bs0.x : bs0.z) : (g == 2 ? bs1.x : bs1.z));
        const int bs_hi = (int)(g < 2 ? (g == 0 ? bs0.y : bs0.w) : (g == 2 ? bs1.y : bs1.w));
        /* |sums| < 2^23 and scales < 2^6: 24-bit multiplies are exact */
        acc += d * (float)(__mul24(sc_lo, lo) + __mul24(sc_hi, hi)) -
               dmin * (float)(__mul24(m_lo, bs_lo) + __mul24(m_hi, bs_hi));
    }
    return xd * acc;
}

/* One lane's half of a Q6_K block: 64 bytes of ql, 32 of qh, 8 int8
 * sub-scales and the f16 d (low 16 bits). */
struct Q6Half {
    u32x4 la0, la1, lb0, lb1, h0, h1;
    u32x2 sc;
    uint32_t d;
};
/* Half h of block j (0..23) of an 8-row group in the row-group layout. */
__device__ inline Q6Half lds_q6half(const uint8_t *grp, int j, int h) {
    Q6Half r;
    const uint8_t *ql = grp + 128 * j + 64 * h;
    const uint8_t *qh = grp + 24 * 128 + 64 * j + 32 * h;
    r.la0 = *reinterpret_cast<const u32x4 *>(ql);
    r.la1 = *reinterpret_cast<const u32x4 *>(ql + 16);
    r.lb0 = *reinterpret_cast<const u32x4 *>(ql + 32);
    r.lb1 = *reinterpret_cast<const u32x4 *>(ql + 48);
    r.h0 = *reinterpret_cast<const u32x4 *>(qh);
    r.h1 = *reinterpret_cast<const u32x4 *>(qh + 16);
    r.sc = *reinterpret_cast<const u32x2 *>(grp + 24 * 192 + 16 * j + 8 * h);
    const uint32_t dw = *reinterpret_cast<const uint32_t *>(grp + 24 * 208 + 4 * (j >> 1));
    r.d = (dw >> (16 * (j & 1))) & 0xFFFFu;
    return r;
}
/* dot_q6k_q8 over one 128-value half (csrc/libtinygiant.c:384-443):
 * q = (ql nibble | 2 qh bits << 4) - 32; the 16-value integer sums are
 * exact (the -32 offset is folded in with the 16-value x sums) and weighted
 * by their int8 sub-scales in integer, then scaled by d and the q8 scale. */
__device__ inline float dot_q6half(const Q6Half &q, const int8_t *xq, const int32_t *s16, float xd) {
    const uint32_t m4 = 0x0F0F0F0Fu, m2 = 0x30303030u;
    const u32x4 *xp = reinterpret_cast<const u32x4 *>(xq);
    int S[8];
#pragma unroll
    for (int i = 0; i < 8; i++) S[i] = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const u32x4 &A = j < 4 ? q.la0 : q.la1;
        const u32x4 &B = j < 4 ? q.lb0 : q.lb1;
        const u32x4 &H = j < 4 ? q.h0 : q.h1;
        const int c = j & 3;
        const uint32_t la = c == 0 ? A.x : c == 1 ? A.y : c == 2 ? A.z : A.w;
        const uint32_t lb = c == 0 ? B.x : c == 1 ? B.y : c == 2 ? B.z : B.w;
        const uint32_t hh = c == 0 ? H.x : c == 1 ? H.y : c == 2 ? H.z : H.w;
        const uint32_t q1 = (la & m4) | ((hh << 4) & m2);
        const uint32_t q2 = (lb & m4) | ((hh << 2) & m2);
        const uint32_t q3 = ((la >> 4) & m4) | (hh & m2);
        const uint32_t q4 = ((lb >> 4) & m4) | ((hh >> 2) & m2);
        const int hf = j >> 2;   /* 16-value group within each 32-value run */
        const u32x4 x1 = xp[(j >> 2)], x2 = xp[2 + (j >> 2)], x3 = xp[4 + (j >> 2)], x4 = xp[6 + (j >> 2)];
        const uint32_t a1 = c == 0 ? x1.x : c == 1 ? x1.y : c == 2 ? x1.z : x1.w;
        const uint32_t a2 = c == 0 ? x2.x : c == 1 ? x2.y : c == 2 ? x2.z : x2.w;
        const uint32_t a3 = c == 0 ? x3.x : c == 1 ? x3.y : c == 2 ? x3.z : x3.w;
        const uint32_t a4 = c == 0 ? x4.x : c == 1 ? x4.y : c == 2 ? x4.z : x4.w;
        S[0 + hf] = dot4(q1, a1, S[0 + hf]);
        S[2 + hf] = dot4(q2, a2, S[2 + hf]);
        S[4 + hf] = dot4(q3, a3, S[4 + hf]);
        S[6 + hf] = dot4(q4, a4, S[6 + hf]);
    }
    const u32x4 t0 = *reinterpret_cast<const u32x4 *>(s16), t1 = *reinterpret_cast<const u32x4 *>(s16 + 4);
    const int xs[8] = {(int)t0.x, (int)t0.y, (int)t0.z, (int)t0.w, (int)t1.x, (int)t1.y, (int)t1.z, (int)t1.w};
    int A = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int sc = (int)(int8_t)((i < 4 ? q.sc.x : q.sc.y) >> (8 * (i & 3)));
        A += __mul24(sc, S[i] - 32 * xs[i]);   /* |S - 32 xs| < 2^18: exact */
    }
    return ref_f16(q.d) * xd * (float)A;
}

/* q8 of 4 consecutive values per lane of one wave = one 256-block
 * (quantize_q8, csrc/libtinygiant.c:169-208; same arithmetic as
 * k_quantize_q8).  Returns the packed quants; fills the block scale and the
 * 16/32-element sums when the pointers are given. */
__device__ inline uint32_t q8_block_wave(float v0, float v1, float v2, float v3, int lane, float *d, int32_t *s32,
                                         int32_t *s16) {
    const float amax = wave_max(fmaxf(fmaxf(fabsf(v0), fabsf(v1)), fmaxf(fabsf(v2), fabsf(v3))));
    const float inv = amax > 0.f ? 127.f / amax : 0.f;
    int q0 = (int)__builtin_rintf(v0 * inv), q1 = (int)__builtin_rintf(v1 * inv);
    int q2 = (int)__builtin_rintf(v2 * inv), q3 = (int)__builtin_rintf(v3 * inv);
    int s = q0 + q1 + q2 + q3;
    s += dpp_i<0xB1>(s, s);
    s += dpp_i<0x4E>(s, s);                  /* 16-element sum in every lane of the quad */
    const int t32 = s + dpp_i<0x141>(s, s);  /* 32-element sum (half-row mirror pairs quads) */
    if (s16 && (lane & 3) == 0) s16[lane >> 2] = s;
    if (s32 && (lane & 7) == 0) s32[lane >> 3] = t32;
    if (lane == 0) *d = amax / 127.f;
    return (uint32_t)(q0 & 0xFF) | ((uint32_t)(q1 & 0xFF) << 8) | ((uint32_t)(q2 & 0xFF) << 16) |
           ((uint32_t)(q3 & 0xFF) << 24);
}

__device__ inline float silu_mul(float g, float u) { return g / (1.f + expf(-g)) * u; }

}  // namespace

/* Tags are base + layer + 1 in every region, so a launch never mistakes a
 * slot of an earlier layer or launch for its own.  A slot of parity p is
 * rewritten two layers later only after every reader of it has published
 * something the writer waited for in between. */
__global__ __launch_bounds__(NT) void k_decode_qwen(const DecodeLayer *__restrict__ layers, int L, float *h,
                                                    u32x4 *slots, unsigned *abort_flag, float eps,
                                                    uint8_t *dbg, uint64_t *times, unsigned *place, int pol) {
    __shared__ __attribute__((aligned(16))) uint8_t wgs[WGB];          /* gate/up rows of the slice */
    __shared__ __attribute__((aligned(16))) uint8_t wds[D_INS * 1024]; /* down rows of the slice (row groups) */
    __shared__ __attribute__((aligned(16))) float nws[D];              /* this layer's RMSNorm weight */
    __shared__ __attribute__((aligned(16))) float hx[D];               /* this layer's input h */
    __shared__ __attribute__((aligned(16))) float hid[I];              /* this XCD's expert hidden vector */
    __shared__ LdsX sx;
    __shared__ LdsH sh;
    __shared__ float ssq[NR];                                          /* sum of h^2 of each 64-row slice */
    __shared__ float gu[2 * RA];                                       /* gate and up row sums */
    __shared__ float part6[RB * HB];                                   /* down half-block partial dots */
    __shared__ float pp[NE][RB];                                       /* down values of every expert, own rows */
    __shared__ int lds_fail;
    __shared__ DecodeLayer lys[MAX_LAYERS];

    int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int cl = (int)threadIdx.x - NW * 64;   /* communication lane, valid in the communication waves */
    const int ct = (int)threadIdx.x;             /* compute lane, valid when < NW * 64 */
    __shared__ unsigned epoch_s;
    if (threadIdx.x == 0) {
        lds_fail = 0;
        epoch_s = read_epoch(abort_flag);
        unsigned x;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
        if (place) place[blockIdx.x] = x;
    }
    const int wg = blockIdx.x;
    const int xe = wg % NX, rk = wg / NX;        /* expert slot (= XCD) and rank */
    Buf sl = make_buf(slots, NSLOTS * 16u);
    const bool sc1_all = pol != 0;
    const bool comm = wave >= NW;

    /* gate/up: compute lane t owns block t % 8 of row-task t / 8 (tasks 0-23
     * gate rows, 24-47 up rows); down: compute lane t owns half-block t % 6
     * of down row t / 6 */
    const int ta = ct >> 3, ba = ct & 7;
    const int tb = ct / HB, hbb = ct % HB;

    /* copies into LDS: batch D (down rows), N (RMSNorm weight), A (the first
     * G_SPLIT gate/up KiB), B (the rest of the gate/up rows).  The buffer
     * descriptors are formed once per batch: the copies' memory clobber
     * would otherwise make every copy re-read the layer table from LDS. */
    struct Descs {
        u32x4 g, u;
    };
    auto descs = [&](const DecodeLayer &ly) {
        Descs d;
        d.g = buf_desc(ly.gate[xe], (uint32_t)I * GATE_RB);
        d.u = buf_desc(ly.up[xe], (uint32_t)I * GATE_RB);
        return d;
    };
    const uint32_t goff = (uint32_t)(RA * rk) * GATE_RB;
    auto copy_gate_up = [&](const Descs &d, int k) {
        if (k < SEG / 1024) copy_1k(d.g, goff + 1024u * (uint32_t)k, lds_addr(wgs + 1024 * k), lane);
        else copy_1k(d.u, goff + 1024u * (uint32_t)(k - SEG / 1024), lds_addr(wgs + 1024 * k), lane);
    };
    auto batch_d = [&](const DecodeLayer &ly) {   /* every wave */
        const u32x4 b = buf_desc(ly.down[xe], (uint32_t)D * DOWN_RB);
        for (int k = wave; k < D_INS; k += NA)
            copy_1k(b, (uint32_t)(rk * WDB) + 1024u * (uint32_t)k, lds_addr(wds + 1024 * k), lane);
    };
    auto batch_a = [&](const DecodeLayer &ly) {   /* every wave */
        const Descs d = descs(ly);
        for (int i = wave; i < G_SPLIT; i += NA) copy_gate_up(d, i);
    };
    auto batch_n = [&](const DecodeLayer &ly, int w0, int nw) {   /* RMSNorm weight: waves w0 .. w0 + nw - 1 */
        if (wave < w0) return;
        /* a layer without an RMSNorm weight still issues its copies, reading
         * nothing, so every wave's copy count stays the same */
        const u32x4 n = buf_desc(ly.norm_w, ly.norm_w != nullptr ? (uint32_t)D * 4u : 0u);
        for (int i = wave - w0; i < N_INS; i += nw) copy_1k(n, 1024u * (uint32_t)i, lds_addr(nws + 256 * i), lane);
    };
    auto batch_b = [&](const DecodeLayer &ly, int w0, int nw) {   /* waves w0 .. w0 + nw - 1 */
        const Descs d = descs(ly);
        for (int k = G_SPLIT + wave - w0; k < G_INS; k += nw) copy_gate_up(d, k);
    };
    auto put = [&](uint32_t slot, unsigned tag, float a, float b, float c, bool cross) {
        if (cross || sc1_all) put_slot<CPOL_SC1>(sl, slot, tag, a, b, c);
        else put_slot<CPOL_PLAIN>(sl, slot, tag, a, b, c);
    };

    /* layer descriptors -> LDS (the loop then never chases pointers in
     * global memory); layer input: the caller's h for layer 0 */
    {
        const uint32_t *src = reinterpret_cast<const uint32_t *>(layers);
        uint32_t *dst = reinterpret_cast<uint32_t *>(lys);
        const int words = L * (int)(sizeof(DecodeLayer) / 4);
        for (int t = threadIdx.x; t < words; t += NT) dst[t] = src[t];
    }
    for (int t = threadIdx.x; t < D / 4; t += NT) reinterpret_cast<u32x4 *>(hx)[t] = reinterpret_cast<const u32x4 *>(h)[t];
    __syncthreads();
    /* slice sums of h^2 for layer 0 (later layers receive them with h) */
#pragma unroll
    for (int i = 0; i < NR / NA; i++) {
        const int sl = wave * (NR / NA) + i;
        const float v = hx[RB * sl + lane];
        const float ss = wave_sum(v * v);
        if (lane == 0) ssq[sl] = ss;
    }
    batch_a(lys[0]);
    batch_b(lys[0], 0, NA);
    batch_n(lys[0], 0, NA);
    wait_copies();
    __syncthreads();

    const unsigned base = epoch_s;   /* read after the prologue barrier */
    for (int l = 0; l < L; l++) {
        const DecodeLayer &ly = lys[l];
        const unsigned par = (unsigned)(l & 1);
        const unsigned tag = base + (unsigned)l + 1u;
        const bool has_nw = ly.norm_w != nullptr;
        const bool more = l + 1 < L;
        /* an opaque copy of the lane keeps per-lane address arithmetic inside
         * the loop instead of hoisted (and live) across every layer */
        int clv = cl;
        asm volatile("" : "+v"(clv));
        asm volatile("" : "+v"(lane));
        /* optional phase timestamps (100 MHz clock): thread 0 after each phase,
         * communication lane 0 when it publishes (checkpoints 9-11) */
        const bool tw = times && threadIdx.x == 0;
        const bool tc = times && clv == 0;
        uint64_t *tr = times ? times + ((size_t)wg * L + l) * NTS : nullptr;
        if (tw) tr[0] = wall_clock64();
        /* ---- 1: gather h from the other ranks of this XCD (the copies of
         * this layer's gate/up rows and RMSNorm weight are ahead of the polls) ---- */
        if (l > 0) {
            {   /* every wave polls: the compute waves are idle here */
                unsigned rounds = 0;
                if (tc) tr[15] = wall_clock64();
                const bool ok = poll_slots<NT, ((NR - 1) * PS + NT - 1) / NT>(
                    sl, (int)threadIdx.x, (NR - 1) * PS, base + (unsigned)l, abort_flag,
                    [&](int f) {
                        const int jj = f / PS, t = f % PS;
                        const int j = jj + (jj >= rk);
                        return HSL + ((par ^ 1u) * NWG + (uint32_t)(xe + NX * j)) * PS + (uint32_t)t;
                    },
                    [&](int f, const u32x4 &v) {
                        const int jj = f / PS, t = f % PS;
                        const int j = jj + (jj >= rk);
                        float *o = hx + RB * j + VPS * t;
                        o[0] = __uint_as_float(v.y);
                        if (t == PS - 1) {
                            ssq[j] = __uint_as_float(v.z);   /* the last slot carries the slice's sum of h^2 */
                        } else {
                            o[1] = __uint_as_float(v.z);
                            o[2] = __uint_as_float(v.w);
                        }
                    },
                    &rounds);
                if (tc) {
                    tr[16] = wall_clock64();
                    tr[17] = rounds;
                }
                if (!ok) lds_fail = 1;
            }
            wait_copies();   /* this layer's gate/up rows and RMSNorm weight (batches N, A, B) */
            bar_lds();
            if (lds_fail) {
                advance_epoch(abort_flag, base, L);
                return;
            }
        }
        if (tw) tr[1] = wall_clock64();
        /* this layer's down rows stream in during RMSNorm, gate/up and the
         * hidden gather */
        batch_d(ly);
        /* ---- 2: RMSNorm (weight norm_w or 1) then q8, in LDS; wave w owns block w.
         * sum h^2 = the 32 slice sums in rank order (each a fixed DPP tree) ---- */
        {
            float tot = 0.f;
#pragma unroll
            for (int i = 0; i < NR; i++) tot += ssq[i];
            const float scale = 1.f / sqrtf(tot / (float)D + eps);
            auto norm_block = [&](int b) {
                const int t = 64 * b + lane;   /* values 4 t .. 4 t + 3 */
                const u32x4 hv = reinterpret_cast<const u32x4 *>(hx)[t];
                u32x4 wv;
                if (has_nw) {
                    wv = reinterpret_cast<const u32x4 *>(nws)[t];
                } else {
                    wv.x = wv.y = wv.z = wv.w = __float_as_uint(1.f);
                }
                const float v0 = (__uint_as_float(hv.x) * scale) * __uint_as_float(wv.x);
                const float v1 = (__uint_as_float(hv.y) * scale) * __uint_as_float(wv.y);
                const float v2 = (__uint_as_float(hv.z) * scale) * __uint_as_float(wv.z);
                const float v3 = (__uint_as_float(hv.w) * scale) * __uint_as_float(wv.w);
                const uint32_t q = q8_block_wave(v0, v1, v2, v3, lane, &sx.d[b], &sx.s32[b * 8], nullptr);
                reinterpret_cast<uint32_t *>(sx.qs + b * XST)[lane] = q;
                if (dbg && wg == 0) {
                    uint8_t *rec = dbg + (size_t)l * DecodeDebug::BYTES;
                    reinterpret_cast<u32x4 *>(rec + DecodeDebug::HIN)[t] = hv;
                    u32x4 xv;
                    xv.x = __float_as_uint(v0);
                    xv.y = __float_as_uint(v1);
                    xv.z = __float_as_uint(v2);
                    xv.w = __float_as_uint(v3);
                    reinterpret_cast<u32x4 *>(rec + DecodeDebug::X)[t] = xv;
                    reinterpret_cast<uint32_t *>(rec + DecodeDebug::XQ)[t] = q;
                }
            };
            norm_block(wave);
        }
        bar_lds();
        if (tw) tr[2] = wall_clock64();
        if (dbg && wg == 0) {
            uint8_t *rec = dbg + (size_t)l * DecodeDebug::BYTES;
            if (threadIdx.x < NBD) reinterpret_cast<float *>(rec + DecodeDebug::XD)[threadIdx.x] = sx.d[threadIdx.x];
            if (threadIdx.x < NBD * 8)
                reinterpret_cast<int32_t *>(rec + DecodeDebug::XS32)[threadIdx.x] = sx.s32[threadIdx.x];
        }
        /* the next layer's RMSNorm weight streams in during gate/up, issued by
         * the communication waves (idle there) */
        if (more && comm) batch_n(lys[l + 1], NW, NC);
        /* ---- 3: gate/up rows [24 rk, 24 rk + 24) of expert xe, one block per lane ---- */
        if (wave < NW) {
            const Q4Blk wa = lds_q4blk(wgs + (ta / RA) * SEG + (ta % RA) * GATE_RB + ba * 144);
            float v = dot_q4blk(wa, sx.qs + ba * XST, sx.s32 + ba * 8, sx.d[ba]);
            v = seg_sum_last<NBD>(v);
            if (ba == NBD - 1) gu[ta] = v;
        }
        bar_lds();
        if (tw) tr[3] = wall_clock64();
        /* ---- 4: all-gather the expert's hidden vector within the XCD (the
         * down rows' copies are ahead of the polls) ---- */
        if (comm) {
            /* SwiGLU, one value per lane of the first communication wave; the
             * same wave then publishes them (its LDS accesses run in order) */
            if (clv < RA) hid[RA * rk + clv] = silu_mul(gu[clv], gu[RA + clv]);
            __builtin_amdgcn_wave_barrier();
            if (clv < GS) {
                const float *a = hid + RA * rk + VPS * clv;
                put(GSL + (par * NWG + (uint32_t)wg) * GS + (uint32_t)clv, tag, a[0], a[1], a[2], false);
            }
            if (tc) tr[9] = wall_clock64();
        }
        {   /* every wave polls the other ranks' slots while the first
             * communication wave publishes this rank's */
            unsigned rounds = 0;
            if (tc) tr[12] = wall_clock64();
            const bool ok = poll_slots<NT, ((NR - 1) * GS + NT - 1) / NT>(
                sl, (int)threadIdx.x, (NR - 1) * GS, tag, abort_flag,
                [&](int f) {
                    const int jj = f / GS, t = f % GS;
                    const int j = jj + (jj >= rk);
                    return GSL + (par * NWG + (uint32_t)(xe + NX * j)) * GS + (uint32_t)t;
                },
                [&](int f, const u32x4 &v) {
                    const int jj = f / GS, t = f % GS;
                    const int j = jj + (jj >= rk);
                    float *o = hid + RA * j + VPS * t;
                    o[0] = __uint_as_float(v.y);
                    o[1] = __uint_as_float(v.z);
                    o[2] = __uint_as_float(v.w);
                },
                &rounds);
            if (tc) {
                tr[13] = wall_clock64();
                tr[14] = rounds;
            }
            if (!ok) lds_fail = 1;
        }
        wait_copies();   /* this layer's down rows (batch D) */
        bar_lds();
        if (lds_fail) {
            advance_epoch(abort_flag, base, L);
            return;
        }
        if (tw) tr[4] = wall_clock64();
        /* part of the next layer's gate/up rows streams in from here (the
         * gate/up region is free) */
        if (more) batch_a(lys[l + 1]);
        /* ---- 5: q8 of the hidden vector, one wave per 256-block ---- */
        if (wave < NBI) {
            const int b = wave;
            const u32x4 hv = reinterpret_cast<const u32x4 *>(hid + b * 256)[lane];
            const uint32_t q = q8_block_wave(__uint_as_float(hv.x), __uint_as_float(hv.y), __uint_as_float(hv.z),
                                             __uint_as_float(hv.w), lane, &sh.d[b], nullptr, &sh.s16[b * 16]);
            reinterpret_cast<uint32_t *>(sh.qs + (2 * b + (lane >> 5)) * HST)[lane & 31] = q;
            if (dbg && rk == 0) {   /* workgroups 0..7: expert slot xe's record */
                uint8_t *rec = dbg + (size_t)l * DecodeDebug::BYTES;
                reinterpret_cast<u32x4 *>(rec + DecodeDebug::HID + (xe * I + b * 256) * 4)[lane] = hv;
                reinterpret_cast<uint32_t *>(rec + DecodeDebug::HQ + xe * I + b * 256)[lane] = q;
            }
        }
        bar_lds();
        if (tw) tr[5] = wall_clock64();
        if (dbg && rk == 0) {
            uint8_t *rec = dbg + (size_t)l * DecodeDebug::BYTES;
            if (threadIdx.x < NBI) reinterpret_cast<float *>(rec + DecodeDebug::HD)[xe * NBI + threadIdx.x] = sh.d[threadIdx.x];
            if (threadIdx.x < NBI * 16)
                reinterpret_cast<int32_t *>(rec + DecodeDebug::HS16)[xe * NBI * 16 + threadIdx.x] = sh.s16[threadIdx.x];
        }
        /* ---- 6: down rows [64 rk, 64 rk + 64) of expert xe, one half-block per lane ---- */
        if (B_AT_DOWN && more && comm) batch_b(lys[l + 1], NW, NC);
        if (wave < NW) {
            const int b = hbb >> 1;
            const Q6Half wb = lds_q6half(wds + (tb >> 3) * DGRP, (tb & 7) * NBI + b, hbb & 1);
            part6[ct] = dot_q6half(wb, sh.qs + hbb * HST, sh.s16 + b * 16 + 8 * (hbb & 1), sh.d[b]);
        }
        bar_lds();
        if (tw) tr[6] = wall_clock64();
        /* ---- 7: cross-XCD hop: rank rk of every XCD trades its 64 down values ---- */
        if (comm) {
            /* row sums of the six half-block dots, in half-block order, one row
             * per lane of the first communication wave, which then publishes */
            if (clv < RB) {
                float a = 0.f;
#pragma unroll
                for (int i = 0; i < HB; i++) a += part6[HB * clv + i];
                pp[xe][clv] = a;
            }
            __builtin_amdgcn_wave_barrier();
            if (clv < PS) {
                const int r0 = VPS * clv;
                put(PSL + (par * NWG + (uint32_t)wg) * PS + (uint32_t)clv, tag, pp[xe][r0],
                    r0 + 1 < RB ? pp[xe][r0 + 1] : 0.f, r0 + 2 < RB ? pp[xe][r0 + 2] : 0.f, true);
            }
            if (tc) tr[10] = wall_clock64();
        }
        if (comm) {   /* the hop is polled by the communication waves alone (every
                       * wave polling it measured slower) */
            unsigned rounds = 0;
            const bool ok = poll_slots<CL, ((NX - 1) * PS + CL - 1) / CL>(
                sl, clv, (NX - 1) * PS, tag, abort_flag,
                [&](int f) {
                    const int xx = f / PS, t = f % PS;
                    const int x = xx + (xx >= xe);
                    return PSL + (par * NWG + (uint32_t)(x + NX * rk)) * PS + (uint32_t)t;
                },
                [&](int f, const u32x4 &v) {
                    const int xx = f / PS, t = f % PS;
                    const int x = xx + (xx >= xe);
                    float *o = pp[x] + VPS * t;
                    o[0] = __uint_as_float(v.y);
                    if (VPS * t + 1 < RB) o[1] = __uint_as_float(v.z);
                    if (VPS * t + 2 < RB) o[2] = __uint_as_float(v.w);
                },
                &rounds);
            if (tc) {
                tr[18] = wall_clock64();
                tr[19] = rounds;
            }
            if (!ok) lds_fail = 1;
        }
        bar_lds();
        if (lds_fail) {
            wait_copies();   /* no copy into LDS outlives the workgroup */
            advance_epoch(abort_flag, base, L);
            return;
        }
        if (tw) tr[7] = wall_clock64();
        /* the rest of the next layer's gate/up rows */
        if (!B_AT_DOWN && more) batch_b(lys[l + 1], 0, NA);
        /* ---- 8: combine rows [64 rk, 64 rk + 64) in expert order, publish ---- */
        /* one row per lane of the first communication wave, which then
         * publishes the slice */
        if (comm && clv < RB) {
            const int r = RB * rk + clv;
            float a = hx[r];
#pragma unroll
            for (int e = 0; e < NE; e++) a += ly.w[e] * pp[e][clv];
            hx[r] = a;
            if (l == L - 1 && xe == 0) h[r] = a;
            const float ss = wave_sum(a * a);   /* this slice's sum of h^2, for the next RMSNorm */
            if (clv == 0) ssq[rk] = ss;
            __builtin_amdgcn_wave_barrier();
            if (more && clv < PS) {
                const float *o = hx + RB * rk + VPS * clv;
                const bool last = clv == PS - 1;   /* row 63 alone, plus the slice sum */
                put(HSL + (par * NWG + (uint32_t)wg) * PS + (uint32_t)clv, tag, o[0], last ? ss : o[1],
                    last ? 0.f : o[2], false);
            }
            if (tc) tr[11] = wall_clock64();
        }
        if (tw) tr[8] = wall_clock64();
    }
    wait_copies();
    advance_epoch(abort_flag, base, L);
}

/* Rewrites a Q6_K matrix (nrows x nb 210-byte blocks, nrows a multiple of
 * 8) into the row-group layout the persistent step reads: group g of rows
 * [8 g, 8 g + 8) is {ql[8 nb][128] | qh[8 nb][64] | sc[8 nb][16] | d[8 nb]},
 * block j = r * nb + b, the same 8 * nb * 210 bytes.  One thread per block. */
__global__ void k_q6k_row_groups(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int nrows, int nb) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nrows * nb) return;
    const int row = t / nb, b = t % nb, g = row >> 3, j = (row & 7) * nb + b;
    const uint8_t *s = src + (size_t)t * 210;
    uint8_t *o = dst + (size_t)g * 8 * nb * 210;
    const int n8 = 8 * nb;
    for (int i = 0; i < 128; i++) o[128 * j + i] = s[i];
    for (int i = 0; i < 64; i++) o[128 * n8 + 64 * j + i] = s[128 + i];
    for (int i = 0; i < 16; i++) o[192 * n8 + 16 * j + i] = s[192 + i];
    o[208 * n8 + 2 * j] = s[208];
    o[208 * n8 + 2 * j + 1] = s[209];
}

hipError_t launch_q6k_row_groups(const void *src, void *dst, int nrows, int nb, hipStream_t st) {
    const int n = nrows * nb;
    hipLaunchKernelGGL(k_q6k_row_groups, dim3((n + 255) / 256), dim3(256), 0, st, (const uint8_t *)src,
                       (uint8_t *)dst, nrows, nb);
    return hipGetLastError();
}

DecodeShape decode_qwen_shape() { return DecodeShape{D, I, TG_FMT_Q4K, TG_FMT_Q6K, DECODE_MAXE, NT}; }

int decode_qwen_max_grid() {
    int dev = 0, per_cu = 0;
    hipDeviceProp_t pr;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&pr, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *)k_decode_qwen, NT, 0) != hipSuccess)
        return 0;
    return per_cu * pr.multiProcessorCount;
}

size_t decode_qwen_slot_bytes(int) { return (size_t)NSLOTS * 16; }

hipError_t launch_decode_qwen(const DecodeLayer *layers_dev, int L, float *h_dev, void *slots_dev,
                              unsigned *abort_dev, float eps, uint8_t *debug_dev, uint64_t *times_dev,
                              unsigned *place_dev, int pol, int grid, bool cooperative, hipStream_t st) {
    void *args[] = {(void *)&layers_dev, (void *)&L,         (void *)&h_dev,     (void *)&slots_dev,
                    (void *)&abort_dev,  (void *)&eps,       (void *)&debug_dev, (void *)&times_dev,
                    (void *)&place_dev,  (void *)&pol};
    if (cooperative) return hipLaunchCooperativeKernel((const void *)k_decode_qwen, dim3(grid), dim3(NT), args, 0, st);
    return hipLaunchKernel((const void *)k_decode_qwen, dim3(grid), dim3(NT), args, 0, st);
}

const void *decode_qwen_fn() { return (const void *)k_decode_qwen; }
int decode_threads() { return NT; }

}  // namespace tg
