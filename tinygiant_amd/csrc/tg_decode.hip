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
 * Only step 7 crosses XCDs.  Each layer's weights are loaded into registers
 * one layer ahead: a compute lane holds one Q4_K block (gate or up) and one
 * Q6_K half-block (down).  The next layer's gate/up blocks are issued during
 * step 4 and its down half-blocks and RMSNorm weight during step 7, while the
 * compute waves would otherwise wait; the six compute waves issue one after
 * another so few weight requests sit in the CU's memory queue ahead of the
 * exchange polls.
 *
 * Exchanges use epoch-tagged 16-byte slots {tag, v0, v1, v2}, written and
 * polled with device-coherent (sc1) vector accesses so the tag and its values
 * arrive together.  Two communication waves per workgroup do the polling and
 * publishing, so a poll never waits behind the compute waves' outstanding
 * weight loads.  Every wait is bounded; a timed-out wait raises an abort flag
 * that releases every other waiter, so the grid always drains.  Placement
 * only affects speed: every exchange is device-coherent wherever the
 * workgroups run.
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
static_assert(NE == NX, "one expert per XCD");
static_assert(NR * RA == I && NR * RB == D && RA % VPS == 0, "row split");
static_assert(2 * RA * NBD == NW * 64, "gate/up: one Q4_K block per compute lane");
static_assert(RB * HB == NW * 64, "down: one Q6_K half-block per compute lane");
static_assert((NR - 1) * PS <= 6 * CL && (NR - 1) * GS <= 2 * CL && (NX - 1) * PS <= 2 * CL, "poll shares");
static_assert(NBI <= NA && NBD == NA, "q8 blocks per wave");
static_assert(RB == VPS * (PS - 1) + 1, "the last slice slot holds one row and the slice's sum of h^2");
static_assert(NR % NA == 0, "layer-0 slice sums: whole slices per wave");

/* A slot is 16 bytes {tag, v0, v1, v2} written and read as one vector access,
 * so its tag and values arrive together.  Cross-XCD slots are stored and
 * loaded with device-scope coherence (sc1: the store writes through to
 * memory, the load does not allocate in the reader's L2, so it never sees a
 * stale line).  Slots read only inside the writer's XCD are stored plainly
 * (the line stays in that XCD's L2) and loaded with sc1, which bypasses the
 * CU's L1 and reads the L2 line: measured coherent, and ~0.4 us faster per
 * exchange than writing through to memory. */
constexpr int PREFETCH_STAGGER = 16;   /* s_sleep units (64 cycles) between compute waves' prefetch issue */
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
__device__ inline Q4Blk load_q4blk(Buf b, uint32_t off) {
    Q4Blk r;
#pragma unroll
    for (int i = 0; i < 9; i++) r.w[i] = ld16(b, off + 16u * i);
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
 * sub-scales and the f16 d. */
struct Q6Half {
    u32x4 la0, la1, lb0, lb1, h0, h1;
    u32x2 sc;
    uint32_t d;   /* d is the high 16 bits */
};
__device__ inline Q6Half load_q6half(Buf b, uint32_t blk, int h) {
    Q6Half r;
    const uint32_t ql = blk + 64u * h, qh = blk + 128u + 32u * h;
    r.la0 = ld16(b, ql);
    r.la1 = ld16(b, ql + 16);
    r.lb0 = ld16(b, ql + 32);
    r.lb1 = ld16(b, ql + 48);
    r.h0 = ld16(b, qh);
    r.h1 = ld16(b, qh + 16);
    r.sc = ld8(b, blk + 192u + 8u * h);
    r.d = ld4(b, blk + 206u);
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
    return ref_f16(q.d >> 16) * xd * (float)A;
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
                                                    u32x4 *slots, unsigned *abort_flag, unsigned base, float eps,
                                                    uint8_t *dbg, uint64_t *times) {
    __shared__ __attribute__((aligned(16))) float hx[D];          /* this layer's input h */
    __shared__ __attribute__((aligned(16))) float nws[D];         /* this layer's RMSNorm weight */
    __shared__ __attribute__((aligned(16))) float hid[I];         /* this XCD's expert hidden vector */
    __shared__ LdsX sx;
    __shared__ LdsH sh;
    __shared__ float ssq[NR];                                     /* sum of h^2 of each 64-row slice */
    __shared__ float gu[2 * RA];                                  /* gate and up row sums */
    __shared__ float part6[RB * HB];                              /* down half-block partial dots */
    __shared__ float pp[NE][RB];                                  /* down values of every expert, own rows */
    __shared__ int lds_fail;
    __shared__ DecodeLayer lys[MAX_LAYERS];

    int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int cl = (int)threadIdx.x - NW * 64;   /* communication lane, valid when >= 0 */
    const int ct = (int)threadIdx.x;             /* compute lane, valid when < NW * 64 */
    if (threadIdx.x == 0) lds_fail = 0;
    const int wg = blockIdx.x;
    const int xe = wg % NX, rk = wg / NX;        /* expert slot (= XCD) and rank */
    Buf sl = make_buf(slots, NSLOTS * 16u);

    Q4Blk wa;                                    /* this lane's gate or up block */
    Q6Half wb;                                   /* this lane's down half-block */
    u32x4 nw0, nw1;                              /* next layer's RMSNorm weight (compute lanes) */
    /* gate/up: compute lane t owns block t % 8 of row-task t / 8 (tasks 0-23
     * gate rows, 24-47 up rows); down: compute lane t owns half-block t % 6
     * of down row t / 6 */
    const int ta = ct >> 3, ba = ct & 7;
    const int tb = ct / HB, hbb = ct % HB;

    /* loads are unconditional so the registers' live ranges end at their
     * use; an inactive step reads through an empty descriptor (zeros, no
     * memory access) */
    auto load_a = [&](const DecodeLayer &ly) {
        /* waves 0-2 hold gate rows, waves 3-5 up rows (uniform per wave) */
        const bool cw = wave < NW;
        const uint8_t *m = wave < NW / 2 ? ly.gate[xe] : ly.up[xe];
        Buf gb = make_buf_uniform(cw ? m : nullptr, cw ? (uint32_t)I * GATE_RB : 0u);
        const uint32_t r = (uint32_t)(RA * rk + (ta % RA));
        wa = load_q4blk(gb, r * GATE_RB + (uint32_t)ba * 144u);
    };
    auto load_b = [&](const DecodeLayer &ly) {
        const bool cw = wave < NW;
        Buf db = make_buf_uniform(cw ? ly.down[xe] : nullptr, cw ? (uint32_t)D * DOWN_RB : 0u);
        const uint32_t r = (uint32_t)(RB * rk + tb);
        wb = load_q6half(db, r * DOWN_RB + (uint32_t)(hbb >> 1) * 210u, hbb & 1);
    };
    /* RMSNorm weight: compute lane t holds float4 t and (t < 128) float4 384 + t */
    auto load_nw = [&](const DecodeLayer &ly) {
        const bool on = wave < NW && ly.norm_w != nullptr;
        Buf nb = make_buf_uniform(on ? ly.norm_w : nullptr, on ? (uint32_t)D * 4u : 0u);
        nw0 = ld16(nb, (uint32_t)ct * 16u);
        nw1 = ld16(nb, (uint32_t)(NW * 64 + ct) * 16u);
    };
    auto store_nw = [&]() {
        if (wave < NW) {
            reinterpret_cast<u32x4 *>(nws)[ct] = nw0;
            if (ct < D / 4 - NW * 64) reinterpret_cast<u32x4 *>(nws)[NW * 64 + ct] = nw1;
        }
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
    load_nw(lys[0]);
    load_a(lys[0]);
    load_b(lys[0]);
    store_nw();

    for (int l = 0; l < L; l++) {
        const DecodeLayer &ly = lys[l];
        const unsigned par = (unsigned)(l & 1);
        const unsigned tag = base + (unsigned)l + 1u;
        const bool has_nw = ly.norm_w != nullptr;
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
        /* ---- 1: gather h from the other ranks of this XCD ---- */
        if (l > 0) {
            if (cl >= 0) {
                unsigned rounds = 0;
                if (tc) tr[15] = wall_clock64();
                const bool ok = poll_slots<CL, 6>(
                    sl, clv, (NR - 1) * PS, base + (unsigned)l, abort_flag,
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
                    tc ? &rounds : nullptr);
                if (tc) {
                    tr[16] = wall_clock64();
                    tr[17] = rounds;
                }
                if (!ok) lds_fail = 1;
            } else {
                store_nw();
            }
            __syncthreads();
            if (lds_fail) return;
        }
        if (tw) tr[1] = wall_clock64();
        /* ---- 2: RMSNorm (weight norm_w or 1) then q8, in LDS; wave w owns block w.
         * sum h^2 = the 32 slice sums in rank order (each a fixed DPP tree) ---- */
        if (l == 0) __syncthreads();
        {
            float tot = 0.f;
#pragma unroll
            for (int i = 0; i < NR; i++) tot += ssq[i];
            const float scale = 1.f / sqrtf(tot / (float)D + eps);
            const u32x4 hv = reinterpret_cast<const u32x4 *>(hx)[threadIdx.x];
            u32x4 wv;
            if (has_nw) {
                wv = reinterpret_cast<const u32x4 *>(nws)[threadIdx.x];
            } else {
                wv.x = wv.y = wv.z = wv.w = __float_as_uint(1.f);
            }
            const float v0 = (__uint_as_float(hv.x) * scale) * __uint_as_float(wv.x);
            const float v1 = (__uint_as_float(hv.y) * scale) * __uint_as_float(wv.y);
            const float v2 = (__uint_as_float(hv.z) * scale) * __uint_as_float(wv.z);
            const float v3 = (__uint_as_float(hv.w) * scale) * __uint_as_float(wv.w);
            const uint32_t q = q8_block_wave(v0, v1, v2, v3, lane, &sx.d[wave], &sx.s32[wave * 8], nullptr);
            reinterpret_cast<uint32_t *>(sx.qs + wave * XST)[lane] = q;
            if (dbg && wg == 0) {
                uint8_t *rec = dbg + (size_t)l * DecodeDebug::BYTES;
                reinterpret_cast<u32x4 *>(rec + DecodeDebug::HIN)[threadIdx.x] = hv;
                u32x4 xv;
                xv.x = __float_as_uint(v0);
                xv.y = __float_as_uint(v1);
                xv.z = __float_as_uint(v2);
                xv.w = __float_as_uint(v3);
                reinterpret_cast<u32x4 *>(rec + DecodeDebug::X)[threadIdx.x] = xv;
                reinterpret_cast<uint32_t *>(rec + DecodeDebug::XQ)[threadIdx.x] = q;
            }
        }
        __syncthreads();
        if (tw) tr[2] = wall_clock64();
        if (dbg && wg == 0) {
            uint8_t *rec = dbg + (size_t)l * DecodeDebug::BYTES;
            if (threadIdx.x < NBD) reinterpret_cast<float *>(rec + DecodeDebug::XD)[threadIdx.x] = sx.d[threadIdx.x];
            if (threadIdx.x < NBD * 8)
                reinterpret_cast<int32_t *>(rec + DecodeDebug::XS32)[threadIdx.x] = sx.s32[threadIdx.x];
        }
        /* ---- 3: gate/up rows [24 rk, 24 rk + 24) of expert xe, one block per lane ---- */
        if (wave < NW) {
            float v = dot_q4blk(wa, sx.qs + ba * XST, sx.s32 + ba * 8, sx.d[ba]);
            v = seg_sum_last<NBD>(v);
            if (ba == NBD - 1) gu[ta] = v;
        }
        __syncthreads();
        if (tw) tr[3] = wall_clock64();
        /* ---- 4: all-gather the expert's hidden vector within the XCD ---- */
        /* meanwhile the compute waves issue the next layer's gate/up blocks,
         * one wave after another, so the weight requests queued ahead of the
         * polls stay short */
        if (cl < 0 && l + 1 < L) {
            for (int z = 0; z < wave; z++) __builtin_amdgcn_s_sleep(PREFETCH_STAGGER);
            load_a(lys[l + 1]);
        }
        if (cl >= 0) {
            /* SwiGLU, one value per lane of the first communication wave; the
             * same wave then publishes them (its LDS accesses run in order) */
            if (clv < RA) hid[RA * rk + clv] = silu_mul(gu[clv], gu[RA + clv]);
            __builtin_amdgcn_wave_barrier();
            if (clv < GS) {
                const float *a = hid + RA * rk + VPS * clv;
                put_slot<CPOL_PLAIN>(sl, GSL + (par * NWG + (uint32_t)wg) * GS + (uint32_t)clv, tag, a[0], a[1], a[2]);
            }
            if (tc) tr[9] = wall_clock64();
            unsigned rounds = 0;
            if (tc) tr[12] = wall_clock64();
            const bool ok = poll_slots<CL, 2>(
                sl, clv, (NR - 1) * GS, tag, abort_flag,
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
                tc ? &rounds : nullptr);
            if (tc) {
                tr[13] = wall_clock64();
                tr[14] = rounds;
            }
            if (!ok) lds_fail = 1;
        }
        __syncthreads();
        if (lds_fail) return;
        if (tw) tr[4] = wall_clock64();
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
        __syncthreads();
        if (tw) tr[5] = wall_clock64();
        if (dbg && rk == 0) {
            uint8_t *rec = dbg + (size_t)l * DecodeDebug::BYTES;
            if (threadIdx.x < NBI) reinterpret_cast<float *>(rec + DecodeDebug::HD)[xe * NBI + threadIdx.x] = sh.d[threadIdx.x];
            if (threadIdx.x < NBI * 16)
                reinterpret_cast<int32_t *>(rec + DecodeDebug::HS16)[xe * NBI * 16 + threadIdx.x] = sh.s16[threadIdx.x];
        }
        /* ---- 6: down rows [64 rk, 64 rk + 64) of expert xe, one half-block per lane ---- */
        if (wave < NW) {
            const int b = hbb >> 1;
            part6[ct] = dot_q6half(wb, sh.qs + hbb * HST, sh.s16 + b * 16 + 8 * (hbb & 1), sh.d[b]);
        }
        __syncthreads();
        if (tw) tr[6] = wall_clock64();
        /* ---- 7: cross-XCD hop: rank rk of every XCD trades its 64 down values ---- */
        /* meanwhile the next layer's RMSNorm weight and down rows are issued */
        if (cl < 0 && l + 1 < L) {
            for (int z = 0; z < wave; z++) __builtin_amdgcn_s_sleep(PREFETCH_STAGGER);
            load_nw(lys[l + 1]);
            load_b(lys[l + 1]);
        }
        if (cl >= 0) {
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
                put_slot<CPOL_SC1>(sl, PSL + (par * NWG + (uint32_t)wg) * PS + (uint32_t)clv, tag, pp[xe][r0],
                                   r0 + 1 < RB ? pp[xe][r0 + 1] : 0.f, r0 + 2 < RB ? pp[xe][r0 + 2] : 0.f);
            }
            if (tc) tr[10] = wall_clock64();
            unsigned rounds = 0;
            const bool ok = poll_slots<CL, 2>(
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
                tc ? &rounds : nullptr);
            if (tc) {
                tr[18] = wall_clock64();
                tr[19] = rounds;
            }
            if (!ok) lds_fail = 1;
        }
        __syncthreads();
        if (lds_fail) return;
        if (tw) tr[7] = wall_clock64();
        /* ---- 8: combine rows [64 rk, 64 rk + 64) in expert order, publish ---- */
        /* one row per lane of the first communication wave, which then
         * publishes the slice */
        if (cl >= 0 && clv < RB) {
            const int r = RB * rk + clv;
            float a = hx[r];
#pragma unroll
            for (int e = 0; e < NE; e++) a += ly.w[e] * pp[e][clv];
            hx[r] = a;
            if (l == L - 1 && xe == 0) h[r] = a;
            const float ss = wave_sum(a * a);   /* this slice's sum of h^2, for the next RMSNorm */
            if (clv == 0) ssq[rk] = ss;
            __builtin_amdgcn_wave_barrier();
            if (l + 1 < L && clv < PS) {
                const float *o = hx + RB * rk + VPS * clv;
                const bool last = clv == PS - 1;   /* row 63 alone, plus the slice sum */
                put_slot<CPOL_PLAIN>(sl, HSL + (par * NWG + (uint32_t)wg) * PS + (uint32_t)clv, tag, o[0],
                                     last ? ss : o[1], last ? 0.f : o[2]);
            }
            if (tc) tr[11] = wall_clock64();
        }
        if (tw) tr[8] = wall_clock64();
    }
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
                              unsigned *abort_dev, unsigned base, float eps, uint8_t *debug_dev, uint64_t *times_dev,
                              int grid, bool cooperative, hipStream_t st) {
    void *args[] = {(void *)&layers_dev, (void *)&L, (void *)&h_dev, (void *)&slots_dev, (void *)&abort_dev,
                    (void *)&base, (void *)&eps, (void *)&debug_dev, (void *)&times_dev};
    if (cooperative) return hipLaunchCooperativeKernel((const void *)k_decode_qwen, dim3(grid), dim3(NT), args, 0, st);
    return hipLaunchKernel((const void *)k_decode_qwen, dim3(grid), dim3(NT), args, 0, st);
}

}  // namespace tg
