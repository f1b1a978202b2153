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
 * one layer ahead (gate/up after step 3, down and the RMSNorm weight after
 * step 6), so the weight stream overlaps the exchanges.
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
constexpr int SA = 32;                /* lanes per gate/up row: 8 blocks x 4 items */
constexpr int SB = 16;                /* lanes per down row: 3 blocks x 4 items = 12 used */
constexpr int STEPS_A = RA / 2;       /* two-row wave steps: 12 */
constexpr int STEPS_B = RB / 4;       /* four-row wave steps: 16 */
constexpr int MAX_A = (STEPS_A + NW - 1) / NW;   /* 2 */
constexpr int MAX_B = (STEPS_B + NW - 1) / NW;   /* 3 */
constexpr int VPS = 3;                /* values per slot */
constexpr int GS = RA / VPS;          /* hidden slots per workgroup: 8 */
constexpr int PS = (RB + VPS - 1) / VPS;   /* slots per 64-row slice: 22 */
constexpr unsigned SPIN_LIMIT = 1u << 20;
constexpr int MAX_LAYERS = 64;        /* layer descriptors staged in LDS */
constexpr int NTS = 16;               /* timestamps per layer */
static_assert(NE == NX, "one expert per XCD");
static_assert(NR * RA == I && NR * RB == D && RA % VPS == 0, "row split");
static_assert(MAX_A == 2 && MAX_B == 3, "register budget assumes 2 gate/up and 3 down steps");
static_assert((NR - 1) * PS <= 6 * CL && (NR - 1) * GS <= 2 * CL && (NX - 1) * PS <= 2 * CL, "poll shares");
static_assert(NBI <= NA && NBD == NA, "q8 blocks per wave");

/* A slot is 16 bytes {tag, v0, v1, v2} written and read as one vector access
 * with device-scope coherence (sc1). */
constexpr int CPOL_SC1 = 16;
/* slot regions (u32x4 index), each double buffered by layer parity:
 *   h slices  [2][NWG][PS]   rows [64 j, 64 j + 64) of the layer output
 *   hidden    [2][NWG][GS]   the workgroup's 24 hidden values
 *   partials  [2][NWG][PS]   the workgroup's 64 down values (unweighted) */
constexpr uint32_t HSL = 0, GSL = 2u * NWG * PS, PSL = GSL + 2u * NWG * GS, NSLOTS = PSL + 2u * NWG * PS;

/* ---- LDS images of q8 rows ---- */
struct __attribute__((aligned(16))) LdsX {   /* q8(RMSNorm(h)) : D values */
    int8_t qs[D];
    float d[NBD];
    int32_t s32[NBD * 8];
};
struct __attribute__((aligned(16))) LdsH {   /* q8(hidden) of this XCD's expert : I values */
    int8_t qs[I];
    float d[NBI];
    int32_t s16[NBI * 16];
};

__device__ inline FQ4K::X q4k_x_lds(const LdsX &x, int item) {
    const int b = item >> 2, g = item & 3;
    const u32x4 *p = reinterpret_cast<const u32x4 *>(x.qs + b * 256 + 64 * g);
    FQ4K::X r;
    r.a0 = p[0];
    r.a1 = p[1];
    r.b0 = p[2];
    r.b1 = p[3];
    r.s_lo = x.s32[b * 8 + 2 * g];
    r.s_hi = x.s32[b * 8 + 2 * g + 1];
    r.d = x.d[b];
    return r;
}

__device__ inline FQ6K::X q6k_x_lds(const LdsH &h, int item) {
    const int b = item >> 2, u = item & 3, hh = u >> 1, l0 = (u & 1) * 16;
    const int8_t *base = h.qs + b * 256 + 128 * hh + l0;
    FQ6K::X r;
    r.x0 = *reinterpret_cast<const u32x4 *>(base);
    r.x1 = *reinterpret_cast<const u32x4 *>(base + 32);
    r.x2 = *reinterpret_cast<const u32x4 *>(base + 64);
    r.x3 = *reinterpret_cast<const u32x4 *>(base + 96);
    const int sg = b * 16 + 8 * hh + (u & 1);
    r.s0 = h.s16[sg];
    r.s1 = h.s16[sg + 2];
    r.s2 = h.s16[sg + 4];
    r.s3 = h.s16[sg + 6];
    r.d = h.d[b];
    return r;
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

__device__ inline void put_slot(Buf sl, uint32_t slot, unsigned tag, float a, float b, float c) {
    u32x4 v;
    v.x = tag;
    v.y = __float_as_uint(a);
    v.z = __float_as_uint(b);
    v.w = __float_as_uint(c);
    __builtin_amdgcn_raw_buffer_store_b128(v, sl.r, (int)(slot * 16u), 0, CPOL_SC1);
}

/* Polls this communication lane's share of `total` slots (flat indices
 * cl, cl + CL, ...; slot(f) maps a flat index to a slot) until each carries
 * `tag`, handing every arrived slot to take(f, v).  All pending slots are
 * re-read as one batch per round.  Returns false if the wait timed out or
 * another workgroup aborted. */
template <int MAXP, class Slot, class Take>
__device__ inline bool poll_slots(Buf sl, int cl, int total, unsigned tag, unsigned *abort_flag, Slot slot, Take take) {
    uint32_t pending = 0;
#pragma unroll
    for (int i = 0; i < MAXP; i++)
        if (cl + CL * i < total) pending |= 1u << i;
    unsigned spins = 0;
    while (pending) {
        u32x4 v[MAXP];
#pragma unroll
        for (int i = 0; i < MAXP; i++)
            if (pending & (1u << i))
                v[i] = __builtin_amdgcn_raw_buffer_load_b128(sl.r, (int)(slot(cl + CL * i) * 16u), 0, CPOL_SC1);
#pragma unroll
        for (int i = 0; i < MAXP; i++)
            if ((pending & (1u << i)) && v[i].x == tag) {
                take(cl + CL * i, v[i]);
                pending &= ~(1u << i);
            }
        if (!pending) break;
        if ((++spins & 63) == 0 && __hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
            return false;
        if (spins > SPIN_LIMIT) {
            __hip_atomic_store(abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    return true;
}

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
    __shared__ float red[NA];
    __shared__ float aval[RA];
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

    typename FQ4K::W wg_[MAX_A], wu_[MAX_A];
    typename FQ6K::W wd_[MAX_B];
    u32x4 nw0, nw1;                              /* next layer's RMSNorm weight (compute lanes) */

    /* loads are unconditional so the registers' live ranges end at their
     * use; an inactive step reads through an empty descriptor (zeros, no
     * memory access) */
    auto load_a = [&](const DecodeLayer &ly) {
        const bool cw = wave < NW;
        Buf gb = make_buf_uniform(cw ? ly.gate[xe] : nullptr, cw ? (uint32_t)I * GATE_RB : 0u);
        Buf ub = make_buf_uniform(cw ? ly.up[xe] : nullptr, cw ? (uint32_t)I * GATE_RB : 0u);
#pragma unroll
        for (int i = 0; i < MAX_A; i++) {
            const int s = wave + i * NW;
            /* an out-of-range step reads past the rows (zeros) */
            const uint32_t r = s < STEPS_A ? (uint32_t)(RA * rk + 2 * s + (lane >> 5)) : (uint32_t)I;
            wg_[i] = FQ4K::load_w(gb, r * GATE_RB, lane & 31);
            wu_[i] = FQ4K::load_w(ub, r * GATE_RB, lane & 31);
        }
    };
    auto load_b = [&](const DecodeLayer &ly) {
        const bool cw = wave < NW;
        Buf db = make_buf_uniform(cw ? ly.down[xe] : nullptr, cw ? (uint32_t)D * DOWN_RB : 0u);
        const int item = (lane & 15) < NBI * 4 ? (lane & 15) : 0;
#pragma unroll
        for (int t = 0; t < MAX_B; t++) {
            const int q = wave + t * NW;
            const uint32_t r = q < STEPS_B ? (uint32_t)(RB * rk + 4 * q + (lane >> 4)) : (uint32_t)D;
            wd_[t] = FQ6K::load_w(db, r * DOWN_RB, item);
        }
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
        /* optional phase timestamps (100 MHz clock) of the first and last workgroup */
        const bool tw = times && threadIdx.x == 0 && (wg == 0 || wg == NWG - 1);
        uint64_t *tr = tw ? times + ((size_t)(wg == 0 ? 0 : 1) * L + l) * NTS : nullptr;
        if (tw) tr[0] = wall_clock64();
        /* ---- 1: gather h from the other ranks of this XCD ---- */
        if (l > 0) {
            if (cl >= 0) {
                const bool ok = poll_slots<6>(
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
                        if (VPS * t + 1 < RB) o[1] = __uint_as_float(v.z);
                        if (VPS * t + 2 < RB) o[2] = __uint_as_float(v.w);
                    });
                if (!ok) lds_fail = 1;
            } else {
                store_nw();
            }
            __syncthreads();
            if (lds_fail) return;
        }
        if (tw) tr[1] = wall_clock64();
        /* ---- 2: RMSNorm (weight norm_w or 1) then q8, in LDS; wave w owns block w ---- */
        {
            const u32x4 hv = reinterpret_cast<const u32x4 *>(hx)[threadIdx.x];
            float v0 = __uint_as_float(hv.x), v1 = __uint_as_float(hv.y);
            float v2 = __uint_as_float(hv.z), v3 = __uint_as_float(hv.w);
            const float ss = wave_sum(v0 * v0 + v1 * v1 + v2 * v2 + v3 * v3);
            if (lane == 0) red[wave] = ss;
        }
        __syncthreads();
        {
            float tot = 0.f;
#pragma unroll
            for (int i = 0; i < NA; i++) tot += red[i];
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
            reinterpret_cast<uint32_t *>(sx.qs)[threadIdx.x] = q;
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
        /* ---- 3: gate/up rows [24 rk, 24 rk + 24) of expert xe -> SwiGLU ---- */
        if (wave < NW) {
#pragma unroll
            for (int i = 0; i < MAX_A; i++) {
                const int s = wave + i * NW;
                const int item = lane & 31;
                FQ4K::X xs = q4k_x_lds(sx, item);
                float vg = FQ4K::value(wg_[i], xs, item);
                float vu = FQ4K::value(wu_[i], xs, item);
                vg = seg_sum_last<SA>(vg);
                vu = seg_sum_last<SA>(vu);
                if (s < STEPS_A && (lane & 31) == 31) aval[2 * s + (lane >> 5)] = silu_mul(vg, vu);
            }
            /* the next layer's gate/up rows load while this layer finishes */
            if (l + 1 < L) load_a(lys[l + 1]);
        }
        __syncthreads();
        if (tw) tr[3] = wall_clock64();
        /* ---- 4: all-gather the expert's hidden vector within the XCD ---- */
        if (cl >= 0) {
            if (clv < GS)
                put_slot(sl, GSL + (par * NWG + (uint32_t)wg) * GS + (uint32_t)clv, tag, aval[VPS * clv],
                         aval[VPS * clv + 1], aval[VPS * clv + 2]);
            if (clv < RA) hid[RA * rk + clv] = aval[clv];
            const bool ok = poll_slots<2>(
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
                });
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
            reinterpret_cast<uint32_t *>(sh.qs + b * 256)[lane] = q;
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
        /* ---- 6: down rows [64 rk, 64 rk + 64) of expert xe ---- */
        if (wave < NW) {
#pragma unroll
            for (int t = 0; t < MAX_B; t++) {
                const int q = wave + t * NW;
                const int item = lane & 15;
                float v = 0.f;
                if (item < NBI * 4) {
                    FQ6K::X xs = q6k_x_lds(sh, item);
                    v = FQ6K::value(wd_[t], xs, item);
                }
                v = seg_sum_last<SB>(v);
                if (q < STEPS_B && (lane & 15) == 15) pp[xe][4 * q + (lane >> 4)] = v;
            }
            /* the next layer's RMSNorm weight and down rows load while h travels */
            if (l + 1 < L) {
                load_nw(lys[l + 1]);
                load_b(lys[l + 1]);
            }
        }
        __syncthreads();
        if (tw) tr[6] = wall_clock64();
        /* ---- 7: cross-XCD hop: rank rk of every XCD trades its 64 down values ---- */
        if (cl >= 0) {
            if (clv < PS) {
                const int r0 = VPS * clv;
                put_slot(sl, PSL + (par * NWG + (uint32_t)wg) * PS + (uint32_t)clv, tag, pp[xe][r0],
                         r0 + 1 < RB ? pp[xe][r0 + 1] : 0.f, r0 + 2 < RB ? pp[xe][r0 + 2] : 0.f);
            }
            const bool ok = poll_slots<2>(
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
                });
            if (!ok) lds_fail = 1;
        }
        __syncthreads();
        if (lds_fail) return;
        if (tw) tr[7] = wall_clock64();
        /* ---- 8: combine rows [64 rk, 64 rk + 64) in expert order, publish ---- */
        if (cl >= 0 && clv < PS) {
            float o[VPS];
#pragma unroll
            for (int k = 0; k < VPS; k++) {
                const int rl = VPS * clv + k;
                if (rl < RB) {
                    float a = hx[RB * rk + rl];
#pragma unroll
                    for (int e = 0; e < NE; e++) a += ly.w[e] * pp[e][rl];
                    o[k] = a;
                    hx[RB * rk + rl] = a;
                    if (l == L - 1 && xe == 0) h[RB * rk + rl] = a;
                } else {
                    o[k] = 0.f;
                }
            }
            if (l + 1 < L) put_slot(sl, HSL + (par * NWG + (uint32_t)wg) * PS + (uint32_t)clv, tag, o[0], o[1], o[2]);
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
