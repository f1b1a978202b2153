/*
 * tg_decode.hip -- persistent single-launch expert decode step for one token.
 *
 * One cooperative launch runs every layer of the step
 *     h <- h + sum_e w_e * down_e( q8( act(gate_e . q8(RMSNorm h), up_e . q8(RMSNorm h)) ) )
 * (tinygiant/engine.py:281-282,335-341 per layer; the expert math is
 * moe_phase_a / moe_phase_b of csrc/libtinygiant.c:1279-1384 for k = 1).
 *
 * Layout: one workgroup of NW compute waves (+1) per CU, all co-resident.
 * Each layer is two phases:
 *   A  every workgroup rebuilds q8(RMSNorm(h)) in LDS, then its waves compute
 *      gate/up rows (two rows per wave step for Q4_K, D = 2048) and write the
 *      activated hidden values;
 *   B  every workgroup re-quantizes all experts' hidden rows into LDS, then for
 *      each group of four output rows wave e computes expert e's down rows;
 *      the workgroup adds them to h in expert order (the reference's combine
 *      order, csrc/libtinygiant.c:1428-1434) and writes h.
 * Each phase's weights are loaded into registers as soon as the previous
 * phase has published its results, so the weight stream overlaps the
 * exchange that the next phase waits for.
 *
 * Workgroups exchange h and the hidden values through epoch-tagged 16-byte
 * slots written and polled with device-scope coherent vector accesses; a
 * ninth wave per workgroup does the polling, so it never waits behind the
 * compute waves' outstanding weight loads.  Every wait is bounded and a
 * timed-out wait raises an abort flag that releases every other waiter, so
 * the grid always drains.
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
constexpr int SA = 32;                /* lanes per gate/up row: 8 blocks x 4 items */
constexpr int SB = 16;                /* lanes per down row: 3 blocks x 4 items = 12 used */
constexpr int MAX_A = 2;              /* gate/up wave steps per wave per layer */
constexpr int MAX_RG = 2;             /* down row groups per workgroup per layer */
constexpr int MAX_B = 3;              /* (row group, expert) down items per wave per layer */
constexpr int HS = 3;                 /* h slots per workgroup (8 rows, 3 values a slot) */
constexpr int GS = 8;                 /* hidden slots per workgroup (<= 24 values) */
constexpr int MAXPOLL = 16;           /* slots one communication lane polls */
constexpr unsigned SPIN_LIMIT = 1u << 20;
constexpr int MAX_LAYERS = 64;        /* layer descriptors staged in LDS */
constexpr int NE = DECODE_MAXE;       /* active experts per layer (top-8 at k = 1) */
constexpr int NWG = DECODE_GRID;      /* workgroups: one per CU */
constexpr int PER_WG_A = NE * (I / 2) / NWG;   /* gate/up wave steps per workgroup: 12 */
static_assert(NE * (I / 2) % NWG == 0, "gate/up steps divide over the grid");
static_assert(PER_WG_A <= NW * MAX_A, "gate/up steps fit the waves");
static_assert(2 * PER_WG_A <= 3 * GS, "hidden values fit the slots");
static_assert(D / 4 <= MAX_RG * NWG && D / 4 > NWG, "row groups: two per workgroup");
static_assert(MAX_RG * NE <= NW * MAX_B, "down items fit the waves");
constexpr int NTS = 16;               /* timestamps per layer */

/* A slot is 16 bytes {tag, v0, v1, v2} written and read as one vector access
 * with device-scope coherence (sc1), so the tag and its values arrive
 * together; consumers poll the tag of the epoch they need. */
constexpr int CPOL_SC1 = 16;

/* ---- LDS images of q8 rows ---- */
struct __attribute__((aligned(16))) LdsX {   /* q8(RMSNorm(h)) : D values */
    int8_t qs[D];
    float d[NBD];
    int32_t s32[NBD * 8];
};
struct __attribute__((aligned(16))) LdsH {   /* q8(hidden_e) for every expert : I values each */
    int8_t qs[DECODE_MAXE][I];
    float d[DECODE_MAXE][NBI];
    int32_t s16[DECODE_MAXE][NBI * 16];
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

__device__ inline FQ6K::X q6k_x_lds(const LdsH &h, int e, int item) {
    const int b = item >> 2, u = item & 3, hh = u >> 1, l0 = (u & 1) * 16;
    const int8_t *base = h.qs[e] + b * 256 + 128 * hh + l0;
    FQ6K::X r;
    r.x0 = *reinterpret_cast<const u32x4 *>(base);
    r.x1 = *reinterpret_cast<const u32x4 *>(base + 32);
    r.x2 = *reinterpret_cast<const u32x4 *>(base + 64);
    r.x3 = *reinterpret_cast<const u32x4 *>(base + 96);
    const int sg = b * 16 + 8 * hh + (u & 1);
    r.s0 = h.s16[e][sg];
    r.s1 = h.s16[e][sg + 2];
    r.s2 = h.s16[e][sg + 4];
    r.s3 = h.s16[e][sg + 6];
    r.d = h.d[e][b];
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

/* Polls `count` slots (this lane's share, slot indices first, first + CL, ...)
 * until each carries `tag`, handing every arrived slot to `take`.  All
 * pending slots are re-read as one batch per round.  Returns false if the
 * wait timed out or another workgroup aborted. */
template <class Take>
__device__ inline bool poll_slots(Buf sl, uint32_t slot_base, int first, int count, unsigned tag, unsigned *abort_flag,
                                  Take take) {
    uint32_t pending = (1u << count) - 1u;   /* count <= MAXPOLL < 32 */
    unsigned spins = 0;
    while (pending) {
        u32x4 v[MAXPOLL];
#pragma unroll
        for (int i = 0; i < MAXPOLL; i++)
            if (pending & (1u << i))
                v[i] = __builtin_amdgcn_raw_buffer_load_b128(sl.r, (int)((slot_base + first + CL * i) * 16), 0,
                                                             CPOL_SC1);
#pragma unroll
        for (int i = 0; i < MAXPOLL; i++)
            if ((pending & (1u << i)) && v[i].x == tag) {
                take(first + CL * i, v[i]);
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

/* Slot layout (u32x4 each, double buffered by layer parity):
 *   hslots [2][grid][HS]  rows of h written by phase B (8 rows per workgroup)
 *   gslots [2][grid][GS]  hidden values written by phase A (<= 24 per workgroup)
 * tags are base + 2 * layer + phase + 1, so a launch never mistakes a slot
 * of an earlier epoch for its own. */
__global__ __launch_bounds__(NT) void k_decode_qwen(const DecodeLayer *__restrict__ layers, int L, float *h,
                                                    u32x4 *slots, unsigned *abort_flag, unsigned base, float eps,
                                                    uint8_t *dbg, uint64_t *times) {
    __shared__ __attribute__((aligned(16))) float hx[D];          /* this layer's input h */
    __shared__ __attribute__((aligned(16))) float nws[D];         /* this layer's RMSNorm weight */
    __shared__ __attribute__((aligned(16))) float hid[DECODE_MAXE][I];
    __shared__ LdsX sx;
    __shared__ LdsH sh;
    __shared__ float red[NA];
    __shared__ float part[MAX_RG][DECODE_MAXE][4];
    __shared__ float aval[3 * GS];
    __shared__ float hout[3 * HS];
    __shared__ int lds_fail;
    __shared__ DecodeLayer lys[MAX_LAYERS];

    constexpr int nwg = NWG;
    int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int cl = (int)threadIdx.x - NW * 64;   /* communication lane, valid when >= 0 */
    if (threadIdx.x == 0) lds_fail = 0;
    const int wg = blockIdx.x;
    const uint32_t hs_base = 0, gs_base = 2u * nwg * HS;
    Buf sl = make_buf(slots, (uint32_t)(2u * nwg * (HS + GS) * 16u));

    typename FQ4K::W wg_[MAX_A], wu_[MAX_A];
    typename FQ6K::W wd_[MAX_B];

    /* phase A steps: (expert, pair of rows); PER_WG_A consecutive steps a workgroup */
    auto a_step = [&](const DecodeLayer &, int i, int &e, int &r) -> bool {
        const int local = wave + i * NW;
        const int s = wg * PER_WG_A + local;
        if (wave >= NW || local >= PER_WG_A) return false;
        e = s / (I / 2);
        r = (s % (I / 2)) * 2 + (lane >> 5);
        return true;
    };
    /* loads are unconditional so the registers' live ranges end at their
     * use; an inactive step reads through an empty descriptor (zeros, no
     * memory access) */
    auto load_a = [&](const DecodeLayer &ly) {
#pragma unroll
        for (int i = 0; i < MAX_A; i++) {
            int e = 0, r = 0;
            const bool act = a_step(ly, i, e, r);
            const uint32_t nb = act ? (uint32_t)I * GATE_RB : 0u;
            Buf gb = make_buf(act ? ly.gate[e] : nullptr, nb);
            Buf ub = make_buf(act ? ly.up[e] : nullptr, nb);
            wg_[i] = FQ4K::load_w(gb, (uint32_t)r * GATE_RB, lane & 31);
            wu_[i] = FQ4K::load_w(ub, (uint32_t)r * GATE_RB, lane & 31);
        }
    };
    /* phase B: row groups rg = wg + i * grid (4 rows each, i < MAX_RG); the
     * (row group, expert) items are spread over the compute waves */
    auto nrg = [&]() { return wg + nwg < D / 4 ? 2 : 1; };
    auto b_item = [&](const DecodeLayer &, int t, int &i, int &e) -> bool {
        const int it = wave + t * NW;
        if (wave >= NW || it >= nrg() * NE) return false;
        i = it / NE;
        e = it % NE;
        return true;
    };
    auto load_b = [&](const DecodeLayer &ly) {
#pragma unroll
        for (int t = 0; t < MAX_B; t++) {
            int i = 0, e = 0;
            const bool act = b_item(ly, t, i, e);
            const int item = (lane & 15) < NBI * 4 ? (lane & 15) : 0;
            const int r = (wg + i * nwg) * 4 + (lane >> 4);
            Buf db = make_buf(act ? ly.down[e] : nullptr, act ? (uint32_t)D * DOWN_RB : 0u);
            wd_[t] = FQ6K::load_w(db, (uint32_t)r * DOWN_RB, item);
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
    load_a(lys[0]);

    for (int l = 0; l < L; l++) {
        const DecodeLayer &ly = lys[l];
        const unsigned par = (unsigned)(l & 1);
        /* an opaque copy of the communication lane keeps the slot address and
         * scatter arithmetic inside the loop instead of hoisted (and live)
         * across every layer */
        int clv = cl;
        asm volatile("" : "+v"(clv));
        asm volatile("" : "+v"(lane));
        /* optional phase timestamps (100 MHz clock) of the first and last workgroup */
        const bool tw = times && threadIdx.x == 0 && (wg == 0 || wg == nwg - 1);
        uint64_t *tr = tw ? times + ((size_t)(wg == 0 ? 0 : 1) * L + l) * NTS : nullptr;
        if (tw) tr[0] = wall_clock64();
        /* ---- phase A: collect h from the previous layer's phase B ---- */
        if (l > 0) {
            if (cl >= 0) {
                const unsigned tag = base + 2u * (unsigned)(l - 1) + 2u;
                const int total = nwg * HS;
                const int cnt = total > clv ? (total - clv + CL - 1) / CL : 0;
                const bool ok = poll_slots(sl, hs_base + ((par ^ 1u) * nwg * HS), clv, cnt, tag, abort_flag,
                                           [&](int s, const u32x4 &v) {
                                               const int p = s / HS, j = s % HS;
                                               const float vv[3] = {__uint_as_float(v.y), __uint_as_float(v.z),
                                                                    __uint_as_float(v.w)};
#pragma unroll
                                               for (int k = 0; k < 3; k++) {
                                                   const int q = 3 * j + k;
                                                   const int rg = p + (q >> 2) * nwg;
                                                   if (q < 8 && rg < D / 4) hx[rg * 4 + (q & 3)] = vv[k];
                                               }
                                           });
                if (!ok) lds_fail = 1;
            }
            __syncthreads();
            if (lds_fail) return;
        }
        /* the RMSNorm weight reaches LDS through the communication waves (the
         * compute waves keep only weight loads in flight) */
        const float *nw = ly.norm_w;
        if (nw) {
            if (cl >= 0)
                for (int t = cl; t < D / 4; t += CL)
                    reinterpret_cast<u32x4 *>(nws)[t] = reinterpret_cast<const u32x4 *>(nw)[t];
            __syncthreads();
        }
        if (tw) tr[1] = wall_clock64();
        /* RMSNorm (weight 1 or norm_w) then q8, all in LDS; wave w owns block w */
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
            const int c = threadIdx.x * 4;
            const u32x4 hv = reinterpret_cast<const u32x4 *>(hx)[threadIdx.x];
            const float v0 = (__uint_as_float(hv.x) * scale) * (nw ? nws[c] : 1.f);
            const float v1 = (__uint_as_float(hv.y) * scale) * (nw ? nws[c + 1] : 1.f);
            const float v2 = (__uint_as_float(hv.z) * scale) * (nw ? nws[c + 2] : 1.f);
            const float v3 = (__uint_as_float(hv.w) * scale) * (nw ? nws[c + 3] : 1.f);
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
        /* gate/up rows of this workgroup */
#pragma unroll
        for (int i = 0; i < MAX_A; i++) {
            int e, r;
            const bool act = a_step(ly, i, e, r);
            float vg = 0.f, vu = 0.f;
            if (act) {
                const int item = lane & 31;
                FQ4K::X xs = q4k_x_lds(sx, item);
                vg = FQ4K::value(wg_[i], xs, item);
                vu = FQ4K::value(wu_[i], xs, item);
            }
            if (tw && i == 0) tr[8] = wall_clock64();
            vg = seg_sum_last<SA>(vg);
            vu = seg_sum_last<SA>(vu);
            if (tw && i == 0) tr[9] = wall_clock64();
            if (act && (lane & 31) == 31) aval[2 * (wave + i * NW) + (lane >> 5)] = silu_mul(vg, vu);
        }
        __syncthreads();
        if (tw) tr[3] = wall_clock64();
        /* publish: GS slots of 3 values (workgroup-local value order) */
        if (threadIdx.x < GS) {
            u32x4 v;
            v.x = base + 2u * (unsigned)l + 1u;   /* slots past 2 * PER_WG_A values carry no data */
            v.y = __float_as_uint(aval[3 * threadIdx.x]);
            v.z = __float_as_uint(aval[3 * threadIdx.x + 1]);
            v.w = __float_as_uint(aval[3 * threadIdx.x + 2]);
            __builtin_amdgcn_raw_buffer_store_b128(v, sl.r, (int)((gs_base + (par * nwg + wg) * GS + threadIdx.x) * 16),
                                                   0, CPOL_SC1);
        }
        /* ---- phase B: fetch the down rows while the hidden values travel ---- */
        if (wave < NW) load_b(ly);
        if (cl >= 0) {
            const unsigned tag = base + 2u * (unsigned)l + 1u;
            const int total = nwg * GS;
            const int cnt = total > clv ? (total - clv + CL - 1) / CL : 0;
            const bool ok = poll_slots(sl, gs_base + par * nwg * GS, clv, cnt, tag, abort_flag,
                                       [&](int s, const u32x4 &v) {
                                           const int p = s / GS, j = s % GS;
                                           const float vv[3] = {__uint_as_float(v.y), __uint_as_float(v.z),
                                                                __uint_as_float(v.w)};
#pragma unroll
                                           for (int k = 0; k < 3; k++) {
                                               const int q = 3 * j + k;      /* value index in producer p */
                                               const int loc = q >> 1;
                                               const int st = p * PER_WG_A + loc;
                                               if (loc < PER_WG_A)
                                                   hid[st / (I / 2)][(st % (I / 2)) * 2 + (q & 1)] = vv[k];
                                           }
                                       });
            if (!ok) lds_fail = 1;
        }
        __syncthreads();
        if (lds_fail) return;
        if (tw) tr[4] = wall_clock64();
        /* q8 of every expert's hidden row: NBI blocks per expert, one wave per block */
        for (int blk = wave; blk < NE * NBI; blk += NA) {
            const int e = blk / NBI, b = blk % NBI;
            const u32x4 hv = reinterpret_cast<const u32x4 *>(&hid[e][b * 256])[lane];
            const uint32_t q = q8_block_wave(__uint_as_float(hv.x), __uint_as_float(hv.y), __uint_as_float(hv.z),
                                             __uint_as_float(hv.w), lane, &sh.d[e][b], nullptr, &sh.s16[e][b * 16]);
            reinterpret_cast<uint32_t *>(sh.qs[e] + b * 256)[lane] = q;
            if (dbg && wg == 0) {
                uint8_t *rec = dbg + (size_t)l * DecodeDebug::BYTES;
                reinterpret_cast<u32x4 *>(rec + DecodeDebug::HID + (e * I + b * 256) * 4)[lane] = hv;
                reinterpret_cast<uint32_t *>(rec + DecodeDebug::HQ + e * I + b * 256)[lane] = q;
            }
        }
        __syncthreads();
        if (tw) tr[5] = wall_clock64();
        if (dbg && wg == 0) {
            uint8_t *rec = dbg + (size_t)l * DecodeDebug::BYTES;
            if (threadIdx.x < DECODE_MAXE * NBI)
                reinterpret_cast<float *>(rec + DecodeDebug::HD)[threadIdx.x] = (&sh.d[0][0])[threadIdx.x];
            for (int t = threadIdx.x; t < DECODE_MAXE * NBI * 16; t += NT)
                reinterpret_cast<int32_t *>(rec + DecodeDebug::HS16)[t] = (&sh.s16[0][0])[t];
        }
        /* down rows of every (row group, expert) item, then the combine in
         * expert order */
#pragma unroll
        for (int t = 0; t < MAX_B; t++) {
            int i, e;
            const bool act = b_item(ly, t, i, e);
            const int item = lane & 15;
            float v = 0.f;
            if (act && item < NBI * 4) {
                FQ6K::X xs = q6k_x_lds(sh, e, item);
                v = FQ6K::value(wd_[t], xs, item);
            }
            v = seg_sum_last<SB>(v);
            if (act && (lane & 15) == 15) part[i][e][lane >> 4] = v;
        }
        __syncthreads();
        if ((int)threadIdx.x < 4 * nrg()) {
            const int i = threadIdx.x >> 2, t4 = threadIdx.x & 3;
            const int r = (wg + i * nwg) * 4 + t4;
            float o = hx[r];
#pragma unroll
            for (int e = 0; e < NE; e++) o += ly.w[e] * part[i][e][t4];
            hout[threadIdx.x] = o;
            if (l == L - 1) h[r] = o;
        }
        __syncthreads();
        if (tw) tr[6] = wall_clock64();
        /* publish this workgroup's h rows for the next layer */
        if (l + 1 < L && threadIdx.x < HS) {
            u32x4 v;
            v.x = base + 2u * (unsigned)l + 2u;
            v.y = __float_as_uint(hout[3 * threadIdx.x]);
            v.z = __float_as_uint(hout[3 * threadIdx.x + 1]);
            v.w = __float_as_uint(hout[3 * threadIdx.x + 2]);
            __builtin_amdgcn_raw_buffer_store_b128(v, sl.r, (int)((hs_base + (par * nwg + wg) * HS + threadIdx.x) * 16),
                                                   0, CPOL_SC1);
        }
        /* the next layer's gate/up rows load while h travels */
        if (l + 1 < L && wave < NW) load_a(lys[l + 1]);
        if (tw) tr[7] = wall_clock64();
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

size_t decode_qwen_slot_bytes(int grid) { return (size_t)2 * grid * (HS + GS) * 16; }

hipError_t launch_decode_qwen(const DecodeLayer *layers_dev, int L, float *h_dev, void *slots_dev,
                              unsigned *abort_dev, unsigned base, float eps, uint8_t *debug_dev, uint64_t *times_dev,
                              int grid, hipStream_t st) {
    void *args[] = {(void *)&layers_dev, (void *)&L, (void *)&h_dev, (void *)&slots_dev, (void *)&abort_dev,
                    (void *)&base, (void *)&eps, (void *)&debug_dev, (void *)&times_dev};
    return hipLaunchCooperativeKernel((const void *)k_decode_qwen, dim3(grid), dim3(NT), args, 0, st);
}

}  // namespace tg
