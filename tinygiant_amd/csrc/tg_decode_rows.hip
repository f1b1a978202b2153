/*
 * tg_decode_rows.hip -- the persistent multi-row decode step: L planned
 * Qwen3-30B-A3B expert layers (D = 2048, I = 768, Q4_K gate/up, Q6_K down,
 * SiLU, no biases) over k = 2..16 rows of h in one cooperative launch of 256
 * workgroups.  Per layer it runs the chain tinygiant/engine.py:281-282,
 * 335-341 applies to the rows of forward_rows -- a verify pass of K + 1 rows
 * (tinygiant/specdec.py:66) or a prefill chunk (engine.py:213-217):
 *
 *   A  gate/up items (active expert, 16 rows of I), once the k rows of x are
 *      flagged: both dots and the SiLU product for every pair of the expert
 *      -> hidden[pair]
 *   B  down items (active expert, 64 rows of D), once the expert's hidden
 *      rows are there: their q8 into LDS, then w_pair * dot for every pair
 *      -> part[pair]
 *   C  workgroup r < k, row r, once its partials are there: h_r += them in
 *      expert order (k_moe_combine); x_r = RMSNorm(h_r) * w_{l+1}; q8(x_r)
 *
 * No barrier separates the phases: every value one workgroup writes and
 * another reads sits in a buffer of its layer as an 8-byte word {tag, value}
 * (hidden values, partials, the 4-byte units of the q8 rows of x), the tag
 * being the layer's in this launch, and the reader polls the words it needs until their tags
 * match (a lane reloads only the words whose tags did not).  A workgroup
 * thus waits only for what it reads: a down item for its expert's hidden
 * rows, a row's combine for the row's partials.
 *
 * Each workgroup takes a contiguous range of the layer's A items and one of
 * its B items (split on the host by an estimate of each item's time) and
 * streams them through registers: the next item's weight loads are in flight
 * while the current item computes, and a phase's first item is loaded before
 * the wait that opens the phase.  The per-row arithmetic is that of the
 * per-layer kernels the plans run (k_rms_norm_q8, k_moe_ax<FQ4K, 32>,
 * k_moe_bx<FQ6K, 16>, k_moe_combine): the step gives their bits.
 *
 * Exchanged data is stored with sc1, written through to memory, and loaded
 * with sc1, which takes no stale line from the reader's L2: the workgroups
 * sit on all 8 XCDs.  Tags grow by L per launch from a device word (the last
 * workgroup to leave advances it), so the node of a graph replays unchanged,
 * and every wait is bounded (a wait that runs out raises the abort word,
 * which releases the rest).
 */
#include <algorithm>
#include <vector>

#include "tg_decode.h"
#include "tg_kernels.h"
#include "tg_xchg.hpp"

namespace tg {
namespace {

constexpr int NT = 512, NWV = NT / 64;
constexpr int D = 2048, I = 768, NBX = D / 256, NBH = I / 256;
constexpr uint32_t GRB = 1152, DRB = 630;            /* Q4_K row of 2048 values, Q6_K row of 768 */
constexpr uint32_t GMB = I * GRB, DMB = D * DRB;     /* bytes of a gate (up) and of a down matrix */
constexpr int A_ROWS = 16, A_TILES = I / A_ROWS;     /* 8 waves x 2 rows of 32 lanes */
constexpr int B_PASS = 2, B_ROWS = 32 * B_PASS;      /* 8 waves x 4 rows of 16 lanes, twice */
constexpr int B_TILES = D / B_ROWS;
constexpr int B_ITEMS = 12;                          /* Q6_K items of a 768-value row */
constexpr uint32_t OOB = 0x80000000u;                /* past every buffer: reads zeros, touches nothing */
constexpr uint32_t XS = q8_lds_stride(NBX), HS = q8_lds_stride(NBH);
constexpr int NTS = 24;                              /* timing words per (workgroup, layer) */
static_assert(XS == 2848 && HS == 1072, "q8 LDS image");
static_assert(XS % 16 == 0, "the x image moves in 16-byte units");

__device__ inline void st1(Buf b, uint32_t off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), b.r, (int)off, 0, CPOL_SC1);
}
__device__ inline void st1(Buf b, uint32_t off, uint32_t v) {
    __builtin_amdgcn_raw_buffer_store_b32(v, b.r, (int)off, 0, CPOL_SC1);
}
__device__ inline u32x4 ld1x4(Buf b, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(b.r, (int)off, 0, CPOL_SC1);
}

/* ---- tagged words ----
 * A value another workgroup reads is stored as one 8-byte word {tag, value}
 * (the tag of its layer in this launch); the reader polls the words it
 * needs until every tag matches, so no store waits for its completion and
 * no barrier separates the phases. */
__device__ inline void st_tag(Buf b, uint32_t idx, unsigned tag, float v) {
    u32x2 w;
    w.x = tag;
    w.y = __float_as_uint(v);
    __builtin_amdgcn_raw_buffer_store_b64(w, b.r, (int)(idx * 8u), 0, CPOL_SC1);
}

/* a bounded poll round: false once the wait has run out or another
 * workgroup aborted (then the abort word is set) */
__device__ inline bool poll_more(unsigned &spins, unsigned *abort_flag) {
    if ((++spins & 63) == 0 && __hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return false;
    if (spins > SPIN_LIMIT) {
        __hip_atomic_store(abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
    }
    __builtin_amdgcn_s_sleep(1);
    return true;
}

/* ---- the layer's tables, staged in LDS ----
 * Values every lane of the workgroup reads alike come through LDS and
 * readfirstlane: a vector load from global memory here would return behind
 * the weight loads in flight (a CU returns its loads in order), and a
 * descriptor built from a VGPR would wrap every load in a waterfall loop. */
__device__ inline int ufl(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ inline const void *ufl_ptr(uint64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return (const void *)(uintptr_t)(((uint64_t)hi << 32) | lo);
}
struct Tab {
    const RowsExp *ex;
    const int *prow;
    const float *pw;
    const int *roff, *rpair;
};
__device__ inline Tab tab_view(const uint8_t *t, int n_act, int P, int k) {
    const int *pr = reinterpret_cast<const int *>(t + n_act * 32);
    return Tab{reinterpret_cast<const RowsExp *>(t), pr, reinterpret_cast<const float *>(pr + P), pr + 2 * P,
               pr + 2 * P + k + 1};
}
/* the layer's table (tab_bytes, 16-byte units) into LDS, one load a thread */
__device__ inline void tab_load(const RowsLayer &ly, uint8_t *dst) {
    const Buf b = make_buf(ly.tab, (uint32_t)ly.tab_bytes);
    if (threadIdx.x * 16 < (unsigned)ly.tab_bytes)
        *reinterpret_cast<u32x4 *>(dst + 16 * threadIdx.x) = ld16(b, threadIdx.x * 16u);
}

/* ---- items ---- */

struct WA {
    FQ4K::W g, u;
};
struct WB {
    FQ6K::W w[B_PASS];
};

/* gate/up row of A item `item` this lane's segment works on */
__device__ inline int a_row(int item, int wave, int lane) { return (item % A_TILES) * A_ROWS + 2 * wave + (lane >> 5); }
__device__ inline int b_row(int item, int q, int wave, int lane) {
    return (item % B_TILES) * B_ROWS + 32 * q + 4 * wave + (lane >> 4);
}

/* the weights of A item `item` (item < 0: out-of-range loads, zeros); tb
 * may be read from global memory (nothing in flight then) or LDS */
__device__ inline WA a_load(const Tab &tb, int item, int wave, int lane) {
    item = ufl(item);
    const int it = item < 0 ? 0 : item;
    const RowsExp &e = tb.ex[it / A_TILES];
    const uint32_t off = item < 0 ? OOB : (uint32_t)a_row(it, wave, lane) * GRB;
    const Buf gb = make_buf(ufl_ptr(e.gate), GMB), ub = make_buf(ufl_ptr(e.up), GMB);
    WA w;
    w.g = FQ4K::load_w(gb, off, lane & 31);
    w.u = FQ4K::load_w(ub, off, lane & 31);
    return w;
}
__device__ inline WB b_load(const Tab &tb, int item, int wave, int lane) {
    item = ufl(item);
    const int it = item < 0 ? 0 : item;
    const RowsExp &e = tb.ex[it / B_TILES];
    const int sl = lane & 15;
    const bool v = item >= 0 && sl < B_ITEMS;
    const Buf db = make_buf(ufl_ptr(e.down), DMB);
    WB w;
#pragma unroll
    for (int q = 0; q < B_PASS; q++)
        w.w[q] = FQ6K::load_w(db, v ? (uint32_t)b_row(it, q, wave, lane) * DRB : OOB, v ? sl : 0);
    return w;
}

/* ---- down items staged in LDS ----
 * A workgroup's first B_STAGE down items of a layer are copied into LDS
 * (direct-to-LDS copies, 1 KiB an instruction) at the end of the layer
 * before, while it waits for that layer's rows of x; the rest stream through
 * registers, one item ahead.  An item is 64 rows of 630 bytes, contiguous and
 * 16-byte aligned in the down matrix. */
constexpr int B_STAGE = 2;
constexpr int B_SLOT = B_ROWS * (int)DRB;            /* 40,320 bytes */
constexpr int B_COP = (B_SLOT + 1023) / 1024;        /* 40 copies, the last of 24 lanes */
constexpr int B_LAST = (B_SLOT - 1024 * (B_COP - 1)) / 16;
static_assert(B_SLOT % 16 == 0 && B_LAST > 0 && B_LAST <= 64, "whole 16-byte pieces");
/* copies of items i0 .. i0 + B_STAGE - 1 (those below i1) into the slots;
 * their count */
__device__ inline int b_stage(const Tab &tb, int i0, int i1, uint8_t *slots, int wave, int lane) {
    const int ns = ufl(i1 - i0 < B_STAGE ? i1 - i0 : B_STAGE);
    for (int t = 0; t < ns; t++) {
        const int item = i0 + t;
        const RowsExp &e = tb.ex[item / B_TILES];
        const u32x4 dd = buf_desc(ufl_ptr(e.down), DMB);
        const uint32_t src = (uint32_t)(item % B_TILES) * (uint32_t)B_SLOT + 16u * (uint32_t)lane;
        for (int c = wave; c < B_COP; c += NWV)
            if (c < B_COP - 1 || lane < B_LAST) copy_lanes(dd, src + 1024u * (uint32_t)c, lds_addr(slots + t * B_SLOT + 1024 * c));
    }
    return ns > 0 ? ns : 0;
}
/* 16, 8 and 4 bytes at LDS offset a (a even): the covering dwords from
 * a & ~3, shifted by a & 3 bytes (rows of 630 bytes and blocks of 210 put the
 * fields of odd rows and odd blocks at 2 mod 4) */
__device__ inline u32x4 lds_u16(const uint8_t *base, uint32_t a) {
    const uint32_t *p = reinterpret_cast<const uint32_t *>(base + (a & ~3u));
    const uint32_t sh = a & 3u;
    return u32x4{__builtin_amdgcn_alignbyte(p[1], p[0], sh), __builtin_amdgcn_alignbyte(p[2], p[1], sh),
                 __builtin_amdgcn_alignbyte(p[3], p[2], sh), __builtin_amdgcn_alignbyte(p[4], p[3], sh)};
}
__device__ inline u32x2 lds_u8(const uint8_t *base, uint32_t a) {
    const uint32_t *p = reinterpret_cast<const uint32_t *>(base + (a & ~3u));
    const uint32_t sh = a & 3u;
    return u32x2{__builtin_amdgcn_alignbyte(p[1], p[0], sh), __builtin_amdgcn_alignbyte(p[2], p[1], sh)};
}
/* the f16 at LDS offset a (a even) in the high half, as load_w's d word */
__device__ inline uint32_t lds_f16_hi(const uint8_t *base, uint32_t a) {
    const uint32_t v = *reinterpret_cast<const uint32_t *>(base + (a & ~3u));
    return (a & 2u) ? (v & 0xFFFF0000u) : (v << 16);
}
/* the lane's weights of a staged item: FQ6K::load_w's bytes, from LDS */
__device__ inline WB b_lds(const uint8_t *slot, int wave, int lane) {
    const int sl = lane & 15, it = sl < B_ITEMS ? sl : 0;
    const uint32_t u = (uint32_t)it & 3u, h = u >> 1, l0 = (u & 1u) * 16u;
    WB w;
#pragma unroll
    for (int q = 0; q < B_PASS; q++) {
        const uint32_t pr = (uint32_t)(32 * q + 4 * wave + (lane >> 4)) * DRB + (uint32_t)(it >> 2) * 210u;
        w.w[q].qla = lds_u16(slot, pr + 64u * h + l0);
        w.w[q].qlb = lds_u16(slot, pr + 64u * h + 32u + l0);
        w.w[q].qh = lds_u16(slot, pr + 128u + 32u * h + l0);
        w.w[q].sc = lds_u8(slot, pr + 192u + 8u * h);
        w.w[q].d = lds_f16_hi(slot, pr + 208u);
    }
    return w;
}

/* gate/up + SiLU of every pair of the item's expert (k_moe_ax's sums) */
__device__ inline void a_compute(const Tab &tb, int item, const WA &w, const uint8_t *xl, Buf hid, unsigned tag,
                                 float *dbg_hid, int wave, int lane) {
    item = ufl(item);
    const int s = item / A_TILES, p0 = ufl(tb.ex[s].p0), np = ufl(tb.ex[s].np);
    const int r = a_row(item, wave, lane), sl = lane & 31;
    const FQ4K::Wd g = FQ4K::decode(w.g, sl), u = FQ4K::decode(w.u, sl);
    for (int j = 0; j < np; j++) {
        const int p = p0 + j;
        const Q8Lds xr = q8_lds_slot(xl, NBX, ufl(tb.prow[p]));
        const FQ4K::X x = FQ4K::load_x(xr, sl);
        float ag = 0.f, au = 0.f;
        ag += FQ4K::value_d(g, x);
        au += FQ4K::value_d(u, x);
        const float vg = seg_sum_x<32>(ag), vu = seg_sum_x<32>(au);
        if (sl == 0) {
            const float hv = act_fn(TG_ACT_SILU, vg, vu);
            st_tag(hid, (uint32_t)(p * I + r), tag, hv);
            if (dbg_hid) dbg_hid[p * I + r] = hv;
        }
    }
}

/* tags of a loaded 16-byte unit: two tagged words */
__device__ inline bool tagged(const u32x4 &v, unsigned tag) { return v.x == tag && v.z == tag; }

/* q8 of the expert's hidden rows into LDS slots 0..np-1, one 256-block per
 * wave (q8_quant_rows_lds's arithmetic), once every value carries the
 * layer's tag: a lane reloads only the units whose tags did not match; false
 * if the wait ran out */
__device__ inline bool b_hidden_q8(int p0, int np, Buf hid, unsigned tag, unsigned *abort_flag, uint8_t *hl, int wave,
                                   int lane) {
    constexpr int BATCH = 4;
    const int nblk = np * NBH;
    for (int u0 = wave; u0 < nblk; u0 += NWV * BATCH) {
        u32x4 raw[BATCH][2];
        uint32_t off[BATCH];
        bool got[BATCH];
#pragma unroll
        for (int i = 0; i < BATCH; i++) {
            const int u = u0 + i * NWV;
            const int s = u / NBH, b = u % NBH;
            off[i] = u < nblk ? (uint32_t)((p0 + s) * I + b * 256 + 4 * lane) * 8u : OOB;
            raw[i][0] = ld1x4(hid, off[i]);
            raw[i][1] = ld1x4(hid, off[i] == OOB ? OOB : off[i] + 16u);
            got[i] = u >= nblk;
        }
        unsigned spins = 0;
        while (true) {
            bool in = true;
#pragma unroll
            for (int i = 0; i < BATCH; i++) {
                got[i] = got[i] || (tagged(raw[i][0], tag) && tagged(raw[i][1], tag));
                in &= got[i];
            }
            if (__ballot(!in) == 0) break;
            if (!poll_more(spins, abort_flag)) return false;
#pragma unroll
            for (int i = 0; i < BATCH; i++)
                if (!got[i]) {
                    raw[i][0] = ld1x4(hid, off[i]);
                    raw[i][1] = ld1x4(hid, off[i] + 16u);
                }
        }
#pragma unroll
        for (int i = 0; i < BATCH; i++) {
            const int u = u0 + i * NWV;
            if (u >= nblk) continue;   /* uniform per wave */
            const int s = u / NBH, b = u % NBH;
            const Q8Quant q = q8_block_quant_dpp(__uint_as_float(raw[i][0].y), __uint_as_float(raw[i][0].w),
                                                 __uint_as_float(raw[i][1].y), __uint_as_float(raw[i][1].w));
            uint8_t *slot = hl + (size_t)s * HS;
            reinterpret_cast<uint32_t *>(slot + b * 256)[lane] = q.packed;
            if ((lane & 3) == 0) reinterpret_cast<int32_t *>(slot + NBH * 288)[b * 16 + (lane >> 2)] = q.s16;
            if ((lane & 7) == 0) reinterpret_cast<int32_t *>(slot + NBH * 256)[b * 8 + (lane >> 3)] = q.s32;
            if (lane == 0) reinterpret_cast<float *>(slot + NBH * 352)[b] = q.sc;
        }
    }
    return true;
}

/* down rows of every pair of the item's expert, weighted (k_moe_bx's sums) */
__device__ inline void b_compute(const Tab &tb, int item, const WB &w, const uint8_t *hl, Buf part, unsigned tag,
                                 int wave, int lane) {
    item = ufl(item);
    const int s = item / B_TILES, p0 = ufl(tb.ex[s].p0), np = ufl(tb.ex[s].np);
    const int sl = lane & 15;
    FQ6K::Wd wd[B_PASS];
#pragma unroll
    for (int q = 0; q < B_PASS; q++) wd[q] = FQ6K::decode(w.w[q], sl);
    for (int j = 0; j < np; j++) {
        const int p = p0 + j;
        const Q8Lds xr = q8_lds_slot(hl, NBH, j);
        const float pw = __int_as_float(ufl(__float_as_int(tb.pw[p])));
        const FQ6K::X x = FQ6K::load_x(xr, sl < B_ITEMS ? sl : 0);
#pragma unroll
        for (int q = 0; q < B_PASS; q++) {
            float acc = 0.f;
            if (sl < B_ITEMS) acc += FQ6K::value_d(wd[q], x);
            const float v = seg_sum_x<16>(acc);
            if (sl == 0) st_tag(part, (uint32_t)(p * D + b_row(item, q, wave, lane)), tag, pw * (v + 0.f));
        }
    }
}

/* Items i0 .. i1-1 through two register sets: item i + 1's loads are issued
 * before item i computes (pre(i, its registers) runs before that issue).
 * s0 holds item i0's loads on entry.  The loop has one exit and no register
 * copies, so the compiler's waits for the loads stay partial. */
template <class W, class Load, class Pre, class Comp>
__device__ inline void pipe(int i0, int i1, W s0, Load load, Pre pre, Comp comp) {
    const int n = i1 - i0;
    W s1;
    int j = 0;
    for (; j + 2 <= n; j += 2) {
        pre(i0 + j, s0);
        s1 = load(i0 + j + 1);
        __builtin_amdgcn_sched_barrier(0);
        comp(i0 + j, s0);
        pre(i0 + j + 1, s1);
        s0 = load(i0 + j + 2 < i1 ? i0 + j + 2 : -1);
        __builtin_amdgcn_sched_barrier(0);
        comp(i0 + j + 1, s1);
    }
    if (j < n) {
        pre(i0 + j, s0);
        comp(i0 + j, s0);
    }
}

/* Phase C for workgroup r < k: layer ly's combine of row r (ly non-null),
 * then the RMSNorm (weight nx->norm_w) and q8 of the row for layer nx (when
 * non-null), thread t owning values 4t .. 4t+3 as k_rms_norm_q8's lane t % 64
 * of wave t / 64 does.  The q8 row goes out as tagged words: byte o of row
 * r's LDS image is the value half of the word at byte 2 o of row r's 2 XS
 * bytes.  False if a wait for a partial ran out. */
__device__ inline void st_x(Buf xb, uint32_t o, unsigned tag, uint32_t v) {
    u32x2 w;
    w.x = tag;
    w.y = v;
    __builtin_amdgcn_raw_buffer_store_b64(w, xb.r, (int)(2u * o), 0, CPOL_SC1);
}
__device__ inline bool phase_c(const RowsLayer *ly, const Tab *tb, const RowsLayer *nx, int r, float *h, float eps,
                               float *red, uint8_t *rec_next, unsigned tag, unsigned next_tag, unsigned *abort_flag,
                               int wave, int lane, uint64_t *ts) {
    const int t = threadIdx.x;
    const Buf hb = make_buf(h + (size_t)r * D, D * 4u);
    __builtin_amdgcn_s_waitcnt(0x0F70);   /* vmcnt(0): the previous layer's store of these values is done */
    const u32x4 hv = ld1x4(hb, (uint32_t)t * 16u);
    float o[4] = {__uint_as_float(hv.x), __uint_as_float(hv.y), __uint_as_float(hv.z), __uint_as_float(hv.w)};
    /* the next layer's RMSNorm weights, loaded now: after the partials they
     * would add a memory round trip to every layer */
    float nw[4] = {1.f, 1.f, 1.f, 1.f};
    if (nx && nx->norm_w) {
        const u32x4 wv = ld16(make_buf(nx->norm_w, D * 4u), (uint32_t)t * 16u);
        nw[0] = __uint_as_float(wv.x);
        nw[1] = __uint_as_float(wv.y);
        nw[2] = __uint_as_float(wv.z);
        nw[3] = __uint_as_float(wv.w);
    }
    bool good = true;   /* a wave whose wait ran out goes on (the barriers below count every wave) */
    if (ly) {
        /* row r's partials, up to eight pairs at a time; a lane reloads only
         * the units whose tags did not match; added in expert order */
        const Buf pb = make_buf(ly->part, (uint32_t)ly->P * D * 8u);
        const int q0 = ufl(tb->roff[r]), q1 = ufl(tb->roff[r + 1]);
        for (int qb = q0; qb < q1; qb += 8) {
            u32x4 v[8][2];
            uint32_t off[8];
            bool got[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                off[i] = qb + i < q1 ? (uint32_t)(ufl(tb->rpair[qb + i]) * D + 4 * t) * 8u : OOB;
                v[i][0] = ld1x4(pb, off[i]);
                v[i][1] = ld1x4(pb, off[i] == OOB ? OOB : off[i] + 16u);
                got[i] = qb + i >= q1;
            }
            unsigned spins = 0;
            while (good) {
                bool in = true;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    got[i] = got[i] || (tagged(v[i][0], tag) && tagged(v[i][1], tag));
                    in &= got[i];
                }
                if (__ballot(!in) == 0) break;
                good = poll_more(spins, abort_flag);
#pragma unroll
                for (int i = 0; i < 8; i++)
                    if (!got[i]) {
                        v[i][0] = ld1x4(pb, off[i]);
                        v[i][1] = ld1x4(pb, off[i] + 16u);
                    }
            }
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (qb + i < q1) {
                    o[0] += __uint_as_float(v[i][0].y);
                    o[1] += __uint_as_float(v[i][0].w);
                    o[2] += __uint_as_float(v[i][1].y);
                    o[3] += __uint_as_float(v[i][1].w);
                }
        }
        if (ts) ts[6] = wall_clock64();   /* the partials are in (wave 0) */
        u32x4 ov;
        ov.x = __float_as_uint(o[0]);
        ov.y = __float_as_uint(o[1]);
        ov.z = __float_as_uint(o[2]);
        ov.w = __float_as_uint(o[3]);
        __builtin_amdgcn_raw_buffer_store_b128(ov, hb.r, (int)(t * 16u), 0, CPOL_SC1);
    }
    if (!nx) return good;
    if (rec_next) reinterpret_cast<float4 *>(rec_next + (size_t)r * D * 4)[t] = make_float4(o[0], o[1], o[2], o[3]);
    /* RMSNorm: the lane's squares in order, the wave's butterfly, the waves' sum in order */
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < 4; c++) ss += o[c] * o[c];
    ss = wave_sum_x(ss);
    if (lane == 0) red[wave] = ss;
    bar_lds();
    if (ts) ts[7] = wall_clock64();   /* every wave's squares are in */
    float tot = 0.f;
    for (int i = 0; i < NWV; i++) tot += red[i];
    const float scale = 1.f / sqrtf(tot / (float)D + eps);
    float x[4];
#pragma unroll
    for (int c = 0; c < 4; c++) x[c] = (o[c] * scale) * nw[c];
    if (rec_next)
        reinterpret_cast<float4 *>(rec_next + (size_t)(nx->k + r) * D * 4)[t] = make_float4(x[0], x[1], x[2], x[3]);
    /* q8 of block `wave` into row r's tagged image */
    const Q8Quant q = q8_block_quant_dpp(x[0], x[1], x[2], x[3]);
    const Buf xb = make_buf(nx->xq + (size_t)r * 2 * XS, 2 * XS);
    const int b = wave;
    st_x(xb, (uint32_t)(b * 256 + 4 * lane), next_tag, q.packed);
    if ((lane & 3) == 0) st_x(xb, (uint32_t)(NBX * 288 + (b * 16 + (lane >> 2)) * 4), next_tag, (uint32_t)q.s16);
    if ((lane & 7) == 0) st_x(xb, (uint32_t)(NBX * 256 + (b * 8 + (lane >> 3)) * 4), next_tag, (uint32_t)q.s32);
    if (lane == 0) st_x(xb, (uint32_t)(NBX * 352 + b * 4), next_tag, __float_as_uint(q.sc));
    return good;
}

/* the k tagged q8 rows of layer ly's x into LDS, each wave polling its own
 * units (a lane reloads only those whose tags did not match); false in the
 * waves whose wait ran out */
__device__ inline bool x_load(const RowsLayer &ly, int k, unsigned tag, unsigned *abort_flag, uint8_t *xl) {
    constexpr int XU = (ROWS_MAXK * (XS / 8) + NT - 1) / NT;   /* 16-byte units (2 tagged words) a thread */
    const uint32_t nu = (uint32_t)k * (XS / 8);
    const Buf xg = make_buf(ly.xq, nu * 16u);
    u32x4 v[XU];
    bool got[XU];
#pragma unroll
    for (int i = 0; i < XU; i++) {
        const uint32_t m = threadIdx.x + i * NT;
        v[i] = ld1x4(xg, m < nu ? m * 16u : OOB);
        got[i] = m >= nu;
    }
    unsigned spins = 0;
    while (true) {
        bool in = true;
#pragma unroll
        for (int i = 0; i < XU; i++) {
            got[i] = got[i] || tagged(v[i], tag);
            in &= got[i];
        }
        if (__ballot(!in) == 0) break;
        if (!poll_more(spins, abort_flag)) return false;
#pragma unroll
        for (int i = 0; i < XU; i++)
            if (!got[i]) v[i] = ld1x4(xg, (threadIdx.x + i * NT) * 16u);
    }
#pragma unroll
    for (int i = 0; i < XU; i++) {
        const uint32_t m = threadIdx.x + i * NT;
        if (m < nu) {
            u32x2 w;
            w.x = v[i].y;
            w.y = v[i].w;
            *reinterpret_cast<u32x2 *>(xl + 8 * m) = w;
        }
    }
    return true;
}

__global__ __launch_bounds__(NT) void k_decode_rows(const RowsLayer *__restrict__ layers, int L, float *h,
                                                    void *slots, unsigned *sync, float eps, uint8_t *debug,
                                                    uint64_t *times, unsigned *place, int pol) {
    (void)slots;
    (void)pol;
    __shared__ __attribute__((aligned(16))) uint8_t xl[ROWS_MAXK * XS];   /* q8 rows of x */
    __shared__ __attribute__((aligned(16))) uint8_t hl[ROWS_MAXK * HS];   /* q8 hidden rows of one expert */
    __shared__ __attribute__((aligned(16))) uint8_t tabs[2][ROWS_TAB_BYTES];   /* layer tables, by parity */
    __shared__ __attribute__((aligned(16))) uint8_t bst[B_STAGE * B_SLOT];     /* staged down items */
    __shared__ float red[NWV];
    __shared__ unsigned s_base;
    /* a wait ran out, one word per kind of wait (x, B, C): each only goes
     * from 1 to 0, and is read after the barrier that follows its writes */
    __shared__ int s_okx, s_okb, s_okc;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, wg = blockIdx.x;
    unsigned *abort_flag = sync;
    if (threadIdx.x == 0) {
        s_okx = s_okb = s_okc = 1;
        s_base = read_epoch(sync);
        if (place) {
            unsigned xcc;
            asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
            place[wg] = xcc;
        }
    }
    tab_load(layers[0], tabs[0]);
    bar_lds();
    const unsigned base = s_base;
    const int k = layers[0].k;
    bool ok = true;

    /* C(-1): the first layer's RMSNorm and q8 */
    if (wg < k)
        phase_c(nullptr, nullptr, &layers[0], wg, h, eps, red, debug, 0u, base + 1u, abort_flag, wave, lane, nullptr);
    WA a0;
    int nsb;   /* down items of the layer staged in bst */
    {
        const RowsLayer &ly = layers[0];
        const Tab tb = tab_view(tabs[0], ly.n_act, ly.P, ly.k);
        const int i0 = ly.split[wg], i1 = ly.split[wg + 1];
        a0 = a_load(tb, i0 < i1 ? i0 : -1, wave, lane);
        nsb = b_stage(tb, ly.split[ROWS_GRID + 1 + wg], ly.split[ROWS_GRID + 2 + wg], bst, wave, lane);
    }

    for (int l = 0; l < L && ok; l++) {
        const RowsLayer &ly = layers[l];
        const unsigned tag = base + 1u + (unsigned)l;   /* this layer's tag in this launch */
        const Tab tb = tab_view(tabs[l & 1], ly.n_act, ly.P, ly.k);
        const bool tw = times && threadIdx.x == 0;
        uint64_t *tr = times ? times + ((size_t)wg * L + l) * NTS : nullptr;
        uint8_t *rec = debug ? debug + (size_t)l * ly.rec_bytes : nullptr;
        const int ia0 = ly.split[wg], ia1 = ly.split[wg + 1];
        const int ib0 = ly.split[ROWS_GRID + 1 + wg], ib1 = ly.split[ROWS_GRID + 2 + wg];
        const Buf hid = make_buf(ly.hidden, (uint32_t)ly.P * I * 8u);
        /* ---- A ---- */
        {
            if (tw) tr[8] = wall_clock64();   /* the wait for x starts */
            if (!x_load(ly, k, tag, abort_flag, xl)) s_okx = 0;
            bar_lds();
            if (s_okx == 0) {
                ok = false;
                break;
            }
            if (tw) tr[0] = wall_clock64();
            float *dh = rec ? reinterpret_cast<float *>(rec + (size_t)2 * k * D * 4) : nullptr;
            pipe(
                ia0, ia1, a0, [&](int i) { return a_load(tb, i, wave, lane); }, [](int, const WA &) {},
                [&](int i, const WA &w) { a_compute(tb, i, w, xl, hid, tag, dh, wave, lane); });
        }
        if (tw) tr[1] = wall_clock64();
        /* ---- B: each expert's hidden rows are polled when its first item
         * starts; the first nsb items are in bst (every wave's copies have
         * landed once it has waited for them and passed the barrier in pre) ---- */
        {
            wait_copies();
            const int ibr = ib0 + nsb;   /* the first item through registers */
            WB b0 = b_load(tb, ibr < ib1 ? ibr : -1, wave, lane);
            const Buf part = make_buf(ly.part, (uint32_t)ly.P * D * 8u);
            int cur = -1;   /* expert whose q8 hidden rows hl holds */
            bool bok = true;
            auto pre = [&](int i, const WB &) {
                const int s = ufl(i) / B_TILES;
                if (s != cur) {
                    bar_lds();   /* every wave is done with the previous rows */
                    const bool got =
                        b_hidden_q8(ufl(tb.ex[s].p0), ufl(tb.ex[s].np), hid, tag, abort_flag, hl, wave, lane);
                    if (!got) s_okb = 0;   /* every wave that gave up says so */
                    bar_lds();
                    bok &= s_okb != 0;
                    if (tw && cur < 0) tr[2] = wall_clock64();
                    cur = s;
                }
            };
            for (int t = 0; t < nsb; t++) {
                pre(ib0 + t, b0);   /* the first turn passes a barrier */
                const WB w = b_lds(bst + t * B_SLOT, wave, lane);
                b_compute(tb, ib0 + t, w, hl, part, tag, wave, lane);
            }
            pipe(
                ibr, ib1, b0, [&](int i) { return b_load(tb, i, wave, lane); }, pre,
                [&](int i, const WB &w) { b_compute(tb, i, w, hl, part, tag, wave, lane); });
            if (!bok) {
                ok = false;
                break;
            }
        }
        if (tw) tr[3] = wall_clock64();
        /* ---- C ---- */
        const bool more = l + 1 < L;
        if (wg < k) {
            const bool got = phase_c(&ly, &tb, more ? &layers[l + 1] : nullptr, wg, h, eps, red,
                                     debug && more ? debug + (size_t)(l + 1) * ly.rec_bytes : nullptr, tag, tag + 1u,
                                     abort_flag, wave, lane, tw ? tr : nullptr);
            if (!got) s_okc = 0;
            if (tw) tr[4] = wall_clock64();
            bar_lds();
            if (s_okc == 0) {
                ok = false;
                break;
            }
        }
        if (tw) tr[5] = wall_clock64();
        if (!more) break;
        {
            /* the next layer's table, then its first gate/up item in flight
             * while the rows of x are awaited */
            const RowsLayer &nl = layers[l + 1];
            tab_load(nl, tabs[(l + 1) & 1]);
            bar_lds();
            const Tab nt = tab_view(tabs[(l + 1) & 1], nl.n_act, nl.P, nl.k);
            const int i0 = nl.split[wg], i1 = nl.split[wg + 1];
            a0 = a_load(nt, i0 < i1 ? i0 : -1, wave, lane);
            /* the slots were last read before the barrier above */
            nsb = b_stage(nt, nl.split[ROWS_GRID + 1 + wg], nl.split[ROWS_GRID + 2 + wg], bst, wave, lane);
        }
    }
    wait_copies();
    /* the last workgroup to finish advances the launch epoch by L (every
     * workgroup read it before taking its ticket) and clears the ticket word */
    if (threadIdx.x == 0 &&
        __hip_atomic_fetch_add(sync + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1) {
        __hip_atomic_store(sync + 2, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(sync + 1, base + (unsigned)L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace

int decode_rows_max_grid() {
    int dev = 0, per_cu = 0;
    hipDeviceProp_t pr;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&pr, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *)k_decode_rows, NT, 0) != hipSuccess)
        return 0;
    return per_cu * pr.multiProcessorCount;
}

hipError_t launch_decode_rows(const RowsLayer *layers_dev, int L, float *h_dev, unsigned *sync_dev, float eps,
                              uint8_t *debug_dev, uint64_t *times_dev, unsigned *place_dev, bool cooperative,
                              hipStream_t st) {
    void *slots = nullptr;
    int pol = 1;
    void *args[] = {(void *)&layers_dev, (void *)&L,         (void *)&h_dev,     (void *)&slots,
                    (void *)&sync_dev,   (void *)&eps,       (void *)&debug_dev, (void *)&times_dev,
                    (void *)&place_dev,  (void *)&pol};
    if (cooperative)
        return hipLaunchCooperativeKernel((const void *)k_decode_rows, dim3(ROWS_GRID), dim3(NT), args, 0, st);
    return hipLaunchKernel((const void *)k_decode_rows, dim3(ROWS_GRID), dim3(NT), args, 0, st);
}

const void *decode_rows_fn() { return (const void *)k_decode_rows; }
int decode_rows_threads() { return NT; }

/* Item ranges of one layer.  Each active expert gets workgroups and its
 * items are split evenly over them, so a workgroup works on one expert per
 * phase: a down item that starts another expert would first wait a memory
 * round trip for that expert's hidden rows.  A workgroup's time in a phase is
 * about its items x an item's cost, fitted on per-workgroup phase times of
 * 48-layer steps: an A item 0.91 us + 0.34 us a pair of its expert, a B item
 * 0.90 us + 0.38 us a pair after the expert's hidden rows are in.  The split
 * takes the smallest such time every expert can meet within the workgroups
 * (items a workgroup = floor(T / cost), at least one), then hands the
 * workgroups left over, one at a time, to the expert whose workgroups take
 * longest.  Proportional shares rounded to whole workgroups had left some
 * workgroups of the busiest experts one item over the rest (k = 5, 9 rows:
 * 1,373-1,376 and 1,990-1,994 us a 48-layer pass against 1,283-1,295 and
 * 1,812-1,820); a floor under the cost of an item (a CU's share of the
 * weight stream, 1.5 us) moved workgroups off the busiest experts and was
 * slower (1,342-1,357 and 1,908-1,916).  The down items
 * skip workgroups 0 .. c - 1, which combine the rows: they start a row's
 * combine as soon as its last partial lands. */
static void split_phase(const int *np, int n_act, int tiles, int w0, double c1, int *s) {
    const int G = ROWS_GRID - w0;
    std::vector<int> wgs(n_act, 1);
    if (n_act > 0 && n_act <= G) {
        std::vector<double> c(n_act);
        for (int e = 0; e < n_act; e++) c[e] = 1.0 + c1 * np[e];   /* in units of an item without pairs */
        /* workgroups each expert needs so that none takes longer than T */
        auto need = [&](double T, std::vector<int> &w) {
            long tot = 0;
            for (int e = 0; e < n_act; e++) {
                const int m = std::min(tiles, (int)(T / c[e] + 1e-9));
                if (m < 1) return false;
                w[e] = (tiles + m - 1) / m;
                tot += w[e];
            }
            return tot <= G;
        };
        std::vector<double> cand;
        for (int e = 0; e < n_act; e++)
            for (int m = 1; m <= tiles; m++) cand.push_back(m * c[e]);
        std::sort(cand.begin(), cand.end());
        size_t lo = 0, hi = cand.size() - 1;   /* the largest candidate needs one workgroup an expert */
        std::vector<int> w(n_act);
        while (lo < hi) {
            const size_t mid = (lo + hi) / 2;
            if (need(cand[mid], w)) hi = mid;
            else lo = mid + 1;
        }
        need(cand[lo], wgs);
        int used = 0;
        for (int e = 0; e < n_act; e++) used += wgs[e];
        for (; used < G; used++) {
            int best = -1;
            double bt = -1.0;
            for (int e = 0; e < n_act; e++) {
                const double t = ((tiles + wgs[e] - 1) / wgs[e]) * c[e];
                if (wgs[e] < tiles && t > bt) {
                    bt = t;
                    best = e;
                }
            }
            if (best < 0) break;
            wgs[best]++;
        }
    }
    int w = w0;
    for (int i = 0; i <= w0; i++) s[i] = 0;
    for (int e = 0; e < n_act; e++)
        for (int j = 0; j < wgs[e] && w < ROWS_GRID; j++) s[++w] = e * tiles + (int)((int64_t)tiles * (j + 1) / wgs[e]);
    while (w < ROWS_GRID) {
        s[w + 1] = s[w];
        w++;
    }
    s[ROWS_GRID] = n_act * tiles;
}

void decode_rows_split(const int *np, int n_act, int c, int *split) {
    split_phase(np, n_act, A_TILES, 0, 0.34 / 0.91, split);
    split_phase(np, n_act, B_TILES, c, 0.38 / 0.90, split + ROWS_GRID + 1);
}

}  // namespace tg
