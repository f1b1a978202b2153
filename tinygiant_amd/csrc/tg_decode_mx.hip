/*
 * tg_decode_mx.hip -- persistent single-launch expert decode step for the
 * gpt-oss-120b expert shape: one token, D = I = 2880, top-4 MXFP4 experts
 * with gate/up/down biases and the clamped SwiGLU, every layer
 *     h <- h + sum_e w_e * (down_e(q8(act(gate_e . q8(x) + bg, up_e . q8(x) + bu))) + bd)
 * with x = RMSNorm(h) (tinygiant/engine.py:281-282,335-341 per layer; the
 * expert math is moe_phase_a / moe_phase_b of csrc/libtinygiant.c:1279-1384
 * for k = 1, the MXFP4 dot of :533-547, the activation of :1250-1257).
 *
 * Placement.  256 workgroups, one per CU; workgroup g runs on XCD x = g % 8
 * as rank j = g / 8 of 32.  The layer's expert e is computed by XCDs 2e and
 * 2e + 1: its 64 ranks R = 32 (x & 1) + j each own the 45-row slice
 * [45 R, 45 R + 45) of the expert's gate, up and down rows.  Per layer:
 *   1  gather h: each XCD's 32 ranks all-gather the 64 slices of h (rank j
 *      of every XCD holds slices j and 32 + j, see 8)
 *   2  RMSNorm + q8 of h, then the fp8 halves of q8(x) for the MFMA, in LDS
 *   3  gate/up rows of the slice on block-scaled MFMA, the K range split
 *      over the six compute waves (the partial sums are added in wave order)
 *   4  bias + activation -> 45 hidden values; the expert's 64 ranks (two
 *      XCDs) all-gather its 2880 hidden values
 *   5  q8 of the hidden vector and its fp8 halves
 *   6  down rows of the slice on MFMA -> w_e * (down + bias)
 *   7  cross-XCD hop: rank j of every XCD trades its 45 weighted down values,
 *      so each holds all four experts' values for slices j and 32 + j
 *   8  h[r] += the four experts' values in expert order (the reference's
 *      combine order, csrc/libtinygiant.c:1428-1434), published for step 1.
 * The MXFP4 blocks go straight from memory into the MFMA's A operand: a
 * lane's 17 bytes are one block's e8m0 scale and its 16 code bytes, which the
 * MFMA takes as 32 e2m1 values under that scale.  q8(x) enters as two fp8
 * columns of the B operand, x = 16 (x >> 4) + (x & 15) (both halves exact in
 * e4m3, column scales 16 and 1), so the products are exact and each block's
 * integer sum is the reference's; the f32 additions are grouped differently
 * (four blocks inside an MFMA, then per 128 values, per half and per wave),
 * which the f32 bar covers.
 *
 * Every weight byte streams through one LDS region by direct-to-LDS copies
 * (1 KiB an instruction, aligned 16-byte pieces): a CU returns its vector
 * loads in issue order, so each batch is issued right after an exchange and
 * drains during the compute that follows, not ahead of the next poll:
 *   this layer's down rows (one contiguous 45-row range) after the h gather
 *   (1), gathered into registers during the hidden exchange (4);
 *   the next layer's gate segments (each compute wave the 272-byte pieces of
 *   its own K range, one contiguous range of the wave-segment layout made
 *   when the step is created, into its own part of the region) at q8 of the
 *   hidden vector (5), moved into registers at the hop (7);
 *   the next layer's up segments, the same way, at the hop (7), moved into
 *   registers at the next layer's start.
 * Two communication waves per workgroup publish; the two gathers are polled
 * by all eight waves (one or two slots a lane), the hop by the communication
 * waves.
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

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int NW = 6;                 /* compute waves per workgroup */
constexpr int NC = 2;                 /* communication waves per workgroup */
constexpr int NA = NW + NC;
constexpr int NT = NA * 64;
constexpr int CL = NC * 64;           /* communication lanes */
constexpr int D = 2880;               /* gpt-oss-120b: D = I = 2880 */
constexpr int NBLK = D / 32;          /* MXFP4 blocks per row: 90 */
constexpr int RB = NBLK * 17;         /* bytes per MXFP4 row: 1530 */
constexpr int NQ = (D + 255) / 256;   /* q8 blocks per row: 12, the last holds 64 values */
constexpr int NCH = (NBLK + 3) / 4;   /* 128-value MFMA chunks per row: 23 */
constexpr int NSB = 4 * NCH;          /* block slots of the fp8 images (two past the row stay zero) */
constexpr int NE = DECODE_MX_E;       /* active experts per layer */
constexpr int NWG = DECODE_GRID;
constexpr int NX = 8;                 /* XCDs; workgroup g runs on XCD g % NX */
constexpr int NR = NWG / NX;          /* ranks per XCD: 32 */
constexpr int NRK = 2 * NR;           /* ranks per expert (two XCDs): 64 */
constexpr int RS = D / NRK;           /* rows per rank slice: 45 */
constexpr int NG = 3;                 /* 16-row MFMA groups per slice */
constexpr int CPW = 4;                /* chunks per compute wave */
constexpr int VPS = 3;                /* values per slot */
constexpr int SS = RS / VPS;          /* slots per slice: 15 */
constexpr int HS = 2 * SS + 2;        /* h slots per rank: two slices and their sums of h^2 */
constexpr int MAX_LAYERS = 64;
constexpr int NTS = 24;               /* timing words per layer */
constexpr int FMT_FP8 = 0, FMT_FP4 = 4, SCALE_1 = 127, SCALE_16 = 131;
constexpr uint32_t OOB = 0x80000000u;  /* past every buffer: reads zeros, touches no memory */
constexpr int NDMA = 68;               /* 1 KiB direct-to-LDS copy steps of the down rows (16 bytes a lane) */
/* Gate and up matrices arrive in a wave-segment layout made when the step
 * is created (launch_mx_wave_segments): for each 45-row rank slice, compute
 * wave w's 16 blocks [16 w, 16 w + 16) of every row (272 bytes; the last
 * wave's 10 blocks, 170 bytes, at a 176-byte stride) lie contiguous and
 * 16-byte aligned, so a wave copies its segments as one range. */
constexpr int SEGB = 16 * 17;                          /* a wave's segment of one row: 272 bytes */
constexpr int SEGL = (NBLK - 16 * (NW - 1)) * 17;      /* the last wave's: 170 bytes */
constexpr int SEGLS = (SEGL + 15) & ~15;               /* its stride: 176 */
constexpr int WSB = RS * SEGB;                         /* a wave's range of one slice: 12,240 bytes */
constexpr int SLB = (NW - 1) * WSB + RS * SEGLS;       /* one slice: 69,120 bytes */
constexpr uint32_t MXSEG_BYTES = (uint32_t)NRK * SLB;  /* one rewritten matrix: 4,423,680 bytes */
constexpr int GINS = (WSB + 1023) / 1024;              /* copy steps of a wave's segments: 12 */
constexpr int GINSL = (RS * SEGLS + 1023) / 1024;      /* the last wave's: 8 */
constexpr int GREG = GINS * 1024;                      /* LDS bytes of a wave's segments */
constexpr int DZERO = NW * GREG;       /* 32 zero bytes after the copies, read by off-slice lanes */
constexpr int DWS = DZERO + 32;        /* LDS staging of the slice's gate rows, then its down rows */
static_assert(RS * RB + 15 <= NDMA * 1024 && NDMA * 1024 <= DZERO, "the slice's down rows fit the staging");
static_assert(NBLK > 16 * (NW - 1) && NBLK <= 16 * NW && WSB % 16 == 0 && SLB % 16 == 0, "wave segments");
static_assert(NE * 2 == NX, "two XCDs per expert");
static_assert(NRK * RS == D && RS % VPS == 0 && NG * 16 >= RS && RS <= 64, "slices");
static_assert(NW * CPW >= NCH && (NW - 1) * CPW < NCH, "chunks per wave");
static_assert((NR - 1) * HS <= 8 * CL && (NRK - 1) * SS <= 8 * CL && (NX - 1) * SS <= CL, "poll shares");
static_assert(NQ <= 2 * NA && NQ > NA, "q8 blocks: one or two per wave");
static_assert(D / 4 <= 2 * NW * 64, "RMSNorm weight: two float4 per compute lane");

/* slot regions (u32x4 index), each double buffered by layer parity:
 *   h slices  [2][NWG][HS]   slices j and 32 + j of the layer output, sums of h^2
 *   hidden    [2][NWG][SS]   the rank's 45 hidden values
 *   parts     [2][NWG][SS]   the rank's 45 weighted down values */
constexpr uint32_t HSL = 0, GSL = 2u * NWG * HS, PSL = GSL + 2u * NWG * SS, NSLOTS = PSL + 2u * NWG * SS;

/* Per byte of n (each 0..15), entry n of a 16-byte table t0..t3 (entries
 * 4i..4i+3 in ti, low byte first), by byte permutes. */
__device__ inline uint32_t lut16(uint32_t n, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
    const uint32_t idx = n & 0x07070707u;
    const uint32_t a = __builtin_amdgcn_perm(t1, t0, idx), b = __builtin_amdgcn_perm(t3, t2, idx);
    const uint32_t sel = ((n >> 3) & 0x01010101u) * 0xFFu;
    return (a & ~sel) | (b & sel);
}
/* fp8 e4m3 codes of the halves of four packed q8 values q (-127..127):
 * hi = q >> 4 (-8..7) and lo = q & 15 (0..15), both exact.  With u = q + 128
 * per byte, hi is entry u >> 4 of {-8..7} and lo entry u & 15 of {0..15}. */
__device__ inline void e4m3_halves(uint32_t q4, uint32_t &hi, uint32_t &lo) {
    const uint32_t u = q4 ^ 0x80808080u;
    hi = lut16((u >> 4) & 0x0F0F0F0Fu, 0xCACCCED0u, 0xB8C0C4C8u, 0x44403800u, 0x4E4C4A48u);
    lo = lut16(u & 0x0F0F0F0Fu, 0x44403800u, 0x4E4C4A48u, 0x53525150u, 0x57565554u);
}

/* One MXFP4 block as an MFMA A operand: e8m0 byte (low byte of e) and the
 * 16 code bytes. */
struct MxBlk {
    uint32_t e;
    u32x4 c;
};

/* LDS image of one q8 row for the MFMA: per 32-value block, the fp8 codes of
 * hi = x >> 4 and lo = x & 15 in MFMA K order (byte 2t holds value t, byte
 * 2t + 1 value 16 + t), plus the q8 scale of each 256-value block. */
struct __attribute__((aligned(16))) LdsQ {
    uint8_t sp[NSB][2][32];
    float d[NQ];
};

/* q8 of one 256-value block held by a wave (lane l: values 4l..4l+3, zeros
 * past the row), quantize_q8 (csrc/libtinygiant.c:169-208) in the arithmetic
 * of k_quantize_q8, written as fp8 halves into block slots 8b .. 8b + 7 of q.
 * Lanes l and l + 4 hold values t and 16 + t of the same 32-block, which the
 * MFMA K order interleaves; lane l (l % 8 < 4) writes both. */
__device__ inline void q8_split_block(float v0, float v1, float v2, float v3, int lane, int b, LdsQ &q,
                                      uint32_t *dbg_q = nullptr, float *dbg_d = nullptr) {
    const float amax = wave_max(fmaxf(fmaxf(fabsf(v0), fabsf(v1)), fmaxf(fabsf(v2), fabsf(v3))));
    const float inv = amax > 0.f ? 127.f / amax : 0.f;
    const int q0 = (int)__builtin_rintf(v0 * inv), q1 = (int)__builtin_rintf(v1 * inv);
    const int q2 = (int)__builtin_rintf(v2 * inv), q3 = (int)__builtin_rintf(v3 * inv);
    uint32_t hi, lo;
    e4m3_halves((uint32_t)(q0 & 0xFF) | ((uint32_t)(q1 & 0xFF) << 8) | ((uint32_t)(q2 & 0xFF) << 16) |
                    ((uint32_t)(q3 & 0xFF) << 24),
                hi, lo);
    const uint32_t hi2 = (uint32_t)__shfl_down((int)hi, 4, 64), lo2 = (uint32_t)__shfl_down((int)lo, 4, 64);
    const int blk = 8 * b + (lane >> 3), pos = 8 * (lane & 7);
    if ((lane & 7) < 4 && blk < NSB) {   /* the last q8 block ends inside block slot 91 */
        /* values t = 4 (l % 8) + i at bytes 2t, values 16 + t at bytes 2t + 1 */
        auto inter = [](uint32_t a, uint32_t c, int half) {
            const uint32_t s = 16u * (uint32_t)half;
            const uint32_t a0 = (a >> s) & 0xFFu, a1 = (a >> (s + 8u)) & 0xFFu;
            const uint32_t c0 = (c >> s) & 0xFFu, c1 = (c >> (s + 8u)) & 0xFFu;
            return a0 | (c0 << 8) | (a1 << 16) | (c1 << 24);
        };
        uint32_t *ph = reinterpret_cast<uint32_t *>(&q.sp[blk][0][pos]);
        uint32_t *pl = reinterpret_cast<uint32_t *>(&q.sp[blk][1][pos]);
        ph[0] = inter(hi, hi2, 0);
        ph[1] = inter(hi, hi2, 1);
        pl[0] = inter(lo, lo2, 0);
        pl[1] = inter(lo, lo2, 1);
    }
    if (lane == 0) q.d[b] = amax / 127.f;
    if (dbg_q) {   /* debug record: the block's quants, four per lane, and its scale */
        dbg_q[64 * b + lane] = (uint32_t)(q0 & 0xFF) | ((uint32_t)(q1 & 0xFF) << 8) | ((uint32_t)(q2 & 0xFF) << 16) |
                               ((uint32_t)(q3 & 0xFF) << 24);
        if (lane == 0) dbg_d[b] = amax / 127.f;
    }
}

/* The B operand of chunk c for this lane: column 0 holds the fp8 hi halves of
 * q8(x), column 1 the lo halves, columns 2..15 zeros.  Lane l supplies
 * column l % 16 for K group g = l / 16: bytes 0..15 are values 16 g .. 16 g
 * + 15 of the chunk and bytes 16..31 values 64 + 16 g .. in MFMA K order. */
__device__ inline v8i load_b(const LdsQ &q, int c, int lane) {
    const int g = lane >> 4, col = lane & 15, part = col == 1 ? 1 : 0;
    const int b0 = 4 * c + (g >> 1), b1 = b0 + 2, o = 16 * (g & 1);
    const u32x4 x0 = *reinterpret_cast<const u32x4 *>(&q.sp[b0][part][o]);
    const u32x4 x1 = *reinterpret_cast<const u32x4 *>(&q.sp[b1][part][o]);
    const int on = col < 2 ? -1 : 0;
    return v8i{(int)x0.x & on, (int)x0.y & on, (int)x0.z & on, (int)x0.w & on,
               (int)x1.x & on, (int)x1.y & on, (int)x1.z & on, (int)x1.w & on};
}

/* acc += d * (block-scaled A . B) for one chunk, one MFMA: column 0 is the
 * hi half under scale 16, column 1 the lo half under scale 1 (sb is the
 * lane's B scale); the two columns are added in the row reduction. */
__device__ inline void mma_chunk(const MxBlk &a, const v8i &bx, int sb, float d, v4f &acc) {
    const v8i av = v8i{(int)a.c.x, (int)a.c.y, (int)a.c.z, (int)a.c.w, 0, 0, 0, 0};
    const int e = (int)(a.e & 0xFFu);
    const v4f z = {0.f, 0.f, 0.f, 0.f};
    const v4f r = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bx, z, FMT_FP4, FMT_FP8, 0, e, 0, sb);
    acc[0] += d * r[0];
    acc[1] += d * r[1];
    acc[2] += d * r[2];
    acc[3] += d * r[3];
}

}  // namespace

/* Tags are base + layer + 1 in every region, so a launch never mistakes a
 * slot of an earlier layer or launch for its own.  A slot of parity p is
 * rewritten two layers later only after every reader of it has published
 * something the writer waited for in between. */
__global__ __launch_bounds__(NT) void k_decode_mx(const DecodeLayerMx *__restrict__ layers, int L, float *h,
                                                  u32x4 *slots, unsigned *abort_flag, float eps,
                                                  uint8_t *dbg, uint64_t *times, unsigned *place, int pol) {
    __shared__ __attribute__((aligned(16))) float hx[D];      /* this layer's h */
    __shared__ __attribute__((aligned(16))) float nws[D];     /* this layer's RMSNorm weight */
    __shared__ __attribute__((aligned(16))) float hid[D];     /* the expert's hidden vector */
    __shared__ LdsQ sx, sh;                                   /* fp8 images of q8(x) and q8(hidden) */
    __shared__ float ssq[NRK];                                /* sum of h^2 of each 45-row slice */
    /* per-wave partial row sums, hi and lo columns: red[unit][row][wave][column],
     * so a row's twelve partials are three 16-byte LDS reads */
    __shared__ __attribute__((aligned(16))) float red[2 * NG][16][NW][2];
    __shared__ float pp[NX][RS];                              /* weighted down values of the 8 XCDs */
    __shared__ __attribute__((aligned(16))) uint8_t dws[DWS]; /* staged gate rows, then down rows, of the slice */
    __shared__ int lds_fail;
    __shared__ DecodeLayerMx lys[MAX_LAYERS];

    int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int cl = (int)threadIdx.x - NW * 64;   /* communication lane, valid when >= 0 */
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
    const int xc = wg % NX, rk = wg / NX;        /* XCD and rank in it */
    const int xe = xc >> 1, R = NR * (xc & 1) + rk;   /* expert slot and rank in the expert */
    Buf sl = make_buf(slots, NSLOTS * 16u);
    const int sb = (lane & 15) == 0 ? SCALE_16 : SCALE_1;   /* B scale of this lane's column */

    MxBlk wa[CPW][2 * NG];   /* gate (units 0..2) and up (3..5) blocks of the wave's chunks */
    MxBlk wb[CPW][NG];       /* down blocks, gathered from dws during the hidden exchange */
    u32x4 nw0, nw1;          /* next layer's RMSNorm weight (compute lanes) */

    /* Gate and up rows: compute wave w uses blocks [16 w, 16 w + 16) of each
     * of the slice's 45 rows.  In the wave-segment layout they are one
     * aligned range, which the wave copies into its own region of dws with
     * direct-to-LDS loads and later gathers into registers: no other wave
     * touches the region, so only the wave's own copy has to have landed,
     * and the wave can copy the next matrix in as soon as it has gathered
     * the last one.  An inactive call reads through an empty descriptor
     * (zeros). */
    const int ginsw = wave == NW - 1 ? GINSL : GINS;
    const uint32_t segst = wave == NW - 1 ? (uint32_t)SEGLS : (uint32_t)SEGB;
    auto fetch_seg = [&](const uint8_t *mat, bool on) {
        const u32x4 desc = buf_desc(on ? mat : nullptr, on ? MXSEG_BYTES : 0u);
        const uint32_t a0 = (uint32_t)R * SLB + (uint32_t)wave * WSB;
        for (int k = 0; k < ginsw; k++) copy_1k(desc, a0 + 1024u * (uint32_t)k, lds_addr(dws + GREG * wave + 1024 * k), lane);
    };
    /* The slice's down rows are one contiguous 45-row range of the expert's
     * down matrix.  The compute waves copy it into dws with direct-to-LDS
     * loads, 1 KiB an instruction and 16 bytes a lane, from the 16-byte
     * boundary at or below its start (dsh bytes earlier); the buffer range
     * returns zeros past the matrix.  Issued right after the h gather, the
     * copy drains during RMSNorm and gate/up, not ahead of the hidden
     * exchange's polls, and takes no registers. */
    const uint32_t dsh = (uint32_t)(RS * R * RB) & 15u;
    auto fetch_down = [&](const DecodeLayerMx &ly) {   /* the communication waves */
        const u32x4 desc = buf_desc(ly.down[xe], (uint32_t)D * RB);
        const uint32_t a0 = (uint32_t)(RS * R * RB) - dsh;
        for (int k = wave - NW; k < NDMA; k += NC) copy_1k(desc, a0 + 1024u * (uint32_t)k, lds_addr(dws + 1024 * k), lane);
    };
    /* One MXFP4 block from dws at byte offset off: the e8m0 byte there and
     * the 16 code bytes after it, from the five aligned dwords that start
     * with the first code byte.
     * Off-slice lanes pass on = false and read the zero pad. */
    auto lds_blk_at = [&](uint32_t off, bool on) -> MxBlk {
        off = on ? off : (uint32_t)DZERO;
        const uint32_t cs = off + (on ? 1u : 0u);   /* first code byte */
        const uint32_t *p = reinterpret_cast<const uint32_t *>(dws + (cs & ~3u));
        const uint32_t w0 = p[0], w1 = p[1], w2 = p[2], w3 = p[3], w4 = p[4];
        const uint32_t sft = cs & 3u;
        MxBlk r;
        r.e = dws[off];
        r.c.x = __builtin_amdgcn_alignbyte(w1, w0, sft);
        r.c.y = __builtin_amdgcn_alignbyte(w2, w1, sft);
        r.c.z = __builtin_amdgcn_alignbyte(w3, w2, sft);
        r.c.w = __builtin_amdgcn_alignbyte(w4, w3, sft);
        return r;
    };
    /* down block (gr, i) of this lane from the contiguous copy */
    auto lds_blk = [&](int gr, int i) -> MxBlk {
        const int c = CPW * wave + i, b = 4 * c + (lane >> 4), sr = 16 * gr + (lane & 15);
        const bool on = c < NCH && b < NBLK && sr < RS;
        return lds_blk_at(dsh + (uint32_t)sr * RB + (uint32_t)b * 17u, on);
    };
    /* gate or up block (gr, i) of this lane from the wave's own segments */
    auto seg_blk = [&](int gr, int i) -> MxBlk {
        const int c = CPW * wave + i, b = 4 * c + (lane >> 4), sr = 16 * gr + (lane & 15);
        const bool on = c < NCH && b < NBLK && sr < RS;
        return lds_blk_at((uint32_t)(GREG * wave) + segst * (uint32_t)sr + (uint32_t)(b - 16 * wave) * 17u, on);
    };
    /* the communication waves hold no weights: they zero the registers the
     * compute waves fill, so both paths assign them */
    auto zero_units = [&](int u0) {
        const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < CPW; i++)
#pragma unroll
            for (int u = u0; u < u0 + NG; u++) wa[i][u] = MxBlk{0u, z};
    };
    auto load_nw = [&](const DecodeLayerMx &ly, bool use) {
        const bool on = use && wave < NW && ly.norm_w != nullptr;
        Buf nb = make_buf_uniform(on ? ly.norm_w : nullptr, on ? (uint32_t)D * 4u : 0u);
        nw0 = ld16(nb, (uint32_t)ct * 16u);
        nw1 = ld16(nb, (uint32_t)(NW * 64 + ct) * 16u);
    };
    auto store_nw = [&]() {
        if (wave < NW) {
            if (ct < D / 4) reinterpret_cast<u32x4 *>(nws)[ct] = nw0;
            if (ct < D / 4 - NW * 64) reinterpret_cast<u32x4 *>(nws)[NW * 64 + ct] = nw1;
        }
    };
    /* q8 + fp8 halves of a D-value LDS vector (scaled by `scale` and the
     * RMSNorm weight when norm): wave w quantizes blocks w and w + 8 */
    /* blocks[phase][wave][k]: the q8 blocks each wave quantizes, -1 = none.
     * Phase 0 (q8 of x): the communication waves issue the down rows' copies
     * meanwhile, so the six compute waves take all twelve blocks, three per
     * SIMD (waves w and w + 4 share SIMD w % 4).  Phase 1 (q8 of the hidden
     * vector): every wave, blocks w and w + 8. */
    auto qblock = [&](int phase, int k) -> int {
        if (phase == 0) {
            switch (wave) {
                case 0: return k == 0 ? 0 : k == 1 ? 6 : -1;
                case 1: return k == 0 ? 1 : k == 1 ? 7 : -1;
                case 2: return k == 0 ? 2 : k == 1 ? 8 : 10;
                case 3: return k == 0 ? 3 : k == 1 ? 9 : 11;
                case 4: return k == 0 ? 4 : -1;
                case 5: return k == 0 ? 5 : -1;
                default: return -1;
            }
        }
        const int b = wave + NA * k;   /* waves 0-3: blocks w and w + 8; waves 4-7: block w */
        return k < 2 && b < NQ ? b : -1;
    };
    static_assert(NQ == 12 && NW == 6 && NA == 8, "q8 block assignment");
    auto quantize = [&](int phase, const float *src, bool norm, float scale, bool has_nw, LdsQ &q, float *dbg_x,
                        uint8_t *dbg_q, float *dbg_d) {
#pragma unroll
        for (int k = 0; k < 3; k++) {
            const int b = qblock(phase, k);
            if (b < 0) break;   /* uniform */
            /* lane l: values 4l .. 4l + 3 of the block, all inside the row
             * or all past it (D is a multiple of 4): one 16-byte LDS read of
             * each operand, from a clamped address, then zeros past the row */
            const int i0 = 256 * b + 4 * lane;
            const bool in = i0 < D;
            float4 h4 = *reinterpret_cast<const float4 *>(src + (in ? i0 : 0));
            float4 w4 = *reinterpret_cast<const float4 *>(nws + (in ? i0 : 0));
            if (!in) h4 = float4{0.f, 0.f, 0.f, 0.f};
            if (!(norm && has_nw && in)) w4 = float4{1.f, 1.f, 1.f, 1.f};
            float v[4] = {h4.x, h4.y, h4.z, h4.w};
            const float wv[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                if (norm) v[c] = (v[c] * scale) * wv[c];
                if (dbg_x && in) dbg_x[i0 + c] = v[c];
            }
            q8_split_block(v[0], v[1], v[2], v[3], lane, b, q, reinterpret_cast<uint32_t *>(dbg_q), dbg_d);
        }
    };

    /* layer descriptors -> LDS; layer input: the caller's h */
    {
        const uint32_t *src = reinterpret_cast<const uint32_t *>(layers);
        uint32_t *dst = reinterpret_cast<uint32_t *>(lys);
        const int words = L * (int)(sizeof(DecodeLayerMx) / 4);
        for (int t = threadIdx.x; t < words; t += NT) dst[t] = src[t];
    }
    for (int t = threadIdx.x; t < D / 4; t += NT) reinterpret_cast<u32x4 *>(hx)[t] = reinterpret_cast<const u32x4 *>(h)[t];
    if (threadIdx.x < (DWS - DZERO) / 4) reinterpret_cast<uint32_t *>(dws + DZERO)[threadIdx.x] = 0u;
    /* the fp8 block slots past the row stay zero (chunk 22 reads them) */
    for (int t = threadIdx.x; t < (NSB - NBLK) * 64 / 4; t += NT) {
        reinterpret_cast<uint32_t *>(&sx.sp[NBLK][0][0])[t] = 0u;
        reinterpret_cast<uint32_t *>(&sh.sp[NBLK][0][0])[t] = 0u;
    }
    __syncthreads();
    /* slice sums of h^2 for layer 0 (later layers receive them with h) */
    for (int s = wave; s < NRK; s += NA) {
        const float v = lane < RS ? hx[RS * s + lane] : 0.f;
        const float t = wave_sum(v * v);
        if (lane == 0) ssq[s] = t;
    }
    load_nw(lys[0], true);
    if (wave < NW) {
        fetch_seg(lys[0].gate[xe], true);
        wait_copies();
#pragma unroll
        for (int i = 0; i < CPW; i++)
#pragma unroll
            for (int gr = 0; gr < NG; gr++) wa[i][gr] = seg_blk(gr, i);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        fetch_seg(lys[0].up[xe], true);
    } else {
        const u32x4 z = {0u, 0u, 0u, 0u};
        nw0 = nw1 = z;
        zero_units(0);
    }
    store_nw();
    bar_lds();   /* layer 0's RMSNorm weight is in LDS before step 2 reads it */

    const unsigned base = epoch_s;   /* read after the prologue barrier */
    for (int l = 0; l < L; l++) {
        const DecodeLayerMx &ly = lys[l];
        const unsigned par = (unsigned)(l & 1);
        const unsigned tag = base + (unsigned)l + 1u;
        const bool has_nw = ly.norm_w != nullptr;
        int clv = cl;
        asm volatile("" : "+v"(clv));
        asm volatile("" : "+v"(lane));
        const bool tw = times && threadIdx.x == 0;
        const bool tc = times && clv == 0;
        uint64_t *tr = times ? times + ((size_t)wg * L + l) * NTS : nullptr;
        uint8_t *rec = dbg ? dbg + (size_t)l * DecodeDebugMx::BYTES : nullptr;
        if (tw) tr[0] = wall_clock64();
        /* this layer's up blocks from the wave's own staged segments (copied
         * during the previous layer's hop) into registers; its gate blocks
         * arrived there during that hop */
        if (cl < 0) {
            wait_copies();
#pragma unroll
            for (int i = 0; i < CPW; i++)
#pragma unroll
                for (int gr = 0; gr < NG; gr++) wa[i][NG + gr] = seg_blk(gr, i);
        } else {
            zero_units(NG);
        }
        if (l == 0) bar_lds();   /* every wave is done with dws before the down rows' copy */
        /* the slice's gate, up and down biases (communication lanes, one row
         * each): issued ahead of the h polls, behind no weight copies */
        float gbv = 0.f, ubv = 0.f, dbv = 0.f;
        if (cl >= 0) {
            const bool on = clv < RS;
            const uint32_t o = on ? (uint32_t)(RS * R + clv) * 4u : OOB;
            gbv = __uint_as_float(ld4(make_buf_uniform(ly.gb[xe], ly.gb[xe] ? (uint32_t)D * 4u : 0u), o));
            ubv = __uint_as_float(ld4(make_buf_uniform(ly.ub[xe], ly.ub[xe] ? (uint32_t)D * 4u : 0u), o));
            dbv = __uint_as_float(ld4(make_buf_uniform(ly.db[xe], ly.db[xe] ? (uint32_t)D * 4u : 0u), o));
        }
        /* ---- 1: gather h: slices j' and 32 + j' from the other ranks of this XCD ---- */
        if (l > 0) {
            if (cl < 0) store_nw();
            {   /* every wave polls (one or two slots a lane) */
                unsigned rounds = 0;
                if (tc) tr[15] = wall_clock64();
                const bool ok = poll_slots<NT, ((NR - 1) * HS + NT - 1) / NT>(
                    sl, (int)threadIdx.x, (NR - 1) * HS, base + (unsigned)l, abort_flag,
                    [&](int f) {
                        const int jj = f / HS, t = f % HS;
                        const int j = jj + (jj >= rk);
                        return HSL + ((par ^ 1u) * NWG + (uint32_t)(xc + NX * j)) * HS + (uint32_t)t;
                    },
                    [&](int f, const u32x4 &v) {
                        const int jj = f / HS, t = f % HS;
                        const int j = jj + (jj >= rk);
                        const int half = t / (SS + 1), u = t % (SS + 1);
                        const int s = NR * half + j;
                        if (u == SS) {
                            ssq[s] = __uint_as_float(v.y);
                        } else {
                            float *o = hx + RS * s + VPS * u;
                            o[0] = __uint_as_float(v.y);
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
            }
            bar_lds();
            if (lds_fail) {
            wait_copies();   /* no copy into LDS outlives the workgroup */
            advance_epoch(abort_flag, base, L);
            return;
        }
        }
        if (tw) tr[1] = wall_clock64();
        /* ---- 2: RMSNorm (weight or 1) + q8 + fp8 halves of x ---- */
        if (cl >= 0) fetch_down(ly);
        {
            const float tot = wave_sum(ssq[lane]);   /* the 64 slice sums, one per lane */
            const float scale = 1.f / sqrtf(tot / (float)D + eps);
            if (rec && wg == 0)
                for (int t = threadIdx.x; t < D; t += NT) reinterpret_cast<float *>(rec + DecodeDebugMx::HIN)[t] = hx[t];
            const bool rx = rec && wg == 0;
            quantize(0, hx, true, scale, has_nw, sx, rx ? reinterpret_cast<float *>(rec + DecodeDebugMx::X) : nullptr,
                     rx ? rec + DecodeDebugMx::XQ : nullptr,
                     rx ? reinterpret_cast<float *>(rec + DecodeDebugMx::XD) : nullptr);
        }
        bar_lds();
        if (tw) tr[2] = wall_clock64();
        /* ---- 3: gate/up rows of the slice, chunks [4 w, 4 w + 4) of wave w ---- */
        if (wave < NW) {
            v4f acc[2 * NG];
#pragma unroll
            for (int u = 0; u < 2 * NG; u++) acc[u] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < CPW; i++) {
                const int c = CPW * wave + i;
                if (c >= NCH) break;   /* uniform */
                const v8i bx = load_b(sx, c, lane);
                const float d = sx.d[c >> 1];
#pragma unroll
                for (int u = 0; u < 2 * NG; u++) mma_chunk(wa[i][u], bx, sb, d, acc[u]);
            }
            /* columns 0 and 1 of the MFMA results: lane 16 g + col holds rows 4 g .. 4 g + 3 */
            if ((lane & 15) < 2)
#pragma unroll
                for (int u = 0; u < 2 * NG; u++)
#pragma unroll
                    for (int v = 0; v < 4; v++) red[u][4 * (lane >> 4) + v][wave][lane & 15] = acc[u][v];
        }
        /* the down rows' copy (issued by the communication waves) has landed
         * in dws before the barrier */
        wait_copies();
        bar_lds();
        if (tw) tr[3] = wall_clock64();
        /* ---- 4: bias + activation, all-gather the expert's hidden vector ---- */
        /* meanwhile the compute waves gather their down blocks from dws into
         * registers; the communication waves zero theirs (both paths assign,
         * so no old value stays live) */
        auto gather_down = [&]() {
            if (cl < 0) {
#pragma unroll
                for (int i = 0; i < CPW; i++)
#pragma unroll
                    for (int u = 0; u < NG; u++) wb[i][u] = lds_blk(u, i);
            } else {
                const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
                for (int i = 0; i < CPW; i++)
#pragma unroll
                    for (int u = 0; u < NG; u++) wb[i][u] = MxBlk{0u, z};
            }
        };
        gather_down();
        if (cl >= 0) {
            /* row i of the slice: the six waves' partial sums in wave order */
            if (clv < RS) {
                const int gi = clv >> 4, ri = clv & 15, row = RS * R + clv;
                float pg[2 * NW], pu[2 * NW];
#pragma unroll
                for (int k = 0; k < NW / 2; k++) {
                    const float4 a = reinterpret_cast<const float4 *>(&red[gi][ri][0][0])[k];
                    const float4 b = reinterpret_cast<const float4 *>(&red[NG + gi][ri][0][0])[k];
                    pg[4 * k] = a.x, pg[4 * k + 1] = a.y, pg[4 * k + 2] = a.z, pg[4 * k + 3] = a.w;
                    pu[4 * k] = b.x, pu[4 * k + 1] = b.y, pu[4 * k + 2] = b.z, pu[4 * k + 3] = b.w;
                }
                float g = 0.f, u = 0.f;
#pragma unroll
                for (int w = 0; w < NW; w++) {
                    g += pg[2 * w] + pg[2 * w + 1];
                    u += pu[2 * w] + pu[2 * w + 1];
                }
                hid[row] = act_fn(TG_ACT_GPTOSS, g + gbv, u + ubv);
            }
            __builtin_amdgcn_wave_barrier();
            if (clv < SS) {
                const float *a = hid + RS * R + VPS * clv;
                put_slot<CPOL_SC1>(sl, GSL + (par * NWG + (uint32_t)wg) * SS + (uint32_t)clv, tag, a[0], a[1], a[2]);
            }
            if (tc) tr[9] = wall_clock64();
        }
        {   /* every wave polls the expert's other ranks (one or two slots a lane) */
            unsigned rounds = 0;
            if (tc) tr[12] = wall_clock64();
            const bool ok = poll_slots<NT, ((NRK - 1) * SS + NT - 1) / NT>(
                sl, (int)threadIdx.x, (NRK - 1) * SS, tag, abort_flag,
                [&](int f) {
                    const int rr = f / SS, t = f % SS;
                    const int r2 = rr + (rr >= R);
                    const int w2 = (2 * xe + (r2 >= NR ? 1 : 0)) + NX * (r2 % NR);
                    return GSL + (par * NWG + (uint32_t)w2) * SS + (uint32_t)t;
                },
                [&](int f, const u32x4 &v) {
                    const int rr = f / SS, t = f % SS;
                    const int r2 = rr + (rr >= R);
                    float *o = hid + RS * r2 + VPS * t;
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
        bar_lds();
        if (lds_fail) {
            wait_copies();   /* no copy into LDS outlives the workgroup */
            advance_epoch(abort_flag, base, L);
            return;
        }
        if (tw) tr[4] = wall_clock64();
        /* ---- 5: q8 + fp8 halves of the hidden vector ---- */
        if (rec && (xc & 1) == 0 && rk == 0)   /* workgroup 2e: expert slot e's record */
            for (int t = threadIdx.x; t < D; t += NT)
                reinterpret_cast<float *>(rec + DecodeDebugMx::HID)[xe * D + t] = hid[t];
        /* the next layer's gate segments into dws (free since the down blocks
         * were gathered), draining during this q8, the down rows and the hop */
        if (cl < 0 && l + 1 < L) fetch_seg(lys[l + 1].gate[xe], true);
        {
            const bool rh = rec && (xc & 1) == 0 && rk == 0;
            quantize(1, hid, false, 1.f, false, sh, nullptr, rh ? rec + DecodeDebugMx::HQ + xe * (NQ * 256) : nullptr,
                     rh ? reinterpret_cast<float *>(rec + DecodeDebugMx::HD) + xe * NQ : nullptr);
        }
        bar_lds();
        if (tw) tr[5] = wall_clock64();
        /* ---- 6: down rows of the slice ---- */
        if (wave < NW) {
            v4f acc[NG];
#pragma unroll
            for (int u = 0; u < NG; u++) acc[u] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < CPW; i++) {
                const int c = CPW * wave + i;
                if (c >= NCH) break;   /* uniform */
                const v8i bx = load_b(sh, c, lane);
                const float d = sh.d[c >> 1];
#pragma unroll
                for (int u = 0; u < NG; u++) mma_chunk(wb[i][u], bx, sb, d, acc[u]);
            }
            if ((lane & 15) < 2)
#pragma unroll
                for (int u = 0; u < NG; u++)
#pragma unroll
                    for (int v = 0; v < 4; v++) red[u][4 * (lane >> 4) + v][wave][lane & 15] = acc[u][v];
        }
        bar_lds();
        if (tw) tr[6] = wall_clock64();
        /* ---- 7: cross-XCD hop: rank rk of every XCD trades its 45 weighted down values ---- */
        /* meanwhile each compute wave moves the next layer's gate blocks (its
         * segments landed during q8(hidden) and the down dots) into
         * registers, then copies the next layer's up segments into the same
         * region and loads the next RMSNorm weight; both paths assign the
         * registers (empty loads past the last layer) */
        if (cl < 0) {
            const bool more = l + 1 < L;
            wait_copies();
#pragma unroll
            for (int i = 0; i < CPW; i++)
#pragma unroll
                for (int gr = 0; gr < NG; gr++) wa[i][gr] = seg_blk(gr, i);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   /* read before the copy overwrites */
            fetch_seg(more ? lys[l + 1].up[xe] : nullptr, more);
            load_nw(lys[more ? l + 1 : l], more);
        } else {
            const u32x4 z = {0u, 0u, 0u, 0u};
            nw0 = nw1 = z;
            zero_units(0);
        }
        if (cl >= 0) {
            if (clv < RS) {
                const int gi = clv >> 4, ri = clv & 15;
                float v = 0.f;
#pragma unroll
                for (int k = 0; k < NW / 2; k++) {
                    const float4 a = reinterpret_cast<const float4 *>(&red[gi][ri][0][0])[k];
                    v += a.x + a.y;
                    v += a.z + a.w;
                }
                pp[xc][clv] = ly.w[xe] * (v + dbv);
            }
            __builtin_amdgcn_wave_barrier();
            if (clv < SS) {
                const float *a = pp[xc] + VPS * clv;
                put_slot<CPOL_SC1>(sl, PSL + (par * NWG + (uint32_t)wg) * SS + (uint32_t)clv, tag, a[0], a[1], a[2]);
            }
            if (tc) tr[10] = wall_clock64();
            unsigned rounds = 0;
            const bool ok = poll_slots<CL, 1>(
                sl, clv, (NX - 1) * SS, tag, abort_flag,
                [&](int f) {
                    const int xx = f / SS, t = f % SS;
                    const int x = xx + (xx >= xc);
                    return PSL + (par * NWG + (uint32_t)(x + NX * rk)) * SS + (uint32_t)t;
                },
                [&](int f, const u32x4 &v) {
                    const int xx = f / SS, t = f % SS;
                    const int x = xx + (xx >= xc);
                    float *o = pp[x] + VPS * t;
                    o[0] = __uint_as_float(v.y);
                    o[1] = __uint_as_float(v.z);
                    o[2] = __uint_as_float(v.w);
                },
                tc ? &rounds : nullptr);
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
        /* ---- 8: combine slices rk (first communication wave) and 32 + rk
         * (second) in expert order, publish ---- */
        if (cl >= 0) {
            const int half = clv >> 6, ri = clv & 63, s = NR * half + rk;
            float a = 0.f;
            if (ri < RS) {
                const int r = RS * s + ri;
                a = hx[r];
#pragma unroll
                for (int e = 0; e < NE; e++) a += pp[2 * e + half][ri];
                hx[r] = a;
                if (l == L - 1 && xc == 0) h[r] = a;
            }
            const float sq = wave_sum(a * a);   /* the slice's sum of h^2, for the next RMSNorm */
            if (ri == 0) ssq[s] = sq;
            __builtin_amdgcn_wave_barrier();
            if (l + 1 < L && ri <= SS) {
                const uint32_t slot = HSL + (par * NWG + (uint32_t)wg) * HS + (uint32_t)((SS + 1) * half + ri);
                /* read only inside this XCD: kept in its L2 (policy 0), or
                 * stored device-coherently like every other slot (policy 1) */
                float a0 = sq, a1 = 0.f, a2 = 0.f;   /* the slot after the slice: its sum of h^2 */
                if (ri < SS) {
                    const float *o = hx + RS * s + VPS * ri;
                    a0 = o[0];
                    a1 = o[1];
                    a2 = o[2];
                }
                if (pol) put_slot<CPOL_SC1>(sl, slot, tag, a0, a1, a2);
                else put_slot<CPOL_PLAIN>(sl, slot, tag, a0, a1, a2);
            }
            if (tc) tr[11] = wall_clock64();
        }
        if (tw) tr[8] = wall_clock64();
    }
    advance_epoch(abort_flag, base, L);
}

int decode_mx_max_grid() {
    int dev = 0, per_cu = 0;
    hipDeviceProp_t pr;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&pr, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *)k_decode_mx, NT, 0) != hipSuccess)
        return 0;
    return per_cu * pr.multiProcessorCount;
}

size_t decode_mx_slot_bytes() { return (size_t)NSLOTS * 16; }

/* Rewrites a 2880 x 2880 MXFP4 matrix into the wave-segment layout: slice R
 * (rows 45 R ..), wave w, row sr at R * SLB + w * WSB + sr * stride(w), the
 * wave's bytes [272 w, 272 w + len(w)) of the row (the same bytes; the 6
 * bytes after each last-wave segment are zero).  One thread per (slice,
 * wave, row), two bytes at a time (every offset is even). */
__global__ void k_mx_wave_segments(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= NRK * NW * RS) return;
    const int sr = t % RS, w = (t / RS) % NW, R = t / (RS * NW);
    const int len = w == NW - 1 ? SEGL : SEGB, st = w == NW - 1 ? SEGLS : SEGB;
    const uint16_t *s16 = reinterpret_cast<const uint16_t *>(src + (size_t)(RS * R + sr) * RB + (size_t)SEGB * w);
    uint16_t *d16 = reinterpret_cast<uint16_t *>(dst + (size_t)R * SLB + (size_t)w * WSB + (size_t)sr * st);
    for (int i = 0; i < st / 2; i++) d16[i] = 2 * i < len ? s16[i] : (uint16_t)0;
}

size_t decode_mx_seg_bytes() { return MXSEG_BYTES; }

hipError_t launch_mx_wave_segments(const void *src, void *dst, hipStream_t st) {
    const int n = NRK * NW * RS;
    hipLaunchKernelGGL(k_mx_wave_segments, dim3((n + 255) / 256), dim3(256), 0, st, (const uint8_t *)src,
                       (uint8_t *)dst);
    return hipGetLastError();
}

hipError_t launch_decode_mx(const DecodeLayerMx *layers_dev, int L, float *h_dev, void *slots_dev, unsigned *abort_dev,
                            float eps, uint8_t *debug_dev, uint64_t *times_dev, unsigned *place_dev, int pol,
                            bool cooperative, hipStream_t st) {
    void *args[] = {(void *)&layers_dev, (void *)&L,         (void *)&h_dev,     (void *)&slots_dev,
                    (void *)&abort_dev,  (void *)&eps,       (void *)&debug_dev, (void *)&times_dev,
                    (void *)&place_dev,  (void *)&pol};
    if (cooperative)
        return hipLaunchCooperativeKernel((const void *)k_decode_mx, dim3(DECODE_GRID), dim3(NT), args, 0, st);
    return hipLaunchKernel((const void *)k_decode_mx, dim3(DECODE_GRID), dim3(NT), args, 0, st);
}

const void *decode_mx_fn() { return (const void *)k_decode_mx; }
int decode_mx_threads() { return NT; }

}  // namespace tg
