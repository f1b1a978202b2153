/*
 * tg_device.hpp -- CDNA4 (gfx950) device building blocks for the fused
 * quantized GEMV family: bounds-checked buffer loads, the reference's f16
 * decode, per-format "items" (the slice of a weight row one lane decodes),
 * and wave-segment reductions.
 *
 * Lane model.  A weight row of `ncols` values is cut into items:
 *   Q4_K   4 items per 256-block  (one 32-byte quarter of qs[] + the 16-byte
 *          block header; sub-blocks 2g and 2g+1)
 *   Q6_K   4 items per 256-block  (half h, lanes l0..l0+15: 48 bytes of
 *          ql/qh, 4 int8 sub-scales, d)
 *   MXFP4  1 item per 32-block    (17 bytes)
 *   Q8_0   1 item per 32-block    (34 bytes)
 *   F16    1 item per 8 values    (16 bytes, f32 activations)
 * A wave is split into 64/S segments of S lanes (S a power of two); each
 * segment owns one weight row per step and lane s of the segment decodes
 * items s, s+S, s+2S, ...  The integer sums of every item are exact; the
 * float combine of an item follows the reference's formula, and the
 * segment sum is a butterfly over the S lanes.
 */
#ifndef TG_DEVICE_HPP
#define TG_DEVICE_HPP
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tg_common.h"

namespace tg {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

/* ---- bounds-checked raw buffer loads (out-of-range lanes read zero) ---- */

struct Buf {
    __amdgpu_buffer_rsrc_t r;
};

__device__ inline Buf make_buf(const void *p, uint32_t nbytes) {
    Buf b;
    b.r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)nbytes, 0x00020000);
    return b;
}
/* Descriptor for a pointer that is wave-uniform although the compiler cannot
 * prove it (e.g. read from LDS): readfirstlane keeps the descriptor in SGPRs,
 * where a VGPR descriptor would wrap every access in a waterfall loop. */
__device__ inline Buf make_buf_uniform(const void *p, uint32_t nbytes) {
    const uint64_t a = (uint64_t)(uintptr_t)p;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
    const uint32_t n = (uint32_t)__builtin_amdgcn_readfirstlane((int)nbytes);
    return make_buf((const void *)(uintptr_t)(((uint64_t)hi << 32) | lo), n);
}
__device__ inline u32x4 ld16(Buf b, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(b.r, (int)off, 0, 0);
}
__device__ inline u32x2 ld8(Buf b, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b64(b.r, (int)off, 0, 0);
}
__device__ inline uint32_t ld4(Buf b, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(b.r, (int)off, 0, 0);
}
/* the same loads from a q8 row staged in LDS (offsets aligned to the size) */
__device__ inline u32x4 ld16(const uint8_t *p, uint32_t off) { return *reinterpret_cast<const u32x4 *>(p + off); }
__device__ inline u32x2 ld8(const uint8_t *p, uint32_t off) { return *reinterpret_cast<const u32x2 *>(p + off); }
__device__ inline uint32_t ld4(const uint8_t *p, uint32_t off) { return *reinterpret_cast<const uint32_t *>(p + off); }
__device__ inline uint32_t ld2(Buf b, uint32_t off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(b.r, (int)off, 0, 0);
}
__device__ inline uint32_t ld1(Buf b, uint32_t off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(b.r, (int)off, 0, 0);
}

/* f16 -> f32 exactly as csrc/libtinygiant.c:128-137 decodes it: IEEE for
 * every finite pattern; exponent 31 yields the bit pattern 0xB7800000|m<<13
 * that the reference's 32-bit shift produces. */
__device__ inline float ref_f16(uint32_t h) {
    h &= 0xFFFFu;
    float f = (float)__builtin_bit_cast(_Float16, (uint16_t)h);
    if ((h & 0x7C00u) == 0x7C00u) f = __uint_as_float(0xB7800000u | ((h & 0x3FFu) << 13));
    return f;
}

/* e8m0_to_fp32_half (csrc/libtinygiant.c:516-519) */
__device__ inline float e8m0_half(uint32_t e) {
    uint32_t bits = e < 2 ? (0x00200000u << e) : ((e - 1u) << 23);
    return __uint_as_float(bits);
}

__device__ inline int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

/* ---- DPP cross-lane reductions ----
 * GFX9 DPP controls: quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E,
 * row_half_mirror = 0x141, row_mirror = 0x140, row_bcast:15 = 0x142,
 * row_bcast:31 = 0x143.  Each step adds a lane's value to one partner's, so
 * every lane of a group holds the same (commutatively identical) sum. */
template <int CTRL, int ROW_MASK = 0xF>
__device__ inline int dpp_i(int old, int v) {
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROW_MASK, 0xF, false);
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ inline float dpp_f(float old, float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

/* sum over aligned groups of S lanes (S = 2..64); the result is exact in
 * the group's last lane (lane % S == S - 1), and in every lane for S <= 16 */
template <int S>
__device__ inline float seg_sum_last(float v) {
    static_assert(S >= 2 && S <= 64 && (S & (S - 1)) == 0, "segment");
    v += dpp_f<0xB1>(v, v);
    if (S >= 4) v += dpp_f<0x4E>(v, v);
    if (S >= 8) v += dpp_f<0x141>(v, v);
    if (S >= 16) v += dpp_f<0x140>(v, v);
    if (S >= 32) v += dpp_f<0x142, 0xA>(0.f, v);
    if (S >= 64) v += dpp_f<0x143, 0xC>(0.f, v);
    return v;
}
template <int S>
__device__ inline int seg_isum_last(int v) {
    v += dpp_i<0xB1>(v, v);
    if (S >= 4) v += dpp_i<0x4E>(v, v);
    if (S >= 8) v += dpp_i<0x141>(v, v);
    if (S >= 16) v += dpp_i<0x140>(v, v);
    if (S >= 32) v += dpp_i<0x142, 0xA>(0, v);
    if (S >= 64) v += dpp_i<0x143, 0xC>(0, v);
    return v;
}
/* wave-wide sum / max, broadcast to every lane (fixed combination order) */
__device__ inline float wave_sum(float v) {
    v = seg_sum_last<16>(v);
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 15));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 47));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
    return (a + b) + (c + d);
}
__device__ inline float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v, v));
    v = fmaxf(v, dpp_f<0x4E>(v, v));
    v = fmaxf(v, dpp_f<0x141>(v, v));
    v = fmaxf(v, dpp_f<0x140>(v, v));
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 15));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 47));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

/* ---- segment reductions (segments of S lanes, S power of two <= 64) ---- */

template <int S>
__device__ inline float seg_sum(float v) {
#pragma unroll
    for (int o = S / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ inline float seg_sum_rt(float v, int S) {
    for (int o = S / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

/* The bits of seg_sum<S> (S = 16 or 32) without its chain of LDS round
 * trips.  After the butterfly's stages of strides above s, all lanes of a
 * class i mod 2s hold the same bits (a + b and b + a round alike), so any
 * lane of class (i mod 2s) ^ s is a partner as good as i ^ s: a rotation of
 * the 16-lane row by s is one, once the stride-2s stage is done
 * ((x - s) mod 2s = x ^ s).  Stride 16, which crosses rows, is one
 * ds_swizzle (xor 16 within 32 lanes); stride 8 is row_ror:8, an exact xor
 * inside a row; 4 is row_ror:4; 2 and 1 are exact quad permutations. */
template <int S>
__device__ inline float seg_sum_x(float v) {
    static_assert(S == 16 || S == 32, "segment");
    if (S == 32) v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
    v += dpp_f<0x128>(v, v);   /* row_ror:8 */
    v += dpp_f<0x124>(v, v);   /* row_ror:4 */
    v += dpp_f<0x4E>(v, v);    /* quad_perm [2,3,0,1] */
    v += dpp_f<0xB1>(v, v);    /* quad_perm [1,0,3,2] */
    return v;
}

/* ---- q8 activation rows on the device ----
 * Row r of an activation matrix with nb 256-blocks:
 *   qs  int8[nb*256] (zero padded), d f32[nb] (block scale),
 *   s32 int32[nb*8]  (32-element sums), s16 int32[nb*16] (16-element sums). */
struct Q8Rows {
    int8_t *qs;
    float *d;
    int32_t *s32;
    int32_t *s16;
    int32_t *sum;     /* per-block total (the reference's q8_block.sum) */
    const float *f;   /* the unquantized f32 rows (used by F16 weights) */
    int nb;
    int fstride;      /* floats per f32 row */
};

struct Q8Row {
    Buf qs, d, s32, s16, f;
};

/* One q8 row staged in LDS (no f32 copy): qs int8[nb*256], d f32[nb],
 * s32 int32[nb*8], s16 int32[nb*16], as byte pointers into shared memory. */
struct Q8Lds {
    const uint8_t *qs, *d, *s32, *s16;
};

/* q8 of one 256-value block held by a wave, lane l owning values 4l..4l+3
 * (quantize_q8, csrc/libtinygiant.c:169-208): scale amax/127, quants
 * rint(v * 127/amax) packed four to a word, the lane's 16- and 32-element
 * sums (valid in lanes l % 4 == 0 and l % 8 == 0) and the block total. */
struct Q8Quant {
    uint32_t packed;
    int s16, s32, tot;
    float sc;
};
__device__ inline Q8Quant q8_block_quant(float v0, float v1, float v2, float v3) {
    float amax = fmaxf(fmaxf(fabsf(v0), fabsf(v1)), fmaxf(fabsf(v2), fabsf(v3)));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    Q8Quant r;
    r.sc = amax / 127.f;                  /* correctly rounded */
    const float inv = amax > 0.f ? 127.f / amax : 0.f;
    int q0 = (int)__builtin_rintf(v0 * inv), q1 = (int)__builtin_rintf(v1 * inv);
    int q2 = (int)__builtin_rintf(v2 * inv), q3 = (int)__builtin_rintf(v3 * inv);
    r.packed = (uint32_t)(q0 & 0xFF) | ((uint32_t)(q1 & 0xFF) << 8) | ((uint32_t)(q2 & 0xFF) << 16) |
               ((uint32_t)(q3 & 0xFF) << 24);
    int s = q0 + q1 + q2 + q3;
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);            /* 16-element sum */
    r.s16 = s;
    r.s32 = s + __shfl_xor(s, 4, 64);     /* 32-element sum */
    int tot = r.s32;
    tot += __shfl_xor(tot, 8, 64);
    tot += __shfl_xor(tot, 16, 64);
    tot += __shfl_xor(tot, 32, 64);
    r.tot = tot;
    return r;
}

/* LDS bytes of one staged q8 row of nb blocks: qs [nb*256], s32 [nb*8],
 * s16 [nb*16], d [nb] */
__host__ __device__ constexpr uint32_t q8_lds_stride(int nb) { return ((uint32_t)nb * 356u + 15u) & ~15u; }

__device__ inline Q8Lds q8_lds_slot(const uint8_t *base, int nb, int s) {
    const uint8_t *b = base + (size_t)s * q8_lds_stride(nb);
    return Q8Lds{b, b + nb * 352, b + nb * 256, b + nb * 288};
}

/* q8_block_quant's quants, 16- and 32-element sums and scale (not the block
 * total) without LDS round trips: the maximum and the integer sums are exact
 * in any order, so DPP partners of the right lane class stand in for the
 * xor partners (row_half_mirror pairs the two quads of 8 lanes). */
__device__ inline Q8Quant q8_block_quant_dpp(float v0, float v1, float v2, float v3) {
    const float amax = wave_max(fmaxf(fmaxf(fabsf(v0), fabsf(v1)), fmaxf(fabsf(v2), fabsf(v3))));
    Q8Quant r;
    r.sc = amax / 127.f;                  /* correctly rounded */
    const float inv = amax > 0.f ? 127.f / amax : 0.f;
    int q0 = (int)__builtin_rintf(v0 * inv), q1 = (int)__builtin_rintf(v1 * inv);
    int q2 = (int)__builtin_rintf(v2 * inv), q3 = (int)__builtin_rintf(v3 * inv);
    r.packed = (uint32_t)(q0 & 0xFF) | ((uint32_t)(q1 & 0xFF) << 8) | ((uint32_t)(q2 & 0xFF) << 16) |
               ((uint32_t)(q3 & 0xFF) << 24);
    int s = q0 + q1 + q2 + q3;
    s += dpp_i<0xB1>(s, s);
    s += dpp_i<0x4E>(s, s);               /* 16-element sum */
    r.s16 = s;
    r.s32 = s + dpp_i<0x141>(s, s);       /* 32-element sum */
    r.tot = 0;
    return r;
}

/* The bits of the 64-lane shfl_xor butterfly (strides 32 .. 1) of v: one
 * LDS permute for stride 32, then seg_sum_x<32>. */
__device__ inline float wave_sum_x(float v) {
    v += __shfl_xor(v, 32, 64);
    return seg_sum_x<32>(v);
}

/* q8_block_quant of the wave's block, written to block b of row r */
__device__ inline void q8_block_store(float v0, float v1, float v2, float v3, int lane, const Q8Rows &out, int r,
                                      int b) {
    const Q8Quant q = q8_block_quant(v0, v1, v2, v3);
    const int nb = out.nb;
    int8_t *qrow = out.qs + ((size_t)r * nb + b) * 256;
    reinterpret_cast<uint32_t *>(qrow)[lane] = q.packed;
    const size_t rb = (size_t)r * nb + b;
    if ((lane & 3) == 0) out.s16[rb * 16 + (lane >> 2)] = q.s16;
    if ((lane & 7) == 0) out.s32[rb * 8 + (lane >> 3)] = q.s32;
    if (lane == 0) {
        out.d[rb] = q.sc;
        out.sum[rb] = q.tot;
    }
}

__device__ inline Q8Row q8_row(const Q8Rows &a, int r) {
    Q8Row x;
    x.qs = make_buf(a.qs + (size_t)r * a.nb * 256, (uint32_t)a.nb * 256);
    x.d = make_buf(a.d + (size_t)r * a.nb, (uint32_t)a.nb * 4);
    x.s32 = make_buf(a.s32 + (size_t)r * a.nb * 8, (uint32_t)a.nb * 32);
    x.s16 = make_buf(a.s16 + (size_t)r * a.nb * 16, (uint32_t)a.nb * 64);
    x.f = make_buf(a.f + (size_t)r * a.fstride, (uint32_t)a.fstride * 4);
    return x;
}

/* ====================== formats ====================== */

/* ---- Q4_K: item = (block b, group g) ---- */
struct FQ4K {
    static constexpr int FMT = TG_FMT_Q4K;
    static constexpr int ITEMS_PER_BLOCK = 4, BLOCK_VALS = 256, BLOCK_BYTES = 144;
    static constexpr int NSUMS = 2;   /* integer sums per item */
    struct W { u32x4 hdr, q0, q1; };
    struct X { u32x4 a0, a1, b0, b1; int s_lo, s_hi; float d; };

    __device__ static inline W load_w(Buf w, uint32_t row_off, int item) {
        uint32_t p = row_off + (uint32_t)(item >> 2) * 144u;
        uint32_t g = item & 3;
        W r;
        r.hdr = ld16(w, p);
        r.q0 = ld16(w, p + 16 + 32 * g);
        r.q1 = ld16(w, p + 32 + 32 * g);
        return r;
    }
    template <class R>   /* Q8Row (global) or Q8Lds */
    __device__ static inline X load_x(const R &x, int item) {
        uint32_t b = item >> 2, g = item & 3;
        uint32_t o = b * 256 + 64 * g;
        X r;
        r.a0 = ld16(x.qs, o);
        r.a1 = ld16(x.qs, o + 16);
        r.b0 = ld16(x.qs, o + 32);
        r.b1 = ld16(x.qs, o + 48);
        u32x2 s = ld8(x.s32, (b * 8 + 2 * g) * 4);
        r.s_lo = (int)s.x;
        r.s_hi = (int)s.y;
        r.d = __uint_as_float(ld4(x.d, b * 4));
        return r;
    }
    __device__ static inline void isums(const W &w, const X &x, int *out) {
        const uint32_t m = 0x0F0F0F0Fu;
        int lo = 0, hi = 0;
        lo = dot4(w.q0.x & m, x.a0.x, lo); lo = dot4(w.q0.y & m, x.a0.y, lo);
        lo = dot4(w.q0.z & m, x.a0.z, lo); lo = dot4(w.q0.w & m, x.a0.w, lo);
        lo = dot4(w.q1.x & m, x.a1.x, lo); lo = dot4(w.q1.y & m, x.a1.y, lo);
        lo = dot4(w.q1.z & m, x.a1.z, lo); lo = dot4(w.q1.w & m, x.a1.w, lo);
        hi = dot4((w.q0.x >> 4) & m, x.b0.x, hi); hi = dot4((w.q0.y >> 4) & m, x.b0.y, hi);
        hi = dot4((w.q0.z >> 4) & m, x.b0.z, hi); hi = dot4((w.q0.w >> 4) & m, x.b0.w, hi);
        hi = dot4((w.q1.x >> 4) & m, x.b1.x, hi); hi = dot4((w.q1.y >> 4) & m, x.b1.y, hi);
        hi = dot4((w.q1.z >> 4) & m, x.b1.z, hi); hi = dot4((w.q1.w >> 4) & m, x.b1.w, hi);
        out[0] = lo;
        out[1] = hi;
    }
    /* get_scale_min_k4 (csrc/libtinygiant.c:146-155) for sub-blocks 2g, 2g+1 */
    __device__ static inline void scales(const W &w, int g, int &sc_lo, int &m_lo, int &sc_hi, int &m_hi) {
        uint32_t s0 = w.hdr.y, s1 = w.hdr.z, s2 = w.hdr.w;   /* scales[0..3], [4..7], [8..11] */
        int j = 2 * g;
        if (g < 2) {
            sc_lo = (s0 >> (8 * j)) & 63;        m_lo = (s1 >> (8 * j)) & 63;
            sc_hi = (s0 >> (8 * j + 8)) & 63;    m_hi = (s1 >> (8 * j + 8)) & 63;
        } else {
            int jl = j - 4, jh = j - 3;   /* 0..3 */
            sc_lo = ((s2 >> (8 * jl)) & 0xF) | (((s0 >> (8 * jl + 6)) & 3) << 4);
            m_lo = ((s2 >> (8 * jl + 4)) & 0xF) | (((s1 >> (8 * jl + 6)) & 3) << 4);
            sc_hi = ((s2 >> (8 * jh)) & 0xF) | (((s0 >> (8 * jh + 6)) & 3) << 4);
            m_hi = ((s2 >> (8 * jh + 4)) & 0xF) | (((s1 >> (8 * jh + 6)) & 3) << 4);
        }
    }
    /* the item decoded once for several input rows: its nibbles, scales,
     * mins and the two f16 factors */
    struct Wd {
        uint32_t lo[8], hi[8];
        int sc_lo, m_lo, sc_hi, m_hi;
        float d, dmin;
    };
    __device__ static inline Wd decode(const W &w, int item) {
        const uint32_t m = 0x0F0F0F0Fu;
        const uint32_t q[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
        Wd r;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            r.lo[i] = q[i] & m;
            r.hi[i] = (q[i] >> 4) & m;
        }
        scales(w, item & 3, r.sc_lo, r.m_lo, r.sc_hi, r.m_hi);
        r.d = ref_f16(w.hdr.x);
        r.dmin = ref_f16(w.hdr.x >> 16);
        return r;
    }
    /* x.d * (d*(sc_lo*lo + sc_hi*hi) - dmin*(m_lo*bs_lo + m_hi*bs_hi)):
     * both integer brackets are below 2^24, so they convert exactly. */
    __device__ static inline float value_d(const Wd &w, const X &x) {
        const uint32_t a[8] = {x.a0.x, x.a0.y, x.a0.z, x.a0.w, x.a1.x, x.a1.y, x.a1.z, x.a1.w};
        const uint32_t b[8] = {x.b0.x, x.b0.y, x.b0.z, x.b0.w, x.b1.x, x.b1.y, x.b1.z, x.b1.w};
        int lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            lo = dot4(w.lo[i], a[i], lo);
            hi = dot4(w.hi[i], b[i], hi);
        }
        int A = w.sc_lo * lo + w.sc_hi * hi;
        int B = w.m_lo * x.s_lo + w.m_hi * x.s_hi;
        return x.d * (w.d * (float)A - w.dmin * (float)B);
    }
    __device__ static inline float value(const W &w, const X &x, int item) { return value_d(decode(w, item), x); }
    /* where this item's integer sums go in the per-row isum vector
     * (8 sub-blocks per 256-block) */
    __device__ static inline int isum_index(int item, int i) { return (item >> 2) * 8 + 2 * (item & 3) + i; }
};

/* ---- Q6_K: item = (block b, unit u): half h = u>>1, lanes l0 = 16*(u&1) ---- */
struct FQ6K {
    static constexpr int FMT = TG_FMT_Q6K;
    static constexpr int ITEMS_PER_BLOCK = 4, BLOCK_VALS = 256, BLOCK_BYTES = 210;
    static constexpr int NSUMS = 4;
    struct W { u32x4 qla, qlb, qh; u32x2 sc; uint32_t d; };
    struct X { u32x4 x0, x1, x2, x3; int s0, s1, s2, s3; float d; };

    __device__ static inline W load_w(Buf w, uint32_t row_off, int item) {
        uint32_t p = row_off + (uint32_t)(item >> 2) * 210u;
        uint32_t u = item & 3, h = u >> 1, l0 = (u & 1) * 16;
        W r;
        r.qla = ld16(w, p + 64 * h + l0);
        r.qlb = ld16(w, p + 64 * h + 32 + l0);
        r.qh = ld16(w, p + 128 + 32 * h + l0);
        r.sc = ld8(w, p + 192 + 8 * h);
        r.d = ld4(w, p + 206);   /* sc[14], sc[15], d: d is the high half */
        return r;
    }
    template <class R>   /* Q8Row (global) or Q8Lds */
    __device__ static inline X load_x(const R &x, int item) {
        uint32_t b = item >> 2, u = item & 3, h = u >> 1, l0 = (u & 1) * 16;
        uint32_t o = b * 256 + 128 * h + l0;
        X r;
        r.x0 = ld16(x.qs, o);
        r.x1 = ld16(x.qs, o + 32);
        r.x2 = ld16(x.qs, o + 64);
        r.x3 = ld16(x.qs, o + 96);
        /* 16-element sums of groups 8h + (u&1) + 2q, q = 0..3 */
        uint32_t sb = (b * 16 + 8 * h + (u & 1)) * 4;
        r.s0 = (int)ld4(x.s16, sb);
        r.s1 = (int)ld4(x.s16, sb + 8);
        r.s2 = (int)ld4(x.s16, sb + 16);
        r.s3 = (int)ld4(x.s16, sb + 24);
        r.d = __uint_as_float(ld4(x.d, b * 4));
        return r;
    }
    /* sum_i (q_i - 32) * x_i for the four 16-element groups: the unsigned
     * 6-bit codes are dotted, then 32 * (16-element x sum) is subtracted */
    __device__ static inline void isums(const W &w, const X &x, int *out) {
        const uint32_t m4 = 0x0F0F0F0Fu, m2 = 0x30303030u;
        int a0 = 0, a1 = 0, a2 = 0, a3 = 0;
#define TG_Q6_COL(c)                                                         \
        {                                                                    \
            uint32_t la = w.qla.c, lb = w.qlb.c, hh = w.qh.c;                \
            uint32_t q1 = (la & m4) | ((hh << 4) & m2);                      \
            uint32_t q2 = (lb & m4) | ((hh << 2) & m2);                      \
            uint32_t q3 = ((la >> 4) & m4) | (hh & m2);                      \
            uint32_t q4 = ((lb >> 4) & m4) | ((hh >> 2) & m2);               \
            a0 = dot4(q1, x.x0.c, a0);                                       \
            a1 = dot4(q2, x.x1.c, a1);                                       \
            a2 = dot4(q3, x.x2.c, a2);                                       \
            a3 = dot4(q4, x.x3.c, a3);                                       \
        }
        TG_Q6_COL(x) TG_Q6_COL(y) TG_Q6_COL(z) TG_Q6_COL(w)
#undef TG_Q6_COL
        out[0] = a0 - 32 * x.s0;
        out[1] = a1 - 32 * x.s1;
        out[2] = a2 - 32 * x.s2;
        out[3] = a3 - 32 * x.s3;
    }
    /* the item decoded once for several input rows: the 6-bit codes of its
     * four 16-element groups (q[group][column]), their sub-scales, d */
    struct Wd {
        uint32_t q[4][4];
        int sc[4];
        float d;
    };
    __device__ static inline Wd decode(const W &w, int item) {
        const uint32_t m4 = 0x0F0F0F0Fu, m2 = 0x30303030u;
        const uint32_t la[4] = {w.qla.x, w.qla.y, w.qla.z, w.qla.w};
        const uint32_t lb[4] = {w.qlb.x, w.qlb.y, w.qlb.z, w.qlb.w};
        const uint32_t hh[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
        Wd r;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            r.q[0][c] = (la[c] & m4) | ((hh[c] << 4) & m2);
            r.q[1][c] = (lb[c] & m4) | ((hh[c] << 2) & m2);
            r.q[2][c] = ((la[c] >> 4) & m4) | (hh[c] & m2);
            r.q[3][c] = ((lb[c] >> 4) & m4) | ((hh[c] >> 2) & m2);
        }
        const int odd = item & 1;   /* sub-scale byte (u&1) + 2q of sc[8h..8h+7] */
        r.sc[0] = (int)(int8_t)(w.sc.x >> (8 * odd));
        r.sc[1] = (int)(int8_t)(w.sc.x >> (8 * odd + 16));
        r.sc[2] = (int)(int8_t)(w.sc.y >> (8 * odd));
        r.sc[3] = (int)(int8_t)(w.sc.y >> (8 * odd + 16));
        r.d = ref_f16(w.d >> 16);
        return r;
    }
    __device__ static inline float value_d(const Wd &w, const X &x) {
        const uint32_t xs[4][4] = {{x.x0.x, x.x0.y, x.x0.z, x.x0.w},
                                   {x.x1.x, x.x1.y, x.x1.z, x.x1.w},
                                   {x.x2.x, x.x2.y, x.x2.z, x.x2.w},
                                   {x.x3.x, x.x3.y, x.x3.z, x.x3.w}};
        int a[4] = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int g = 0; g < 4; g++) a[g] = dot4(w.q[g][c], xs[g][c], a[g]);
        const int s0 = a[0] - 32 * x.s0, s1 = a[1] - 32 * x.s1, s2 = a[2] - 32 * x.s2, s3 = a[3] - 32 * x.s3;
        int A = w.sc[0] * s0 + w.sc[1] * s1 + w.sc[2] * s2 + w.sc[3] * s3;
        return w.d * x.d * (float)A;
    }
    __device__ static inline float value(const W &w, const X &x, int item) { return value_d(decode(w, item), x); }
    __device__ static inline int isum_index(int item, int i) {
        int u = item & 3;
        return (item >> 2) * 16 + 8 * (u >> 1) + (u & 1) + 2 * i;
    }
};

/* ---- MXFP4: item = one 32-value block (e8m0 byte + 16 code bytes) ---- */
struct FMXFP4 {
    static constexpr int FMT = TG_FMT_MXFP4;
    static constexpr int ITEMS_PER_BLOCK = 1, BLOCK_VALS = 32, BLOCK_BYTES = 17;
    static constexpr int NSUMS = 1;
    struct W { u32x4 c; uint32_t e; };
    struct X { u32x4 a, b; float d; };

    __device__ static inline W load_w(Buf w, uint32_t row_off, int item) {
        uint32_t p = row_off + (uint32_t)item * 17u;
        W r;
        r.e = ld4(w, p);   /* e8m0 byte + 3 code bytes: the low byte is e */
        r.c = ld16(w, p + 1);
        return r;
    }
    template <class R>   /* Q8Row (global) or Q8Lds */
    __device__ static inline X load_x(const R &x, int item) {
        uint32_t o = (uint32_t)(item >> 3) * 256 + (item & 7) * 32;
        X r;
        r.a = ld16(x.qs, o);
        r.b = ld16(x.qs, o + 16);
        r.d = __uint_as_float(ld4(x.d, (item >> 3) * 4));
        return r;
    }
    /* doubled e2m1 table {0,1,2,3,4,6,8,12} by byte permute; codes 8..15 are
     * the negatives, selected per byte from a second permute */
    __device__ static inline uint32_t lut(uint32_t n) {
        const uint32_t pos_lo = 0x03020100u, pos_hi = 0x0C080604u;
        const uint32_t neg_lo = 0xFDFEFF00u, neg_hi = 0xF4F8FAFCu;
        uint32_t idx = n & 0x07070707u;
        uint32_t p = __builtin_amdgcn_perm(pos_hi, pos_lo, idx);
        uint32_t q = __builtin_amdgcn_perm(neg_hi, neg_lo, idx);
        uint32_t sel = ((n >> 3) & 0x01010101u) * 0xFFu;
        return (p & ~sel) | (q & sel);
    }
    __device__ static inline void isums(const W &w, const X &x, int *out) {
        const uint32_t m = 0x0F0F0F0Fu;
        int acc = 0;
        acc = dot4(lut(w.c.x & m), x.a.x, acc);
        acc = dot4(lut(w.c.y & m), x.a.y, acc);
        acc = dot4(lut(w.c.z & m), x.a.z, acc);
        acc = dot4(lut(w.c.w & m), x.a.w, acc);
        acc = dot4(lut((w.c.x >> 4) & m), x.b.x, acc);
        acc = dot4(lut((w.c.y >> 4) & m), x.b.y, acc);
        acc = dot4(lut((w.c.z >> 4) & m), x.b.z, acc);
        acc = dot4(lut((w.c.w >> 4) & m), x.b.w, acc);
        out[0] = acc;
    }
    __device__ static inline float value(const W &w, const X &x, int item) {
        int s;
        isums(w, x, &s);
        return x.d * e8m0_half(w.e & 0xFFu) * (float)s;
    }
    __device__ static inline int isum_index(int item, int) { return item; }
};

/* ---- Q8_0 weights: item = one 34-byte block (f16 d + 32 int8) ---- */
struct FQ80 {
    static constexpr int FMT = TG_FMT_Q80;
    static constexpr int ITEMS_PER_BLOCK = 1, BLOCK_VALS = 32, BLOCK_BYTES = 34;
    static constexpr int NSUMS = 1;
    struct W { u32x4 q0, q1; uint32_t d; };
    struct X { u32x4 a, b; float d; };

    __device__ static inline W load_w(Buf w, uint32_t row_off, int item) {
        uint32_t p = row_off + (uint32_t)item * 34u;
        W r;
        r.d = ld4(w, p);   /* d + 2 quant bytes: ref_f16 keeps the low half */
        r.q0 = ld16(w, p + 2);
        r.q1 = ld16(w, p + 18);
        return r;
    }
    __device__ static inline X load_x(const Q8Row &x, int item) {
        FMXFP4::X t = FMXFP4::load_x(x, item);
        X r;
        r.a = t.a;
        r.b = t.b;
        r.d = t.d;
        return r;
    }
    __device__ static inline void isums(const W &w, const X &x, int *out) {
        int acc = 0;
        acc = dot4(w.q0.x, x.a.x, acc); acc = dot4(w.q0.y, x.a.y, acc);
        acc = dot4(w.q0.z, x.a.z, acc); acc = dot4(w.q0.w, x.a.w, acc);
        acc = dot4(w.q1.x, x.b.x, acc); acc = dot4(w.q1.y, x.b.y, acc);
        acc = dot4(w.q1.z, x.b.z, acc); acc = dot4(w.q1.w, x.b.w, acc);
        out[0] = acc;
    }
    __device__ static inline float value(const W &w, const X &x, int) {
        int s;
        isums(w, x, &s);
        return x.d * ref_f16(w.d) * (float)s;
    }
    __device__ static inline int isum_index(int item, int) { return item; }
};

/* ---- F16 weights: item = 8 halfs, against the unquantized f32 row ----
 * Rows are multiples of 32 values, so every value goes through the
 * reference's vectorised loop, whose vcvt_f32_f16 is the IEEE conversion
 * (csrc/libtinygiant.c:641-648). */
struct FF16 {
    static constexpr int FMT = TG_FMT_F16;
    static constexpr int ITEMS_PER_BLOCK = 1, BLOCK_VALS = 8, BLOCK_BYTES = 16;
    static constexpr int NSUMS = 0;
    struct W { u32x4 h; };
    struct X { u32x4 a, b; };

    __device__ static inline W load_w(Buf w, uint32_t row_off, int item) {
        W r;
        r.h = ld16(w, row_off + (uint32_t)item * 16u);
        return r;
    }
    __device__ static inline X load_x(const Q8Row &x, int item) {
        X r;
        r.a = ld16(x.f, (uint32_t)item * 32u);
        r.b = ld16(x.f, (uint32_t)item * 32u + 16u);
        return r;
    }
    __device__ static inline float h2f(uint32_t h) {
        return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
    }
    __device__ static inline float value(const W &w, const X &x, int) {
        float s = h2f(w.h.x) * __uint_as_float(x.a.x);
        s = fmaf(h2f(w.h.x >> 16), __uint_as_float(x.a.y), s);
        s = fmaf(h2f(w.h.y), __uint_as_float(x.a.z), s);
        s = fmaf(h2f(w.h.y >> 16), __uint_as_float(x.a.w), s);
        s = fmaf(h2f(w.h.z), __uint_as_float(x.b.x), s);
        s = fmaf(h2f(w.h.z >> 16), __uint_as_float(x.b.y), s);
        s = fmaf(h2f(w.h.w), __uint_as_float(x.b.z), s);
        s = fmaf(h2f(w.h.w >> 16), __uint_as_float(x.b.w), s);
        return s;
    }
    __device__ static inline void isums(const W &, const X &, int *) {}
    __device__ static inline int isum_index(int, int) { return 0; }
};

/* expert activation (csrc/libtinygiant.c:1250-1257; the
 * comparisons keep a NaN as the reference's if-chains do): SiLU(g) * u, or the
 * clamped gpt-oss form g * sigmoid(1.702 g) * (u + 1) */
__device__ inline float act_fn(int act, float g, float u) {
    if (act == TG_ACT_GPTOSS) {
        g = g > 7.f ? 7.f : g;
        u = u > 7.f ? 7.f : (u < -7.f ? -7.f : u);
        return g / (1.f + expf(-1.702f * g)) * (u + 1.f);
    }
    return g / (1.f + expf(-g)) * u;
}


}  // namespace tg
#endif
