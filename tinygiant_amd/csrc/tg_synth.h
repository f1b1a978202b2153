/*
 * tg_synth.h -- seeded synthetic weight generator shared by host and device.
 *
 * Integer-only, so the host (tests, CPU baseline) and the GPU fill kernel
 * produce identical bytes for the same (kind, seed, offset).
 *
 * Byte b of a tensor is byte (b & 7) of splitmix64-finalised word b >> 3,
 * then the scale fields of each quant block are overwritten:
 *   Q4_K  (144 B): d, dmin = f16 of U[1e-3, 2e-2]          bytes 0-3
 *   Q6_K  (210 B): d       = f16 of U[1e-3, 2e-2]          bytes 208-209
 *   MXFP4 ( 17 B): e8m0 exponent uniform in {118..130}      byte 0
 *   Q8_0  ( 34 B): d       = f16 of U[1e-3, 2e-2]          bytes 0-1
 * Everything else (Q4_K 6-bit scale bytes, nibbles, Q6_K ql/qh and int8
 * sub-scales, fp4 codes, int8 values) is a uniform random byte.
 */
#ifndef TG_SYNTH_H
#define TG_SYNTH_H
#include <stdint.h>

#if defined(__HIPCC__)
#define TG_HD __host__ __device__
#else
#define TG_HD
#endif

enum { TG_SYN_RAW = -1, TG_SYN_Q4K = 0, TG_SYN_Q6K = 2, TG_SYN_MXFP4 = 3, TG_SYN_Q80 = 4 };

static TG_HD inline uint64_t tg_syn_fin(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* word i of the stream for `seed` (splitmix64 output number i+1) */
static TG_HD inline uint64_t tg_syn_word(uint64_t seed, uint64_t i) {
    return tg_syn_fin(seed + (i + 1) * 0x9E3779B97F4A7C15ull);
}

/* Round-to-nearest-even f16 of a positive fixed-point value v * 2^-40
 * (v > 0, value in the f16 normal range). */
static TG_HD inline uint16_t tg_syn_fx40_to_f16(uint64_t v) {
    int p = 63;
    while (!((v >> p) & 1)) p--;
    int e = p - 40;                      /* value = 1.f * 2^e */
    int sh = p - 10;                     /* bits below the 10-bit mantissa */
    uint64_t m = v >> sh;                /* 11 bits with the leading one */
    uint64_t rem = v & ((1ull << sh) - 1), half = 1ull << (sh - 1);
    if (rem > half || (rem == half && (m & 1))) m++;
    if (m == 2048) { m = 1024; e++; }
    return (uint16_t)(((e + 15) << 10) | (m & 0x3FF));
}

/* f16 of U[1e-3, 2e-2] from a 24-bit uniform integer u */
static TG_HD inline uint16_t tg_syn_scale_f16(uint32_t u24) {
    const uint64_t lo = 1099511628ull;                 /* 1e-3 * 2^40 */
    uint64_t v = lo + ((uint64_t)u24 * 1245184ull) / 1000ull;  /* + u/2^24 * 0.019 * 2^40 */
    return tg_syn_fx40_to_f16(v);
}

static TG_HD inline int tg_syn_block_bytes(int kind) {
    switch (kind) {
        case TG_SYN_Q4K: return 144;
        case TG_SYN_Q6K: return 210;
        case TG_SYN_MXFP4: return 17;
        case TG_SYN_Q80: return 34;
        default: return 1;
    }
}

/* byte `pos` of a tensor of the given kind */
static TG_HD inline uint8_t tg_syn_byte(int kind, uint64_t seed, uint64_t pos) {
    const uint64_t salt = 0xD1B54A32D192ED03ull;
    uint8_t b = (uint8_t)(tg_syn_word(seed, pos >> 3) >> (8 * (pos & 7)));
    if (kind == TG_SYN_RAW) return b;
    uint64_t bb = (uint64_t)tg_syn_block_bytes(kind);
    uint64_t blk = pos / bb, off = pos % bb;
    if (kind == TG_SYN_Q4K && off < 4) {
        uint64_t w = tg_syn_word(seed ^ salt, blk);
        uint16_t h = tg_syn_scale_f16((uint32_t)((off < 2 ? w : (w >> 24)) & 0xFFFFFF));
        return (uint8_t)(h >> (8 * (off & 1)));
    }
    if (kind == TG_SYN_Q6K && off >= 208) {
        uint16_t h = tg_syn_scale_f16((uint32_t)(tg_syn_word(seed ^ salt, blk) & 0xFFFFFF));
        return (uint8_t)(h >> (8 * (off - 208)));
    }
    if (kind == TG_SYN_MXFP4 && off == 0) return (uint8_t)(118 + tg_syn_word(seed ^ salt, blk) % 13);
    if (kind == TG_SYN_Q80 && off < 2) {
        uint16_t h = tg_syn_scale_f16((uint32_t)(tg_syn_word(seed ^ salt, blk) & 0xFFFFFF));
        return (uint8_t)(h >> (8 * off));
    }
    return b;
}

#endif
