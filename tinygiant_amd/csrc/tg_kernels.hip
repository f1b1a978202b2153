/*
 * tg_kernels.hip -- HIP kernels of libtinygiant_hip for gfx950 and their
 * stream-ordered launchers.
 *
 *   k_quantize_q8   activation rows -> q8 blocks   (quantize_q8, csrc/libtinygiant.c:169-208)
 *   k_gemv          y[j][r] = dot(W[r], x_j) + bias[r]   (tg_matmul, :908-931)
 *   k_moe_a         hidden = act(gate.x + bg, up.x + bu) per (expert, row)  (moe_phase_a, :1279-1327)
 *   k_moe_b         part = w * (down.q8(hidden) + bd)                      (moe_phase_b, :1329-1384)
 *   k_moe_combine   out[row] += part, experts in index order               (:1428-1434)
 *   k_isums         per-sub-block integer dot sums (bit-exactness probe)
 *   k_rms_norm_q8   x * 1/sqrt(mean(x^2)+eps) * w, optionally q8 of it     (tg_rms_norm, :680-698)
 *   k_synth_fill    seeded synthetic weights (tg_synth.h)
 *
 * Every weight and activation read goes through a raw buffer resource sized
 * to its tensor, so an indexing slip reads zeros instead of faulting.
 */
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include <algorithm>
#include <functional>

#include "tg_device.hpp"
#include "tg_kernels.h"
#include "tg_synth.h"

namespace tg {

/* ======================= q8 quantization ======================= */

/* One wave per 256-value block: lane l owns values 4l..4l+3. */
__global__ __launch_bounds__(256) void k_quantize_q8(const float *__restrict__ x, int ncols, int nrows,
                                                     long xstride, Q8Rows out) {
    const int lane = threadIdx.x & 63;
    const int wave = (int)((blockIdx.x * (size_t)blockDim.x + threadIdx.x) >> 6);
    const int nb = out.nb;
    if (wave >= nrows * nb) return;   /* uniform per wave */
    const int r = wave / nb, b = wave % nb;
    const int n = min(256, ncols - b * 256);
    Buf xb = make_buf(x + (size_t)r * xstride + (size_t)b * 256, (uint32_t)n * 4u);
    u32x4 raw = ld16(xb, (uint32_t)lane * 16u);   /* zeros past n */
    q8_block_store(__uint_as_float(raw.x), __uint_as_float(raw.y), __uint_as_float(raw.z), __uint_as_float(raw.w),
                   lane, out, r, b);
}

/* RMSNorm of one row per workgroup, wave w owning the 256-value blocks
 * w, w + NWR, ... (at most RMS_BPW of them), lane l values 4l..4l+3 of each:
 * y = (x * (1/sqrt(ss/n + eps))) * w (tg_rms_norm, csrc/libtinygiant.c:680-698;
 * ss summed per lane, then over the wave, then over the waves in order).
 * Every load of the row is issued before any is used.  With q8 rows given,
 * y is quantized in place of a separate k_quantize_q8 over it (same bits). */
constexpr int RMS_WAVES = 16, RMS_BPW = 4;
__global__ __launch_bounds__(RMS_WAVES * 64) void k_rms_norm_q8(const float *__restrict__ x, const float *__restrict__ w,
                                                                float *__restrict__ y, int n, float eps, Q8Rows q) {
    __shared__ float red[RMS_WAVES];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int r = blockIdx.x;
    Buf xb = make_buf(x + (size_t)r * n, (uint32_t)n * 4u);
    Buf wb = make_buf(w, w ? (uint32_t)n * 4u : 0u);
    float v[RMS_BPW][4], g[RMS_BPW][4];
#pragma unroll
    for (int i = 0; i < RMS_BPW; i++) {
        const uint32_t o = (uint32_t)((wave + nw * i) * 256 + 4 * lane) * 4u;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            v[i][c] = __uint_as_float(ld4(xb, o + 4u * c));   /* zeros past n */
            g[i][c] = w ? __uint_as_float(ld4(wb, o + 4u * c)) : 1.f;
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < RMS_BPW; i++)
#pragma unroll
        for (int c = 0; c < 4; c++) ss += v[i][c] * v[i][c];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int i = 0; i < nw; i++) tot += red[i];
    const float scale = 1.f / sqrtf(tot / (float)n + eps);
    float *yr = y + (size_t)r * n;
#pragma unroll
    for (int i = 0; i < RMS_BPW; i++) {
        const int b = wave + nw * i;
        if (b * 256 >= n) break;   /* uniform per wave */
        float o4[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            o4[c] = (v[i][c] * scale) * g[i][c];
            if (b * 256 + 4 * lane + c < n) yr[b * 256 + 4 * lane + c] = o4[c];
        }
        if (q.qs) q8_block_store(o4[0], o4[1], o4[2], o4[3], lane, q, r, b);
    }
}

/* ======================= generic GEMV ======================= */

constexpr uint32_t ROW_OOB = 0x80000000u;   /* past every weight buffer: reads zeros, touches no memory */

/* acc[m] += the lane's share of dot(row of matrix m, x): items sl, sl + S,
 * ... below nitems, added in item order.  Loads go out in batches of TB
 * items before any is used, so a row costs ceil(T / TB) memory round trips
 * instead of T.  An invalid row (rv false) or an item past the row is read
 * at an out-of-range offset and adds nothing. */
template <class F, int S, int TB, int NM, class R>
__device__ inline void row_dots(const Buf (&w)[NM], uint32_t roff, bool rv, const R &xr, int sl, int nitems,
                                int T, float (&acc)[NM]) {
    for (int t0 = 0; t0 < T; t0 += TB) {
        typename F::X xs[TB];
        typename F::W ws[NM][TB];
#pragma unroll
        for (int u = 0; u < TB; u++) {
            const int item = sl + (t0 + u) * S;
            const bool iv = rv && t0 + u < T && item < nitems;
            xs[u] = F::load_x(xr, iv ? item : 0);
#pragma unroll
            for (int m = 0; m < NM; m++) ws[m][u] = F::load_w(w[m], iv ? roff : ROW_OOB, iv ? item : 0);
        }
#pragma unroll
        for (int u = 0; u < TB; u++) {
            const int item = sl + (t0 + u) * S;
            if (rv && t0 + u < T && item < nitems) {
#pragma unroll
                for (int m = 0; m < NM; m++) acc[m] += F::value(ws[m][u], xs[u], item);
            }
        }
    }
}

/* W: nrows rows of rb bytes.  For each activation row j < k:
 *   y[j*ystride + r] = dot(W[r], x_j) + bias[r]
 * Each wave takes `rows_per_wave` consecutive rows in steps of 64/S. */
template <class F, int S, int TB>
__device__ inline void gemv_rows(const uint8_t *__restrict__ W, uint32_t rb, int nrows,
                                 const float *__restrict__ bias, const Q8Rows &x, int k, float *y, long ystride,
                                 int nitems, int T, int rows_per_wave) {
    constexpr int G = 64 / S;
    const int lane = threadIdx.x & 63;
    const int seg = lane / S, sl = lane % S;
    const int wave = (int)((blockIdx.x * (size_t)blockDim.x + threadIdx.x) >> 6);
    const int row0 = wave * rows_per_wave;
    if (row0 >= nrows) return;
    Buf wb = make_buf(W + (size_t)row0 * rb, (uint32_t)((size_t)min(rows_per_wave, nrows - row0) * rb));
    for (int j = 0; j < k; j++) {
        Q8Row xr = q8_row(x, j);
        for (int rs = 0; rs < rows_per_wave; rs += G) {
            const int rl = rs + seg, r = row0 + rl;
            const bool rv = rl < rows_per_wave && r < nrows;
            float acc[1] = {0.f};
            const Buf ws[1] = {wb};
            row_dots<F, S, TB, 1>(ws, (uint32_t)rl * rb, rv, xr, sl, nitems, T, acc);
            const float v = seg_sum<S>(acc[0]);
            if (rv && sl == 0) y[(size_t)j * ystride + r] = v + (bias ? bias[r] : 0.f);
        }
    }
}

template <class F, int S, int TB>
__global__ __launch_bounds__(256) void k_gemv(const uint8_t *__restrict__ W, uint32_t rb, int nrows,
                                              const float *__restrict__ bias, Q8Rows x, int k, float *y,
                                              long ystride, int nitems, int T, int rows_per_wave) {
    gemv_rows<F, S, TB>(W, rb, nrows, bias, x, k, y, ystride, nitems, T, rows_per_wave);
}

/* Several matrices of one format and width against the same rows in one
 * launch: blockIdx.y picks the matrix. */
template <class F, int S, int TB>
__global__ __launch_bounds__(256) void k_gemv_multi(GemvJobs jobs, uint32_t rb, Q8Rows x, int k, int nitems, int T,
                                                    int rows_per_wave) {
    const GemvJob &jb = jobs.j[blockIdx.y];
    gemv_rows<F, S, TB>(jb.W, rb, jb.nrows, jb.bias, x, k, jb.y, jb.ystride, nitems, T, rows_per_wave);
}

/* q8 of one f32 row of ncols (a multiple of 256) values into LDS by the
 * workgroup's 4 waves, block b by wave b % 4: the arithmetic of
 * k_quantize_q8 */
__device__ inline void q8_row_lds(const float *__restrict__ x, int ncols, uint8_t *xq, float *xd, int32_t *xs32,
                                  int32_t *xs16) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = ncols / 256;
    for (int b = wave; b < nb; b += 4) {
        Buf xb = make_buf(x + (size_t)b * 256, 1024u);
        const u32x4 raw = ld16(xb, (uint32_t)lane * 16u);
        const Q8Quant q = q8_block_quant(__uint_as_float(raw.x), __uint_as_float(raw.y), __uint_as_float(raw.z),
                                         __uint_as_float(raw.w));
        reinterpret_cast<uint32_t *>(xq + b * 256)[lane] = q.packed;
        if ((lane & 3) == 0) xs16[b * 16 + (lane >> 2)] = q.s16;
        if ((lane & 7) == 0) xs32[b * 8 + (lane >> 3)] = q.s32;
        if (lane == 0) xd[b] = q.sc;
    }
}

constexpr int Q8X_MAXP = 4;   /* row passes per wave whose weights are loaded before the q8 */

/* One job's share of k_gemv_q8x: the rows of gemv_rows for wave `wave` of
 * the job, against the q8 row the workgroup builds in LDS.  When each lane
 * holds one item of a row (T == 1), the wave's weights are requested before
 * the q8 is built, so the two latencies overlap; the dots are the same
 * operations in the same order as gemv_rows. */
template <class F, int S, int TB>
__device__ inline void q8x_job(const GemvJob &jb, uint32_t rb, const float *__restrict__ x, int ncols, int nitems,
                               int T, int rows_per_wave, int wave, uint8_t *xq, float *xd, int32_t *xs32,
                               int32_t *xs16) {
    constexpr int G = 64 / S;
    const int lane = threadIdx.x & 63;
    const int seg = lane / S, sl = lane % S;
    const int row0 = wave * rows_per_wave;
    const int nrw = max(0, min(rows_per_wave, jb.nrows - row0));   /* this wave's rows (0 past the job) */
    const Buf wb = make_buf(jb.W + (size_t)min(row0, jb.nrows) * rb, (uint32_t)((size_t)nrw * rb));
    const int P = (rows_per_wave + G - 1) / G;
    const bool pre = T == 1 && P <= Q8X_MAXP;
    typename F::W wp[Q8X_MAXP];
    if (pre) {
#pragma unroll
        for (int p = 0; p < Q8X_MAXP; p++) {
            const int rl = p * G + seg;
            const bool iv = p < P && rl < nrw && sl < nitems;
            wp[p] = F::load_w(wb, iv ? (uint32_t)rl * rb : ROW_OOB, iv ? sl : 0);
        }
    }
    q8_row_lds(x, ncols, xq, xd, xs32, xs16);
    __syncthreads();
    if (nrw == 0) return;
    const Q8Lds xr = {xq, reinterpret_cast<const uint8_t *>(xd), reinterpret_cast<const uint8_t *>(xs32),
                      reinterpret_cast<const uint8_t *>(xs16)};
    if (pre) {
#pragma unroll
        for (int p = 0; p < Q8X_MAXP; p++) {
            const int rl = p * G + seg, r = row0 + rl;
            if (p >= P) break;
            const bool rv = rl < nrw;
            float acc = 0.f;
            if (rv && sl < nitems) acc += F::value(wp[p], F::load_x(xr, sl), sl);
            const float v = seg_sum<S>(acc);
            if (rv && sl == 0) jb.y[r] = v + (jb.bias ? jb.bias[r] : 0.f);
        }
    } else {
        for (int rs = 0; rs < rows_per_wave; rs += G) {
            const int rl = rs + seg, r = row0 + rl;
            const bool rv = rl < nrw;
            float acc[1] = {0.f};
            const Buf ws[1] = {wb};
            row_dots<F, S, TB, 1>(ws, (uint32_t)rl * rb, rv, xr, sl, nitems, T, acc);
            const float v = seg_sum<S>(acc[0]);
            if (rv && sl == 0) jb.y[r] = v + (jb.bias ? jb.bias[r] : 0.f);
        }
    }
}

/* q8 of one f32 row and the GEMVs of up to three Q4_K / Q6_K matrices of
 * its width in one launch (decode attention's Q, K and V projections).
 * Every workgroup quantizes the row into LDS itself, with the arithmetic of
 * k_quantize_q8, then runs its rows as k_gemv_multi does, so the results are
 * the same bits.  The grid is flat: job j owns workgroups
 * [map.wg0[j], map.wg0[j + 1]).  Workgroup 0 also clears n_zero words at
 * `zero` (the counters of a kernel that follows). */
template <int S, int TB>
__global__ __launch_bounds__(256) void k_gemv_q8x(GemvJobs jobs, GemvQ8xMap map, const float *__restrict__ x,
                                                  int ncols, int nitems, int T, int rows_per_wave, unsigned *zero,
                                                  int n_zero) {
    __shared__ __attribute__((aligned(16))) uint8_t xq[Q8X_MAX_BLOCKS * 256];
    __shared__ __attribute__((aligned(16))) float xd[Q8X_MAX_BLOCKS];
    __shared__ __attribute__((aligned(16))) int32_t xs32[Q8X_MAX_BLOCKS * 8];
    __shared__ __attribute__((aligned(16))) int32_t xs16[Q8X_MAX_BLOCKS * 16];
    if (blockIdx.x == 0 && (int)threadIdx.x < n_zero)
        __hip_atomic_store(zero + threadIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    int j = 0;
    while (j < 2 && (int)blockIdx.x >= map.wg0[j + 1]) j++;
    const int jw = ((int)blockIdx.x - map.wg0[j]) * 4 + (int)(threadIdx.x >> 6);
    if (map.fmt[j] == TG_FMT_Q6K)
        q8x_job<FQ6K, S, TB>(jobs.j[j], map.rb[j], x, ncols, nitems, T, rows_per_wave, jw, xq, xd, xs32, xs16);
    else
        q8x_job<FQ4K, S, TB>(jobs.j[j], map.rb[j], x, ncols, nitems, T, rows_per_wave, jw, xq, xd, xs32, xs16);
}

/* ======================= MoE phases ======================= */

/* Phase A: grid (x: wave groups over the I rows, y: pair).  hidden[p][r] of
 * the pair's expert; the pairs of one expert run side by side (their weight
 * rows come from the L2 after the first). */
template <class F, int S, int TB>
__global__ __launch_bounds__(256) void k_moe_a(MoeArgs a, int nitems, int T, int rows_per_wave) {
    constexpr int G = 64 / S;
    const int p = blockIdx.y;
    const int e = a.p_exp[p];
    const int lane = threadIdx.x & 63;
    const int seg = lane / S, sl = lane % S;
    const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int row0 = wave * rows_per_wave;
    if (row0 >= a.I) return;
    const uint32_t rb = a.gate_rb;
    const size_t mbytes = (size_t)a.I * rb;
    Buf gw = make_buf((const void *)a.gate[e], (uint32_t)mbytes);
    Buf uw = make_buf((const void *)a.up[e], (uint32_t)mbytes);
    const float *gb = a.gbias ? (const float *)a.gbias[e] : nullptr;
    const float *ub = a.ubias ? (const float *)a.ubias[e] : nullptr;
    {
        Q8Row xr = q8_row(a.xq, a.p_row[p]);
        for (int rs = 0; rs < rows_per_wave; rs += G) {
            const int r = row0 + rs + seg;
            const bool rv = rs + seg < rows_per_wave && r < a.I;
            float acc[2] = {0.f, 0.f};
            const Buf ws[2] = {gw, uw};
            row_dots<F, S, TB, 2>(ws, (uint32_t)r * rb, rv, xr, sl, nitems, T, acc);
            float vg = seg_sum<S>(acc[0]);
            float vu = seg_sum<S>(acc[1]);
            if (rv && sl == 0) {
                if (gb) vg += gb[r];
                if (ub) vu += ub[r];
                a.hidden[(size_t)p * a.I + r] = act_fn(a.act, vg, vu);
            }
        }
    }
}

/* Phase B: grid (x: wave groups over the D rows, y: pair).  Only pairs whose
 * expert's down format is `fmt` run (one launch per format present). */
template <class F, int S, int TB>
__global__ __launch_bounds__(256) void k_moe_b(MoeArgs a, int fmt, uint32_t rb, int nitems, int T,
                                               int rows_per_wave) {
    constexpr int G = 64 / S;
    const int p = blockIdx.y;
    const int e = a.p_exp[p];
    if (a.down_fmt[e] != fmt) return;
    const int lane = threadIdx.x & 63;
    const int seg = lane / S, sl = lane % S;
    const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int row0 = wave * rows_per_wave;
    if (row0 >= a.D) return;
    Buf dw = make_buf((const void *)a.down[e], (uint32_t)((size_t)a.D * rb));
    const float *db = a.dbias ? (const float *)a.dbias[e] : nullptr;
    {
        Q8Row xr = q8_row(a.hq, p);
        const float w = a.p_w[p];
        for (int rs = 0; rs < rows_per_wave; rs += G) {
            const int r = row0 + rs + seg;
            const bool rv = rs + seg < rows_per_wave && r < a.D;
            float acc[1] = {0.f};
            const Buf ws[1] = {dw};
            row_dots<F, S, TB, 1>(ws, (uint32_t)r * rb, rv, xr, sl, nitems, T, acc);
            const float v = seg_sum<S>(acc[0]);
            if (rv && sl == 0) a.part[(size_t)p * a.D + r] = w * (v + (db ? db[r] : 0.f));
        }
    }
}

/* out[row][c] += part[p][c] for the pairs p of `row`, in expert order. */
__global__ __launch_bounds__(256) void k_moe_combine(MoeArgs a) {
    const size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (idx >= (size_t)a.k * a.D) return;
    const int row = (int)(idx / a.D), c = (int)(idx % a.D);
    float o = a.out[idx];
    for (int q = a.r_off[row]; q < a.r_off[row + 1]; q++) o += a.part[(size_t)a.r_pair[q] * a.D + c];
    a.out[idx] = o;
}

/* ======================= integer-sum probe ======================= */

template <class F, int S>
__global__ __launch_bounds__(256) void k_isums(const uint8_t *__restrict__ W, uint32_t rb, int nrows, Q8Rows x,
                                               int nitems, int T, int nsums_row, int32_t *out) {
    constexpr int G = 64 / S;
    const int lane = threadIdx.x & 63;
    const int seg = lane / S, sl = lane % S;
    const int wave = (int)((blockIdx.x * (size_t)blockDim.x + threadIdx.x) >> 6);
    const int r = wave * G + seg;
    if (r >= nrows) return;
    Buf wb = make_buf(W, (uint32_t)((size_t)nrows * rb));
    Q8Row xr = q8_row(x, 0);
    for (int t = 0; t < T; t++) {
        const int item = sl + t * S;
        if (item >= nitems) continue;
        typename F::W w = F::load_w(wb, (uint32_t)r * rb, item);
        typename F::X xs = F::load_x(xr, item);
        int s[F::NSUMS > 0 ? F::NSUMS : 1];
        F::isums(w, xs, s);
        for (int i = 0; i < F::NSUMS; i++) out[(size_t)r * nsums_row + F::isum_index(item, i)] = s[i];
    }
}

/* ======================= small helpers ======================= */

__global__ __launch_bounds__(256) void k_synth_fill(int kind, uint64_t seed, uint8_t *dst, uint64_t nbytes) {
    const uint64_t nwords = (nbytes + 7) / 8;
    for (uint64_t wi = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; wi < nwords;
         wi += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t p0 = wi * 8;
        if (p0 + 8 <= nbytes) {
            uint64_t v = 0;
            for (int b = 0; b < 8; b++) v |= (uint64_t)tg_syn_byte(kind, seed, p0 + b) << (8 * b);
            reinterpret_cast<uint64_t *>(dst)[wi] = v;
        } else {
            for (uint64_t p = p0; p < nbytes; p++) dst[p] = tg_syn_byte(kind, seed, p);
        }
    }
}

/* Plain 16-byte-per-lane copy: the reference kernel for measured HBM
 * bandwidth and for calibrating the FETCH_SIZE / WRITE_SIZE counters. */
__global__ __launch_bounds__(256) void k_copy(const u32x4 *__restrict__ src, u32x4 *__restrict__ dst, uint64_t n16) {
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

/* ======================= launchers ======================= */

static int pick_S(int nitems, int *T) {
    /* fewest lane slots S*T (S power of two <= 64); ties go to larger S */
    int bestS = 64, bestT = (nitems + 63) / 64, best = bestS * bestT;
    for (int S = 32; S >= 8; S >>= 1) {
        int t = (nitems + S - 1) / S;
        if (S * t < best) {
            best = S * t;
            bestS = S;
            bestT = t;
        }
    }
    *T = bestT;
    return bestS;
}

int items_per_row(int fmt, int ncols) {
    switch (fmt) {
        case TG_FMT_Q4K: return ncols / 256 * 4;
        case TG_FMT_Q6K: return ncols / 256 * 4;
        case TG_FMT_MXFP4: return ncols / 32;
        case TG_FMT_Q80: return ncols / 32;
        case TG_FMT_F16: return ncols / 8;
        default: return -1;
    }
}

uint32_t row_bytes(int fmt, int ncols) {
    switch (fmt) {
        case TG_FMT_Q4K: return (uint32_t)(ncols / 256) * 144u;
        case TG_FMT_Q6K: return (uint32_t)(ncols / 256) * 210u;
        case TG_FMT_MXFP4: return (uint32_t)(ncols / 32) * 17u;
        case TG_FMT_Q80: return (uint32_t)(ncols / 32) * 34u;
        default: return (uint32_t)ncols * 2u;
    }
}

#define TG_DISPATCH_S(S_, CALL) \
    switch (S_) {               \
        case 8: CALL(8); break; \
        case 16: CALL(16); break; \
        case 32: CALL(32); break; \
        default: CALL(64); break; \
    }
/* S and the load batch TB (1, 2 or 4 items per lane in flight) */
#define TG_DISPATCH_TB(TB_, S_, CALL)   \
    switch (TB_) {                      \
        case 1: CALL(S_, 1); break;     \
        case 2: CALL(S_, 2); break;     \
        default: CALL(S_, 4); break;    \
    }
#define TG_DISPATCH_ST(S_, TB_, CALL)                  \
    switch (S_) {                                      \
        case 8: TG_DISPATCH_TB(TB_, 8, CALL) break;    \
        case 16: TG_DISPATCH_TB(TB_, 16, CALL) break;  \
        case 32: TG_DISPATCH_TB(TB_, 32, CALL) break;  \
        default: TG_DISPATCH_TB(TB_, 64, CALL) break;  \
    }
static int pick_TB(int T) { return T >= 3 ? 4 : T; }

#define TG_DISPATCH_F(fmt, BODY)                    \
    switch (fmt) {                                  \
        case TG_FMT_Q4K: { typedef FQ4K F; BODY; } break;   \
        case TG_FMT_Q6K: { typedef FQ6K F; BODY; } break;   \
        case TG_FMT_MXFP4: { typedef FMXFP4 F; BODY; } break; \
        case TG_FMT_Q80: { typedef FQ80 F; BODY; } break;   \
        default: { typedef FF16 F; BODY; } break;   \
    }

void launch_quantize(const float *x, int ncols, int nrows, long xstride, const Q8Rows &out, hipStream_t st) {
    const int waves = nrows * out.nb;
    if (waves <= 0) return;
    hipLaunchKernelGGL(k_quantize_q8, dim3((waves + 3) / 4), dim3(256), 0, st, x, ncols, nrows, xstride, out);
}

void launch_gemv(int fmt, const uint8_t *W, int nrows, int ncols, const float *bias, const Q8Rows &x, int k,
                 float *y, long ystride, hipStream_t st) {
    int T;
    const int nitems = items_per_row(fmt, ncols);
    const int S = pick_S(nitems, &T);
    const uint32_t rb = row_bytes(fmt, ncols);
    const int G = 64 / S;
    const int rpw = G * 2;
    const int waves = (nrows + rpw - 1) / rpw;
    dim3 grid((waves + 3) / 4);
    const int TB = pick_TB(T);
#define CALL(S_, TB_) \
    hipLaunchKernelGGL((k_gemv<F, S_, TB_>), grid, dim3(256), 0, st, W, rb, nrows, bias, x, k, y, ystride, nitems, T, rpw)
    TG_DISPATCH_F(fmt, TG_DISPATCH_ST(S, TB, CALL))
#undef CALL
}

void launch_gemv_multi(int fmt, const GemvJobs &jobs, int njobs, int ncols, const Q8Rows &x, int k, hipStream_t st) {
    int T;
    const int nitems = items_per_row(fmt, ncols);
    const int S = pick_S(nitems, &T);
    const uint32_t rb = row_bytes(fmt, ncols);
    const int rpw = (64 / S) * 2;
    int most = 0;
    for (int i = 0; i < njobs; i++) most = std::max(most, jobs.j[i].nrows);
    const int waves = (most + rpw - 1) / rpw;
    dim3 grid((waves + 3) / 4, njobs);
    const int TB = pick_TB(T);
#define CALL(S_, TB_) \
    hipLaunchKernelGGL((k_gemv_multi<F, S_, TB_>), grid, dim3(256), 0, st, jobs, rb, x, k, nitems, T, rpw)
    TG_DISPATCH_F(fmt, TG_DISPATCH_ST(S, TB, CALL))
#undef CALL
}

bool gemv_q8x_ok(const int *fmts, int njobs, int ncols) {
    if (njobs < 1 || njobs > 3 || ncols <= 0 || ncols % 256 || ncols > Q8X_MAX_BLOCKS * 256) return false;
    for (int i = 0; i < njobs; i++)
        if (fmts[i] != TG_FMT_Q4K && fmts[i] != TG_FMT_Q6K) return false;
    return true;
}

void launch_gemv_q8x(const int *fmts, const GemvJobs &jobs, int njobs, int ncols, const float *x, unsigned *zero,
                     int n_zero, hipStream_t st) {
    int T;
    const int nitems = items_per_row(TG_FMT_Q4K, ncols);   /* Q6_K rows have as many items */
    const int S = pick_S(nitems, &T);
    const int rpw = (64 / S) * 2;
    GemvQ8xMap m;
    int wg = 0;
    for (int i = 0; i < 3; i++) {
        m.wg0[i] = wg;
        if (i < njobs) {
            m.fmt[i] = fmts[i];
            m.rb[i] = row_bytes(fmts[i], ncols);
            const int waves = (jobs.j[i].nrows + rpw - 1) / rpw;
            wg += (waves + 3) / 4;
        } else {
            m.fmt[i] = TG_FMT_Q4K;
            m.rb[i] = 0;
        }
    }
    m.wg0[3] = wg;
    const int TB = pick_TB(T);
#define CALL(S_, TB_) \
    hipLaunchKernelGGL((k_gemv_q8x<S_, TB_>), dim3(wg), dim3(256), 0, st, jobs, m, x, ncols, nitems, T, rpw, zero, n_zero)
    TG_DISPATCH_ST(S, TB, CALL)
#undef CALL
}

void launch_isums(int fmt, const uint8_t *W, int nrows, int ncols, const Q8Rows &x, int nsums_row, int32_t *out,
                  hipStream_t st) {
    int T;
    const int nitems = items_per_row(fmt, ncols);
    const int S = pick_S(nitems, &T);
    const uint32_t rb = row_bytes(fmt, ncols);
    const int G = 64 / S;
    const int waves = (nrows + G - 1) / G;
    dim3 grid((waves + 3) / 4);
#define CALL(S_) hipLaunchKernelGGL((k_isums<F, S_>), grid, dim3(256), 0, st, W, rb, nrows, x, nitems, T, nsums_row, out)
    TG_DISPATCH_F(fmt, TG_DISPATCH_S(S, CALL))
#undef CALL
}

static int g_grouped_min_rows = 4;

void set_grouped_min_rows(int rows) { g_grouped_min_rows = rows < 0 ? 0 : rows; }
int grouped_min_rows() { return g_grouped_min_rows; }

/* the MFMA phases address each weight matrix and q8 table with one 31-bit
 * buffer range, copy 16-byte aligned slabs, and hold two slabs of a gate/up
 * row group in 64 KiB of LDS */
static bool grouped_fits(const MoeArgs &a) {
    const uint64_t lim = 1ull << 31;
    const uint64_t gu = (uint64_t)a.I * row_bytes(TG_FMT_MXFP4, a.D);
    const uint64_t dn = (uint64_t)a.D * row_bytes(TG_FMT_MXFP4, a.I);
    const uint64_t xq = (uint64_t)a.k * a.xq.nb * 256, hq = (uint64_t)a.P * a.hq.nb * 256;
    return a.mx_aligned && gu < lim && dn < lim && xq < lim && hq < lim && grouped_lds_ok(a.D, a.I);
}

void launch_moe(const MoeArgs &a, const int *down_fmts_present, int n_down_fmts, hipStream_t st,
                const std::function<void(int)> *mark, bool quantize_x) {
    /* 1. quantize the k input rows */
    if (quantize_x) {
        launch_quantize(a.xin, a.D, a.k, a.D, a.xq, st);
        if (mark) (*mark)(1);
    }
    /* 2. phase A: MXFP4 experts with many pairs take the MFMA kernel, which
     * reads each weight block once for up to 64 pairs */
    const bool mx_grouped = g_grouped_min_rows > 0 && a.max_rows >= g_grouped_min_rows && grouped_fits(a);
    if (mx_grouped && a.gate_fmt == TG_FMT_MXFP4 && a.xp) {
        launch_mx_split(a.xq, a.k, a.D, a.xp, st);
        launch_moe_a_mx(a, st);
    } else {
        int T;
        const int nitems = items_per_row(a.gate_fmt, a.D);
        const int S = pick_S(nitems, &T);
        const int rpw = 64 / S;
        const int waves = (a.I + rpw - 1) / rpw;
        dim3 grid((waves + 3) / 4, a.P);
        const int TB = pick_TB(T);
#define CALL(S_, TB_) hipLaunchKernelGGL((k_moe_a<F, S_, TB_>), grid, dim3(256), 0, st, a, nitems, T, rpw)
        TG_DISPATCH_F(a.gate_fmt, TG_DISPATCH_ST(S, TB, CALL))
#undef CALL
    }
    if (mark) (*mark)(2);
    /* 3. quantize the hidden rows */
    launch_quantize(a.hidden, a.I, a.P, a.I, a.hq, st);
    if (mark) (*mark)(3);
    /* 4. phase B, once per down format present */
    for (int i = 0; i < n_down_fmts; i++) {
        const int fmt = down_fmts_present[i];
        if (mx_grouped && fmt == TG_FMT_MXFP4 && a.hp) {
            launch_mx_split(a.hq, a.P, a.I, a.hp, st);
            launch_moe_b_mx(a, st);
            continue;
        }
        int T;
        const int nitems = items_per_row(fmt, a.I);
        const int S = pick_S(nitems, &T);
        const int rpw = 64 / S;
        const int waves = (a.D + rpw - 1) / rpw;
        const uint32_t rb = row_bytes(fmt, a.I);
        dim3 grid((waves + 3) / 4, a.P);
        const int TB = pick_TB(T);
#define CALL(S_, TB_) hipLaunchKernelGGL((k_moe_b<F, S_, TB_>), grid, dim3(256), 0, st, a, fmt, rb, nitems, T, rpw)
        TG_DISPATCH_F(fmt, TG_DISPATCH_ST(S, TB, CALL))
#undef CALL
    }
    if (mark) (*mark)(4);
    /* 5. combine */
    const size_t n = (size_t)a.k * a.D;
    hipLaunchKernelGGL(k_moe_combine, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a);
    if (mark) (*mark)(5);
}

static int rms_waves(int n) { return std::min(RMS_WAVES, (n + 255) / 256); }

bool rms_norm_fits(int n) { return n > 0 && n <= RMS_WAVES * RMS_BPW * 256; }

void launch_rms_norm(const float *x, const float *w, float *out, int nrows, int n, float eps, hipStream_t st) {
    Q8Rows none = {};
    hipLaunchKernelGGL(k_rms_norm_q8, dim3(nrows), dim3(64 * rms_waves(n)), 0, st, x, w, out, n, eps, none);
}

void launch_rms_norm_q8(const float *x, const float *w, float *out, int nrows, int n, float eps, const Q8Rows &q,
                        hipStream_t st) {
    hipLaunchKernelGGL(k_rms_norm_q8, dim3(nrows), dim3(64 * rms_waves(n)), 0, st, x, w, out, n, eps, q);
}

void launch_synth_fill(int kind, uint64_t seed, void *dst, uint64_t nbytes, hipStream_t st) {
    hipLaunchKernelGGL(k_synth_fill, dim3(4096), dim3(256), 0, st, kind, seed, (uint8_t *)dst, nbytes);
}

void launch_copy(const void *src, void *dst, uint64_t nbytes, hipStream_t st) {
    hipLaunchKernelGGL(k_copy, dim3(256 * 16), dim3(256), 0, st, (const u32x4 *)src, (u32x4 *)dst, nbytes / 16);
}

}  // namespace tg
