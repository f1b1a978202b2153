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
                                                     long xstride, Q8Rows out, unsigned long long *clear, int nclear) {
    const int lane = threadIdx.x & 63;
    if (blockIdx.x == 0 && (int)threadIdx.x < nclear) clear[threadIdx.x] = 0;
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
                                                                float *__restrict__ y, int n, float eps, Q8Rows q,
                                                                unsigned long long *clear, int nclear) {
    __shared__ float red[RMS_WAVES];
    if (blockIdx.x == 0 && (int)threadIdx.x < nclear) clear[threadIdx.x] = 0;
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

/* ---- expert-major phases for Q4_K / Q6_K experts ----
 * One workgroup column per active expert instead of per pair: each lane
 * loads its weight items once and dots them with the q8 row of every pair of
 * the expert, staged MOE_X_MAXP rows at a time in LDS.  Each pair's sums run
 * over the same items in the same order as k_moe_a / k_moe_b, so the
 * results are the same bits. */
constexpr int MOE_X_MAXP = 8;
static_assert(MOE_X_MAXP == EXP_ROWS, "the first chunk's rows come from the expert descriptor");

/* q8 rows rows[0..n) of q into LDS slots 0..n-1 by the whole workgroup */
__device__ inline void q8_rows_to_lds(const Q8Rows &q, const int *rows, int n, uint8_t *lds) {
    const int nb = q.nb, per = nb * 22;   /* 16-byte units of qs, s32 and s16 */
    for (int u = threadIdx.x; u < n * per; u += blockDim.x) {
        const int s = u / per, v = u % per;
        const size_t r = (size_t)rows[s];
        const u32x4 *src;
        uint32_t dst;
        if (v < nb * 16) {
            src = reinterpret_cast<const u32x4 *>(q.qs + r * nb * 256) + v;
            dst = (uint32_t)v * 16;
        } else if (v < nb * 18) {
            src = reinterpret_cast<const u32x4 *>(q.s32 + r * nb * 8) + (v - nb * 16);
            dst = nb * 256 + (uint32_t)(v - nb * 16) * 16;
        } else {
            src = reinterpret_cast<const u32x4 *>(q.s16 + r * nb * 16) + (v - nb * 18);
            dst = nb * 288 + (uint32_t)(v - nb * 18) * 16;
        }
        *reinterpret_cast<u32x4 *>(lds + (size_t)s * q8_lds_stride(nb) + dst) = *src;
    }
    for (int u = threadIdx.x; u < n * nb; u += blockDim.x) {
        const int s = u / nb, b = u % nb;
        reinterpret_cast<float *>(lds + (size_t)s * q8_lds_stride(nb) + nb * 352)[b] = q.d[(size_t)rows[s] * nb + b];
    }
}

/* q8 of f32 rows src[rows[s] * ld ..] (nb 256-value blocks each) into LDS
 * slots 0..n-1, block per wave, with the arithmetic of k_quantize_q8 (the
 * same bits).  With gw set, row s is also written to q8 row grows[s] of
 * gout. */
constexpr int Q8Q_BATCH = 8;   /* blocks per wave whose loads are in flight together */
__device__ inline void q8_quant_rows_lds(const float *__restrict__ src, int ld, const int *rows, int n, int nb,
                                         uint8_t *lds, bool gw, Q8Rows gout, const int *grows) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    for (int u0 = wave; u0 < n * nb; u0 += nw * Q8Q_BATCH) {
        u32x4 raw[Q8Q_BATCH];
#pragma unroll
        for (int i = 0; i < Q8Q_BATCH; i++) {
            const int u = u0 + i * nw;
            const bool uv = u < n * nb;
            const int s = uv ? u / nb : 0, b = uv ? u % nb : 0;
            /* a row's last block may be partial: zeros past its end, as k_quantize_q8 reads */
            const Buf xb = make_buf(src + (size_t)rows[s] * ld + (size_t)b * 256,
                                    uv ? (uint32_t)min(256, ld - b * 256) * 4u : 0u);
            raw[i] = ld16(xb, (uint32_t)lane * 16u);
        }
#pragma unroll
        for (int i = 0; i < Q8Q_BATCH; i++) {
            const int u = u0 + i * nw;
            if (u >= n * nb) continue;   /* uniform per wave */
            const int s = u / nb, b = u % nb;
            const float v0 = __uint_as_float(raw[i].x), v1 = __uint_as_float(raw[i].y);
            const float v2 = __uint_as_float(raw[i].z), v3 = __uint_as_float(raw[i].w);
            const Q8Quant q = q8_block_quant(v0, v1, v2, v3);
            uint8_t *slot = lds + (size_t)s * q8_lds_stride(nb);
            reinterpret_cast<uint32_t *>(slot + b * 256)[lane] = q.packed;
            if ((lane & 3) == 0) reinterpret_cast<int32_t *>(slot + nb * 288)[b * 16 + (lane >> 2)] = q.s16;
            if ((lane & 7) == 0) reinterpret_cast<int32_t *>(slot + nb * 256)[b * 8 + (lane >> 3)] = q.s32;
            if (lane == 0) reinterpret_cast<float *>(slot + nb * 352)[b] = q.sc;
            if (gw) q8_block_store(v0, v1, v2, v3, lane, gout, grows[s], b);
        }
    }
}

/* Phase A, expert-major: grid (x: wave groups over the I rows, y: active
 * expert a.mx_act[y]).  Each wave owns NP passes of 64/S rows, with all
 * T <= TB items of each row in registers before any pair is dotted.  QX:
 * the workgroup quantizes its pairs' input rows from a.xin itself (no q8
 * launch before it); otherwise it copies them from a.xq. */
template <class F, int S, int TB, int NP, bool QX>
__global__ __launch_bounds__(256) void k_moe_ax(MoeArgs a, int nitems, int T) {
    extern __shared__ __attribute__((aligned(16))) uint8_t xl[];
    __shared__ int srow[MOE_X_MAXP];
    constexpr int G = 64 / S;
    const ExpDesc &d = a.ed[blockIdx.y];
    const int e = d.e, p0 = d.p0, np = d.np;
    const int lane = threadIdx.x & 63;
    const int seg = lane / S, sl = lane % S;
    const int rw = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * NP * G + seg;
    const uint32_t rb = a.gate_rb;
    const size_t mbytes = (size_t)a.I * rb;
    const Buf gw = make_buf((const void *)d.gate, (uint32_t)mbytes);
    const Buf uw = make_buf((const void *)d.up, (uint32_t)mbytes);
    typename F::W wg[NP][TB], wu[NP][TB];
    float gb[NP], ub[NP];
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const int r = rw + i * G;
        const bool rv = r < a.I;
#pragma unroll
        for (int u = 0; u < TB; u++) {
            const int item = sl + u * S;
            const bool iv = rv && u < T && item < nitems;
            wg[i][u] = F::load_w(gw, iv ? (uint32_t)r * rb : ROW_OOB, iv ? item : 0);
            wu[i][u] = F::load_w(uw, iv ? (uint32_t)r * rb : ROW_OOB, iv ? item : 0);
        }
        gb[i] = rv && a.gbias ? ((const float *)a.gbias[e])[r] : 0.f;
        ub[i] = rv && a.ubias ? ((const float *)a.ubias[e])[r] : 0.f;
    }
    for (int c0 = 0; c0 < np; c0 += MOE_X_MAXP) {
        const int nc = min(MOE_X_MAXP, np - c0);
        __syncthreads();   /* the previous chunk's rows are no longer read */
        if ((int)threadIdx.x < nc) srow[threadIdx.x] = c0 == 0 ? d.row[threadIdx.x] : a.p_row[p0 + c0 + threadIdx.x];
        __syncthreads();
        if (QX)
            q8_quant_rows_lds(a.xin, a.D, srow, nc, a.xq.nb, xl, false, a.xq, srow);
        else
            q8_rows_to_lds(a.xq, srow, nc, xl);
        __syncthreads();
        for (int s = 0; s < nc; s++) {
            const Q8Lds xr = q8_lds_slot(xl, a.xq.nb, s);
#pragma unroll
            for (int i = 0; i < NP; i++) {
                const int r = rw + i * G;
                const bool rv = r < a.I;
                float ag = 0.f, au = 0.f;
#pragma unroll
                for (int u = 0; u < TB; u++) {
                    const int item = sl + u * S;
                    if (rv && u < T && item < nitems) {
                        const typename F::X x = F::load_x(xr, item);
                        ag += F::value(wg[i][u], x, item);
                        au += F::value(wu[i][u], x, item);
                    }
                }
                float vg = seg_sum<S>(ag);
                float vu = seg_sum<S>(au);
                if (rv && sl == 0) {
                    if (a.gbias) vg += gb[i];
                    if (a.ubias) vu += ub[i];
                    a.hidden[(size_t)(p0 + c0 + s) * a.I + r] = act_fn(a.act, vg, vu);
                }
            }
        }
    }
}

/* Phase B, expert-major: grid (x: wave groups over the D rows, y: active
 * expert), NP passes of 64/S rows per wave as in k_moe_ax.  Only experts
 * whose down format is `fmt` run.  QH: each workgroup quantizes its pairs'
 * hidden rows itself (column 0 also writes them to a.hq), so no q8 launch
 * runs between the phases; otherwise it copies them from a.hq.
 * CMB: the combine runs here too.  Partials are written through to memory;
 * after its writes have completed, each workgroup takes a ticket on its row
 * tile (a.ctr[blockIdx.x], system scope).  The workgroup with the last of
 * the a.n_act_a tickets has every expert's partials for the tile's rows and
 * adds them into a.out in expert order, as k_moe_combine does, then resets
 * the counter to zero for the next call.  Nothing waits. */
template <class F, int S, int TB, int NP, bool CMB, bool QH>
__global__ __launch_bounds__(256) void k_moe_bx(MoeArgs a, int fmt, uint32_t rb, int nitems, int T) {
    extern __shared__ __attribute__((aligned(16))) uint8_t xl[];
    __shared__ int srow[MOE_X_MAXP];
    constexpr int G = 64 / S;
    const ExpDesc &d = a.ed[blockIdx.y];
    if (d.down_fmt != fmt) return;
    const int e = d.e, p0 = d.p0, np = d.np;
    const int lane = threadIdx.x & 63;
    const int seg = lane / S, sl = lane % S;
    const int rw = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * NP * G + seg;
    const Buf dw = make_buf((const void *)d.down, (uint32_t)((size_t)a.D * rb));
    typename F::W wd[NP][TB];
    float db[NP];
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const int r = rw + i * G;
        const bool rv = r < a.D;
#pragma unroll
        for (int u = 0; u < TB; u++) {
            const int item = sl + u * S;
            const bool iv = rv && u < T && item < nitems;
            wd[i][u] = F::load_w(dw, iv ? (uint32_t)r * rb : ROW_OOB, iv ? item : 0);
        }
        db[i] = rv && a.dbias ? ((const float *)a.dbias[e])[r] : 0.f;
    }
    for (int c0 = 0; c0 < np; c0 += MOE_X_MAXP) {
        const int nc = min(MOE_X_MAXP, np - c0);
        __syncthreads();
        if ((int)threadIdx.x < nc) srow[threadIdx.x] = p0 + c0 + threadIdx.x;
        __syncthreads();
        if (QH)
            q8_quant_rows_lds(a.hidden, a.I, srow, nc, a.hq.nb, xl, blockIdx.x == 0, a.hq, srow);
        else
            q8_rows_to_lds(a.hq, srow, nc, xl);
        __syncthreads();
        for (int s = 0; s < nc; s++) {
            const Q8Lds xr = q8_lds_slot(xl, a.hq.nb, s);
            const int p = p0 + c0 + s;
#pragma unroll
            for (int i = 0; i < NP; i++) {
                const int r = rw + i * G;
                const bool rv = r < a.D;
                float acc = 0.f;
#pragma unroll
                for (int u = 0; u < TB; u++) {
                    const int item = sl + u * S;
                    if (rv && u < T && item < nitems) acc += F::value(wd[i][u], F::load_x(xr, item), item);
                }
                const float v = seg_sum<S>(acc);
                if (rv && sl == 0) {
                    const float o = a.p_w[p] * (v + (a.dbias ? db[i] : 0.f));
                    if (CMB)
                        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(o), make_buf(a.part, 0x7FFFFFFFu).r,
                                                              (int)(((uint32_t)p * (uint32_t)a.D + (uint32_t)r) * 4u),
                                                              0, 16 /* sc1 */);
                    else
                        a.part[(size_t)p * a.D + r] = o;
                }
            }
        }
    }
    if constexpr (CMB) {
        __shared__ unsigned ticket;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (threadIdx.x == 0)
            ticket = __hip_atomic_fetch_add(a.ctr + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __syncthreads();
        if (ticket != (unsigned)(a.n_act_a - 1)) return;
        const int tr = (blockDim.x >> 6) * NP * G, r0 = blockIdx.x * tr;
        const Buf pb = make_buf(a.part, 0x7FFFFFFFu);
        for (int i = threadIdx.x; i < a.k * tr; i += blockDim.x) {
            const int j = i / tr, c = r0 + i % tr;
            if (c >= a.D) continue;
            float o = a.out[(size_t)j * a.D + c];
            /* the row's partials in batches of 8 loads, added in expert order */
            for (int q0 = a.r_off[j]; q0 < a.r_off[j + 1]; q0 += 8) {
                const int nq = min(8, a.r_off[j + 1] - q0);
                float v[8];
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    const uint32_t pr = t < nq ? (uint32_t)a.r_pair[q0 + t] : 0u;
                    v[t] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                        pb.r, t < nq ? (int)((pr * (uint32_t)a.D + (uint32_t)c) * 4u) : (int)ROW_OOB, 0,
                        16 /* sc1 */));
                }
#pragma unroll
                for (int t = 0; t < 8; t++)
                    if (t < nq) o += v[t];
            }
            a.out[(size_t)j * a.D + c] = o;
        }
        if (threadIdx.x == 0) __hip_atomic_store(a.ctr + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

/* out[row][c] += part[p][c] for the pairs p of `row`, in expert order. */
__global__ __launch_bounds__(256) void k_moe_combine(MoeArgs a) {
    const size_t idx = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (idx >= (size_t)a.k * a.D) return;
    const int row = (int)(idx / a.D), c = (int)(idx % a.D);
    float o = a.out[idx];
    /* eight pairs at a time: their indices, then their partials, each group
     * of loads in flight together; the additions stay in expert order */
    const int q0 = a.r_off[row], q1 = a.r_off[row + 1];
    for (int qb = q0; qb < q1; qb += 8) {
        int pr[8];
#pragma unroll
        for (int i = 0; i < 8; i++) pr[i] = qb + i < q1 ? a.r_pair[qb + i] : 0;
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = qb + i < q1 ? a.part[(size_t)pr[i] * a.D + c] : 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (qb + i < q1) o += v[i];
    }
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

void launch_quantize(const float *x, int ncols, int nrows, long xstride, const Q8Rows &out, hipStream_t st,
                     unsigned long long *clear, int nclear) {
    const int waves = nrows * out.nb;
    if (waves <= 0) return;
    hipLaunchKernelGGL(k_quantize_q8, dim3((waves + 3) / 4), dim3(256), 0, st, x, ncols, nrows, xstride, out, clear,
                       clear ? nclear : 0);
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
/* Negative: the default, by shape.  Where both persistent rings run (the
 * Qwen3 expert shape) they beat the v_dot4 phases from ~20 pairs on the
 * busiest expert (128 experts, Zipf top-8: 22 pairs 66 against 74 us, 29
 * pairs 81 against 95 us, 10-15 pairs even); the grid forms of other shapes
 * from ~40.  17 keeps every batch of up to 16 rows (a verify batch) on the
 * v_dot4 phases, whose bits the persistent multi-row step shares. */
constexpr int QK_RING_MIN_ROWS = 17, QK_GRID_MIN_ROWS = 40;
static int g_qk_min_rows = -1;
void set_qk_min_rows(int rows) { g_qk_min_rows = rows < 0 ? -1 : rows; }
int qk_min_rows() { return g_qk_min_rows; }

static int g_expert_major = EM_DEFAULT;

void set_expert_major(int mode) { g_expert_major = mode & EM_ALL; }
int expert_major() { return g_expert_major; }

/* the expert-major phases hold all T items of a row in registers and read
 * Q4_K / Q6_K / MXFP4 q8 items from LDS */
/* the expert-major phases stage up to MOE_X_MAXP q8 rows of nb blocks in
 * dynamic LDS; wider rows than the device allows fall back to the per-pair
 * kernels */
static size_t device_max_lds() {
    static int max_lds = -1;
    if (max_lds < 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
            max_lds = 0;
    }
    return (size_t)max_lds;
}
static bool expert_major_ok(const MoeArgs &a, int fmt, int T, int nb) {
    const size_t lds = (size_t)std::min(a.max_rows, MOE_X_MAXP) * q8_lds_stride(nb);
    return (g_expert_major & EM_ON) && a.n_act_a > 0 && T <= 4 && lds <= device_max_lds() &&
           (fmt == TG_FMT_Q4K || fmt == TG_FMT_Q6K || fmt == TG_FMT_MXFP4);
}
/* Quantizing inside the phases repeats each row's q8 in every workgroup of
 * its expert (~100 of them), and the ticket combine ends the down phase
 * with a write-through and a read of every partial at memory latency: each
 * beats the launch it saves only while the experts hold few pairs
 * (measured on Qwen3-30B-A3B layers: 1 pair, 21.3 -> 17.5 us a layer; 5 to
 * 16 rows, up to 4% slower). */
constexpr int FUSE_MAX_ROWS = 2;
/* ... and the in-phase q8 only for rows of at most 8 blocks: for gpt-oss's
 * 12-block rows (2880 values, ~360 workgroups per expert) it measured 11%
 * slower than the q8 launch (36-layer graph step 1.60 against 1.40 ms) */
constexpr int FUSE_MAX_BLOCKS = 8;

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

/* The expert-major launches.  Each wave takes NP = 1 pass of 64/S rows:
 * two or four passes per wave measured slower at every pair count
 * (Qwen3-30B-A3B verify layers, k = 16: 67.6 -> 76.2 and 90.1 us). */
template <class F, int S, int TB>
static void launch_ax(const MoeArgs &a, int nitems, int T, bool qx, size_t lds, hipStream_t st) {
    const int waves = (a.I + (64 / S) - 1) / (64 / S);
    const dim3 g((waves + 3) / 4, a.n_act_a);
    if (qx)
        hipLaunchKernelGGL((k_moe_ax<F, S, TB, 1, true>), g, dim3(256), lds, st, a, nitems, T);
    else
        hipLaunchKernelGGL((k_moe_ax<F, S, TB, 1, false>), g, dim3(256), lds, st, a, nitems, T);
}
template <class F, int S, int TB>
static void launch_bx(const MoeArgs &a, int fmt, uint32_t rb, int nitems, int T, bool cmb, bool qh, size_t lds,
                      hipStream_t st) {
    const int waves = (a.D + (64 / S) - 1) / (64 / S);
    const dim3 g((waves + 3) / 4, a.n_act_a);
    if (cmb && qh)
        hipLaunchKernelGGL((k_moe_bx<F, S, TB, 1, true, true>), g, dim3(256), lds, st, a, fmt, rb, nitems, T);
    else if (cmb)
        hipLaunchKernelGGL((k_moe_bx<F, S, TB, 1, true, false>), g, dim3(256), lds, st, a, fmt, rb, nitems, T);
    else if (qh)
        hipLaunchKernelGGL((k_moe_bx<F, S, TB, 1, false, true>), g, dim3(256), lds, st, a, fmt, rb, nitems, T);
    else
        hipLaunchKernelGGL((k_moe_bx<F, S, TB, 1, false, false>), g, dim3(256), lds, st, a, fmt, rb, nitems, T);
}

void launch_moe(const MoeArgs &a, const int *down_fmts_present, int n_down_fmts, hipStream_t st,
                const std::function<void(int)> *mark, bool quantize_x) {
    /* Q4_K / Q6_K experts with many pairs: the int8 MFMA phases */
    const bool rings = a.rg_items && a.rb_items && !a.dbias;
    const int qk_min = g_qk_min_rows >= 0 ? g_qk_min_rows : rings ? QK_RING_MIN_ROWS : QK_GRID_MIN_ROWS;
    if (qk_min > 0 && a.max_rows >= qk_min && n_down_fmts == 1 && down_fmts_present[0] == TG_FMT_Q6K &&
        qk_grouped_fits(a)) {
        if (quantize_x) {
            launch_quantize(a.xin, a.D, a.k, a.D, a.xq, st);
            if (mark) (*mark)(1);
        }
        launch_moe_a_qk(a, st);
        if (mark) (*mark)(2);
        launch_quantize(a.hidden, a.I, a.P, a.I, a.hq, st);
        if (mark) (*mark)(3);
        launch_moe_b_qk(a, st);
        if (mark) (*mark)(4);
        const size_t n = (size_t)a.k * a.D;
        hipLaunchKernelGGL(k_moe_combine, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a);
        if (mark) (*mark)(5);
        return;
    }
    /* (an e8m0 scale of 255 keeps the layer on the v_dot4 phases, which
     * apply the reference's 2^127 exactly) */
    const bool mx_grouped = g_grouped_min_rows > 0 && a.max_rows >= g_grouped_min_rows && grouped_fits(a) && !a.mx_e255;
    const bool mx_a = mx_grouped && a.gate_fmt == TG_FMT_MXFP4 && a.xp;
    int Ta;
    pick_S(items_per_row(a.gate_fmt, a.D), &Ta);
    /* expert-major phase A quantizes device-resident input rows itself */
    const bool ax = !mx_a && expert_major_ok(a, a.gate_fmt, Ta, a.xq.nb);
    const bool few = a.max_rows <= FUSE_MAX_ROWS || (g_expert_major & EM_FUSE_ANY);
    const bool q8_fused = (g_expert_major & EM_FUSE_Q8) && few;
    const bool any = g_expert_major & EM_FUSE_ANY;
    const bool qx_fused = quantize_x && ax && !a.xin_remote && q8_fused && (a.xq.nb <= FUSE_MAX_BLOCKS || any);
    /* expert-major phase B (every down format present Q4_K, Q6_K or MXFP4,
     * with one item count per row) quantizes the hidden rows itself when the
     * experts hold few pairs and, given tile counters, also combines */
    int Tb = 0, Sb = 64;
    bool bx = n_down_fmts > 0;
    if (bx) Sb = pick_S(items_per_row(down_fmts_present[0], a.I), &Tb);
    for (int i = 0; i < n_down_fmts; i++) {
        const int f = down_fmts_present[i];
        /* one grid (and one set of row tiles) for every format present */
        bx = bx && expert_major_ok(a, f, Tb, a.hq.nb) && items_per_row(f, a.I) == items_per_row(down_fmts_present[0], a.I) &&
             !(mx_grouped && f == TG_FMT_MXFP4 && a.hp);
    }
    const int tiles_b = ((a.D + 64 / Sb - 1) / (64 / Sb) + 3) / 4;
    const bool qh_fused = bx && q8_fused && (a.hq.nb <= FUSE_MAX_BLOCKS || any);
    const bool cmb = bx && (g_expert_major & EM_TICKETS) && few && a.ctr && tiles_b <= a.ctr_n &&
                     (uint64_t)a.P * a.D * 4 < (1ull << 31);
    /* 1. quantize the k input rows */
    if (quantize_x && !qx_fused) {
        launch_quantize(a.xin, a.D, a.k, a.D, a.xq, st);
        if (mark) (*mark)(1);
    }
    /* 2. phase A: MXFP4 experts with many pairs take the MFMA kernel, which
     * reads each weight block once for up to 64 pairs */
    if (mx_a) {
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
        if (ax) {
            const size_t lds = (size_t)std::min(a.max_rows, MOE_X_MAXP) * q8_lds_stride(a.xq.nb);
#define CALL(S_, TB_) launch_ax<F, S_, TB_>(a, nitems, T, qx_fused, lds, st)
            if (a.gate_fmt == TG_FMT_Q4K) {
                typedef FQ4K F;
                TG_DISPATCH_ST(S, TB, CALL)
            } else if (a.gate_fmt == TG_FMT_Q6K) {
                typedef FQ6K F;
                TG_DISPATCH_ST(S, TB, CALL)
            } else {
                typedef FMXFP4 F;
                TG_DISPATCH_ST(S, TB, CALL)
            }
#undef CALL
        } else {
#define CALL(S_, TB_) hipLaunchKernelGGL((k_moe_a<F, S_, TB_>), grid, dim3(256), 0, st, a, nitems, T, rpw)
            TG_DISPATCH_F(a.gate_fmt, TG_DISPATCH_ST(S, TB, CALL))
#undef CALL
        }
    }
    if (mark) (*mark)(2);
    /* 3. quantize the hidden rows */
    if (!qh_fused) {
        launch_quantize(a.hidden, a.I, a.P, a.I, a.hq, st);
        if (mark) (*mark)(3);
    }
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
        if (bx) {
            const size_t lds = (size_t)std::min(a.max_rows, MOE_X_MAXP) * q8_lds_stride(a.hq.nb);
#define CALL(S_, TB_) launch_bx<F, S_, TB_>(a, fmt, rb, nitems, T, cmb, qh_fused, lds, st)
            if (fmt == TG_FMT_Q4K) {
                typedef FQ4K F;
                TG_DISPATCH_ST(S, TB, CALL)
            } else if (fmt == TG_FMT_Q6K) {
                typedef FQ6K F;
                TG_DISPATCH_ST(S, TB, CALL)
            } else {
                typedef FMXFP4 F;
                TG_DISPATCH_ST(S, TB, CALL)
            }
#undef CALL
            continue;
        }
#define CALL(S_, TB_) hipLaunchKernelGGL((k_moe_b<F, S_, TB_>), grid, dim3(256), 0, st, a, fmt, rb, nitems, T, rpw)
        TG_DISPATCH_F(fmt, TG_DISPATCH_ST(S, TB, CALL))
#undef CALL
    }
    if (mark) (*mark)(4);
    if (cmb) return;
    /* 5. combine */
    const size_t n = (size_t)a.k * a.D;
    hipLaunchKernelGGL(k_moe_combine, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a);
    if (mark) (*mark)(5);
}

static int rms_waves(int n) { return std::min(RMS_WAVES, (n + 255) / 256); }

bool rms_norm_fits(int n) { return n > 0 && n <= RMS_WAVES * RMS_BPW * 256; }

void launch_rms_norm(const float *x, const float *w, float *out, int nrows, int n, float eps, hipStream_t st) {
    Q8Rows none = {};
    hipLaunchKernelGGL(k_rms_norm_q8, dim3(nrows), dim3(64 * rms_waves(n)), 0, st, x, w, out, n, eps, none,
                       (unsigned long long *)nullptr, 0);
}

void launch_rms_norm_q8(const float *x, const float *w, float *out, int nrows, int n, float eps, const Q8Rows &q,
                        hipStream_t st, unsigned long long *clear, int nclear) {
    hipLaunchKernelGGL(k_rms_norm_q8, dim3(nrows), dim3(64 * rms_waves(n)), 0, st, x, w, out, n, eps, q, clear,
                       clear ? nclear : 0);
}

void launch_synth_fill(int kind, uint64_t seed, void *dst, uint64_t nbytes, hipStream_t st) {
    hipLaunchKernelGGL(k_synth_fill, dim3(4096), dim3(256), 0, st, kind, seed, (uint8_t *)dst, nbytes);
}

void launch_copy(const void *src, void *dst, uint64_t nbytes, hipStream_t st) {
    hipLaunchKernelGGL(k_copy, dim3(256 * 16), dim3(256), 0, st, (const u32x4 *)src, (u32x4 *)dst, nbytes / 16);
}

}  // namespace tg
