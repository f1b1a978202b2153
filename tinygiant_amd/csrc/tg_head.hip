/*
 * tg_head.hip -- output head over a batch of rows with the argmax fused in.
 *
 * The reference runs, per row r of a verify batch, tg_rms_norm then
 * tg_matmul over the vocab x D output head (tinygiant/engine.py:347-354;
 * tg_matmul is csrc/libtinygiant.c:908-931 with dot_q6k_q8 :384-443) and
 * takes numpy.argmax of each row's logits (tinygiant/specdec.py:77,90,
 * engine.py:187).  Here the head is read once for all k rows:
 *
 *   k_head_q6k<K>   Q6_K head with 2048 columns: every lane owns one 128-value
 *                   half-block of one vocab row, decodes its 6-bit codes once
 *                   and dots them with the k q8 rows staged in LDS; the 16
 *                   lanes of a row are summed by DPP; the next row group's
 *                   weights are loaded while the current one is computed.
 *                   Each workgroup keeps the best (logit, row) per input row
 *                   and commits it with one 64-bit atomic max.
 *   k_argmax_rows   argmax of materialized logits (any format, via k_gemv).
 *
 * Argmax keys pack an order-preserving image of the f32 logit above the
 * complement of the row index, so the maximum key is the largest logit and,
 * among equal logits, the first row -- numpy.argmax's tie rule.
 */
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "tg_common.h"
#include "tg_device.hpp"
#include "tg_head.h"

namespace tg {

namespace {

constexpr int NBH = 8;          /* 256-blocks per head row (2048 columns) */
constexpr int HPR = 2 * NBH;    /* half-blocks (lanes) per row */
constexpr int RPW = 64 / HPR;   /* rows per wave */
constexpr int HRB = NBH * 210;  /* Q6_K head row bytes */
constexpr int XST = 144;        /* LDS stride of a staged 128-value half (bank spread) */
constexpr int HT = 256;         /* threads per head workgroup */
constexpr int HW = HT / 64;

__device__ inline uint64_t argmax_key(float v, uint32_t row) {
    uint32_t u = v == 0.f ? 0u : __float_as_uint(v);   /* -0 ties with +0, as in numpy */
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint64_t)(0xFFFFFFFFu - row);
}
__device__ inline float key_value(uint64_t key) {
    uint32_t u = (uint32_t)(key >> 32);
    u = (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u;
    return __uint_as_float(u);
}

/* One lane's Q6_K half-block (64 B of ql, 32 B of qh, 8 sub-scales, d). */
struct HHalf {
    u32x4 la0, la1, lb0, lb1, h0, h1;
    u32x2 sc;
    uint32_t d;
};
__device__ inline HHalf load_hhalf(Buf b, uint32_t blk, int h) {
    HHalf r;
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

__device__ inline uint32_t pick(const u32x4 &v, int c) { return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w; }

}  // namespace

/* Q6_K head, 2048 columns, k <= K input rows (q8 rows in x). */
template <int K>
__global__ __launch_bounds__(HT) void k_head_q6k(const uint8_t *__restrict__ W, int nrows, Q8Rows x, int k,
                                                 float *logits, unsigned long long *best) {
    __shared__ __attribute__((aligned(16))) int8_t xq[K][HPR * XST];
    __shared__ __attribute__((aligned(16))) int32_t xs[K][NBH * 16];
    __shared__ float xd[K][NBH];
    __shared__ unsigned long long wb_best[K][HW * RPW];

    /* stage the k q8 rows: 128-value halves at XST strides */
    for (int t = threadIdx.x; t < k * NBH * 64; t += HT) {
        const int j = t / (NBH * 64), rem = t % (NBH * 64), b = rem >> 6, w = rem & 63;
        const uint32_t v = reinterpret_cast<const uint32_t *>(x.qs + ((size_t)j * NBH + b) * 256)[w];
        *reinterpret_cast<uint32_t *>(&xq[j][(2 * b + (w >> 5)) * XST + 4 * (w & 31)]) = v;
    }
    for (int t = threadIdx.x; t < k * NBH * 16; t += HT) xs[t / (NBH * 16)][t % (NBH * 16)] = x.s16[t];
    for (int t = threadIdx.x; t < k * NBH; t += HT) xd[t / NBH][t % NBH] = x.d[t];
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int hb = lane & (HPR - 1), b = hb >> 1, h = hb & 1, rsub = lane / HPR;
    const int gw = blockIdx.x * HW + (threadIdx.x >> 6), nw = gridDim.x * HW;
    const int nq = (nrows + RPW - 1) / RPW;
    Buf wb = make_buf(W, (uint32_t)((size_t)nrows * HRB));   /* rows past nrows read zeros */
    uint64_t mybest[K];
#pragma unroll
    for (int j = 0; j < K; j++) mybest[j] = 0;

    HHalf cur = load_hhalf(wb, (uint32_t)(RPW * gw + rsub) * HRB + (uint32_t)b * 210u, h);
    for (int q = gw; q < nq; q += nw) {
        /* the next row group loads while this one is computed */
        HHalf nxt = load_hhalf(wb, (uint32_t)(RPW * (q + nw) + rsub) * HRB + (uint32_t)b * 210u, h);
        const uint32_t row = (uint32_t)(RPW * q + rsub);
        /* 6-bit codes of the half (q = ql nibble | qh pair << 4), decoded once */
        const uint32_t m4 = 0x0F0F0F0Fu, m2 = 0x30303030u;
        uint32_t qc[4][8];
#pragma unroll
        for (int jj = 0; jj < 8; jj++) {
            const int c = jj & 3;
            const uint32_t la = pick(jj < 4 ? cur.la0 : cur.la1, c), lb = pick(jj < 4 ? cur.lb0 : cur.lb1, c);
            const uint32_t hh = pick(jj < 4 ? cur.h0 : cur.h1, c);
            qc[0][jj] = (la & m4) | ((hh << 4) & m2);
            qc[1][jj] = (lb & m4) | ((hh << 2) & m2);
            qc[2][jj] = ((la >> 4) & m4) | (hh & m2);
            qc[3][jj] = ((lb >> 4) & m4) | ((hh >> 2) & m2);
        }
        int sc[8];
#pragma unroll
        for (int i = 0; i < 8; i++) sc[i] = (int)(int8_t)((i < 4 ? cur.sc.x : cur.sc.y) >> (8 * (i & 3)));
        const float dw = ref_f16(cur.d >> 16);
#pragma unroll
        for (int j = 0; j < K; j++) {
            float v = 0.f;
            if (j < k) {
                const u32x4 *xp = reinterpret_cast<const u32x4 *>(&xq[j][hb * XST]);
                int S[8];
#pragma unroll
                for (int i = 0; i < 8; i++) S[i] = 0;
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const u32x4 x0 = xp[2 * g], x1 = xp[2 * g + 1];
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) S[2 * g] = dot4(qc[g][jj], pick(x0, jj), S[2 * g]);
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) S[2 * g + 1] = dot4(qc[g][4 + jj], pick(x1, jj), S[2 * g + 1]);
                }
                const int32_t *s16 = &xs[j][b * 16 + 8 * h];
                int A = 0;
#pragma unroll
                for (int i = 0; i < 8; i++) A += __mul24(sc[i], S[i] - 32 * s16[i]);   /* |S - 32 s| < 2^18 */
                v = dw * xd[j][b] * (float)A;
            }
            v = seg_sum_last<HPR>(v);
            if (j < k && hb == HPR - 1 && row < (uint32_t)nrows) {
                if (logits) logits[(size_t)j * nrows + row] = v;
                const uint64_t key = argmax_key(v, row);
                mybest[j] = key > mybest[j] ? key : mybest[j];
            }
        }
        cur = nxt;
    }
    /* workgroup best per input row, then one atomic max each */
    if (hb == HPR - 1) {
#pragma unroll
        for (int j = 0; j < K; j++) wb_best[j][(threadIdx.x >> 6) * RPW + rsub] = mybest[j];
    }
    __syncthreads();
    if ((int)threadIdx.x < k) {
        uint64_t m = 0;
        for (int i = 0; i < HW * RPW; i++) m = wb_best[threadIdx.x][i] > m ? wb_best[threadIdx.x][i] : m;
        atomicMax(&best[threadIdx.x], (unsigned long long)m);
    }
}

/* argmax of logits [k][nrows] (one workgroup per input row) */
__global__ __launch_bounds__(256) void k_argmax_rows(const float *__restrict__ logits, int nrows,
                                                     unsigned long long *best) {
    __shared__ unsigned long long red[256];
    const int j = blockIdx.x;
    uint64_t m = 0;
    for (int r = threadIdx.x; r < nrows; r += 256) {
        const uint64_t key = argmax_key(logits[(size_t)j * nrows + r], (uint32_t)r);
        m = key > m ? key : m;
    }
    red[threadIdx.x] = m;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s && red[threadIdx.x + s] > red[threadIdx.x]) red[threadIdx.x] = red[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) best[j] = red[0];
}

__global__ void k_argmax_init(unsigned long long *best, int k) {
    if ((int)threadIdx.x < k) best[threadIdx.x] = 0;
}

__global__ void k_argmax_finish(const unsigned long long *best, int k, int32_t *idx, float *val) {
    const int j = threadIdx.x;
    if (j >= k) return;
    const uint64_t key = best[j];
    idx[j] = (int32_t)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFu));
    if (val) val[j] = key_value(key);
}

bool head_fast_ok(int fmt, int ncols, int k) { return fmt == TG_FMT_Q6K && ncols == NBH * 256 && k >= 1 && k <= 16; }

void launch_head_q6k(const uint8_t *W, int nrows, const Q8Rows &x, int k, float *logits, unsigned long long *best,
                     hipStream_t st) {
    int dev = 0, cus = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const int nq = (nrows + RPW - 1) / RPW;
    const int grid = std::max(1, std::min(cus * 4, (nq + HW - 1) / HW));
    hipLaunchKernelGGL(k_argmax_init, dim3(1), dim3(64), 0, st, best, k);
    if (k <= 1)
        hipLaunchKernelGGL(k_head_q6k<1>, dim3(grid), dim3(HT), 0, st, W, nrows, x, k, logits, best);
    else if (k <= 2)
        hipLaunchKernelGGL(k_head_q6k<2>, dim3(grid), dim3(HT), 0, st, W, nrows, x, k, logits, best);
    else if (k <= 4)
        hipLaunchKernelGGL(k_head_q6k<4>, dim3(grid), dim3(HT), 0, st, W, nrows, x, k, logits, best);
    else if (k <= 8)
        hipLaunchKernelGGL(k_head_q6k<8>, dim3(grid), dim3(HT), 0, st, W, nrows, x, k, logits, best);
    else
        hipLaunchKernelGGL(k_head_q6k<16>, dim3(grid), dim3(HT), 0, st, W, nrows, x, k, logits, best);
}

void launch_argmax_rows(const float *logits, int nrows, int k, unsigned long long *best, hipStream_t st) {
    hipLaunchKernelGGL(k_argmax_rows, dim3(k), dim3(256), 0, st, logits, nrows, best);
}

void launch_argmax_finish(const unsigned long long *best, int k, int32_t *idx, float *val, hipStream_t st) {
    hipLaunchKernelGGL(k_argmax_finish, dim3(1), dim3(64), 0, st, best, k, idx, val);
}

}  // namespace tg
