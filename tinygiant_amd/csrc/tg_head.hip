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
 *                   Each lane ends with one input row's sum (a DPP
 *                   reduce-scatter over the 16 lanes); each workgroup keeps
 *                   the best (logit, row) per input row, commits it with one
 *                   64-bit atomic max, and the last workgroup to finish
 *                   writes the argmax.
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

/* One step of the segment reduce-scatter below: the lanes of each pair
 * (given by the DPP pattern CTRL) split the first M slots, the lane with
 * `hi` set keeping the upper half, and add what the partner sends; once one
 * slot is left the step only adds. */
template <int CTRL, int M>
__device__ inline void rs_step(float *v, bool hi) {
    if constexpr (M >= 2) {
#pragma unroll
        for (int i = 0; i < M / 2; i++) {
            const float send = hi ? v[i] : v[i + M / 2];
            const float keep = hi ? v[i + M / 2] : v[i];
            v[i] = keep + dpp_f<CTRL>(0.f, send);
        }
    } else {
        v[0] += dpp_f<CTRL>(0.f, v[0]);
    }
}
/* Sums N slots (N a power of two <= 16) over the 16 lanes of each row of a
 * wave and leaves slot hb >> (4 - log2 N) in lane hb: a butterfly over the
 * lane pairs hb ^ 15, hb ^ 7, hb ^ 2, hb ^ 1 (the four masks are independent,
 * so each lane ends with all 16 lanes' share of its slot). */
template <int N>
__device__ inline float rscatter16(float *v, int hb) {
    rs_step<0x140, N>(v, (hb & 8) != 0);                    /* row_mirror */
    rs_step<0x141, (N >= 2 ? N / 2 : 1)>(v, (hb & 4) != 0);  /* row_half_mirror */
    rs_step<0x4E, (N >= 4 ? N / 4 : 1)>(v, (hb & 2) != 0);   /* quad_perm 2,3,0,1 */
    rs_step<0xB1, (N >= 8 ? N / 8 : 1)>(v, (hb & 1) != 0);   /* quad_perm 1,0,3,2 */
    return v[0];
}

constexpr int pow2_at_least(int k) { return k <= 1 ? 1 : k <= 2 ? 2 : k <= 4 ? 4 : k <= 8 ? 8 : 16; }
constexpr int log2_of(int n) { return n <= 1 ? 0 : n == 2 ? 1 : n == 4 ? 2 : n == 8 ? 3 : 4; }

/* Q6_K head, 2048 columns, k <= K input rows (q8 rows in x).  best[0..k)
 * receive the argmax keys and best[16] counts finished workgroups; both
 * start at zero (cleared by the kernel that quantizes x).  The last
 * workgroup to finish writes idx[j] / val[j]. */
template <int K>
__global__ __launch_bounds__(HT) void k_head_q6k(const uint8_t *__restrict__ W, int nrows, Q8Rows x, int k,
                                                 float *logits, unsigned long long *best, int32_t *idx, float *val) {
    constexpr int N = pow2_at_least(K);
    __shared__ __attribute__((aligned(16))) int8_t xq[K][HPR * XST];
    __shared__ __attribute__((aligned(16))) int32_t xs[K][NBH * 16];   /* -32 x the 16-value sums */
    __shared__ float xd[K][NBH];
    __shared__ unsigned long long wb_best[K][HW * RPW];
    __shared__ int last_wg;

    /* stage the k q8 rows: 128-value halves at XST strides */
    for (int t = threadIdx.x; t < k * NBH * 64; t += HT) {
        const int j = t / (NBH * 64), rem = t % (NBH * 64), b = rem >> 6, w = rem & 63;
        const uint32_t v = reinterpret_cast<const uint32_t *>(x.qs + ((size_t)j * NBH + b) * 256)[w];
        *reinterpret_cast<uint32_t *>(&xq[j][(2 * b + (w >> 5)) * XST + 4 * (w & 31)]) = v;
    }
    for (int t = threadIdx.x; t < k * NBH * 16; t += HT) xs[t / (NBH * 16)][t % (NBH * 16)] = -32 * x.s16[t];
    for (int t = threadIdx.x; t < k * NBH; t += HT) xd[t / NBH][t % NBH] = x.d[t];
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int hb = lane & (HPR - 1), b = hb >> 1, h = hb & 1, rsub = lane / HPR;
    /* after the reduce-scatter lane hb holds input row `slot`; with N < 16
     * several lanes hold the same one and the first of them owns it */
    const int slot = hb >> (4 - log2_of(N));
    const bool owner = (hb & (16 / N - 1)) == 0 && slot < k;
    const int gw = blockIdx.x * HW + (threadIdx.x >> 6), nw = gridDim.x * HW;
    const int nq = (nrows + RPW - 1) / RPW;
    Buf wb = make_buf(W, (uint32_t)((size_t)nrows * HRB));   /* rows past nrows read zeros */
    uint64_t mybest = 0;

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
        float vv[N];
#pragma unroll
        for (int j = 0; j < N; j++) vv[j] = 0.f;
#pragma unroll
        for (int j = 0; j < K; j++) {
            if (j < k) {
                const u32x4 *xp = reinterpret_cast<const u32x4 *>(&xq[j][hb * XST]);
                /* the 16-value sums start at -32 x the x sums: the -32 offset of
                 * the 6-bit codes */
                const u32x4 s0 = *reinterpret_cast<const u32x4 *>(&xs[j][b * 16 + 8 * h]);
                const u32x4 s1 = *reinterpret_cast<const u32x4 *>(&xs[j][b * 16 + 8 * h + 4]);
                int S[8] = {(int)s0.x, (int)s0.y, (int)s0.z, (int)s0.w, (int)s1.x, (int)s1.y, (int)s1.z, (int)s1.w};
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const u32x4 x0 = xp[2 * g], x1 = xp[2 * g + 1];
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) S[2 * g] = dot4(qc[g][jj], pick(x0, jj), S[2 * g]);
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) S[2 * g + 1] = dot4(qc[g][4 + jj], pick(x1, jj), S[2 * g + 1]);
                }
                int A = 0;
#pragma unroll
                for (int i = 0; i < 8; i++) A += __mul24(sc[i], S[i]);   /* |S| < 2^18 */
                vv[j] = dw * xd[j][b] * (float)A;
            }
        }
        const float v = rscatter16<N>(vv, hb);
        if (owner && row < (uint32_t)nrows) {
            if (logits) logits[(size_t)slot * nrows + row] = v;
            const uint64_t key = argmax_key(v, row);
            mybest = key > mybest ? key : mybest;
        }
        cur = nxt;
    }
    /* workgroup best per input row, then one atomic max each */
    if (owner && slot < K) wb_best[slot][(threadIdx.x >> 6) * RPW + rsub] = mybest;
    __syncthreads();
    if ((int)threadIdx.x < k) {
        uint64_t m = 0;
        for (int i = 0; i < HW * RPW; i++) m = wb_best[threadIdx.x][i] > m ? wb_best[threadIdx.x][i] : m;
        /* the returned value is stored (to a slot already read), so the max
         * has been performed before this thread reaches the barrier below */
        wb_best[threadIdx.x][0] = atomicMax(&best[threadIdx.x], (unsigned long long)m);
    }
    __syncthreads();
    if (threadIdx.x == 0) last_wg = atomicAdd(&best[16], 1ull) == (unsigned long long)(gridDim.x - 1);
    __syncthreads();
    if (last_wg == 1 && (int)threadIdx.x < k) {
        const uint64_t key = __hip_atomic_load(&best[threadIdx.x], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        idx[threadIdx.x] = (int32_t)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFu));
        if (val) val[threadIdx.x] = key_value(key);
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

__global__ void k_argmax_finish(const unsigned long long *best, int k, int32_t *idx, float *val) {
    const int j = threadIdx.x;
    if (j >= k) return;
    const uint64_t key = best[j];
    idx[j] = (int32_t)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFu));
    if (val) val[j] = key_value(key);
}

bool head_fast_ok(int fmt, int ncols, int k) { return fmt == TG_FMT_Q6K && ncols == NBH * 256 && k >= 1 && k <= 16; }

void launch_head_q6k(const uint8_t *W, int nrows, const Q8Rows &x, int k, float *logits, unsigned long long *best,
                     int32_t *idx, float *val, hipStream_t st) {
    int dev = 0, cus = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const int nq = (nrows + RPW - 1) / RPW;
    const int grid = std::max(1, std::min(cus * 4, (nq + HW - 1) / HW));
/* k is rounded up to an instantiated K; rows j >= k skip their dots */
#define TG_HEAD(KK) hipLaunchKernelGGL(k_head_q6k<KK>, dim3(grid), dim3(HT), 0, st, W, nrows, x, k, logits, best, idx, val)
    if (k <= 1) TG_HEAD(1);
    else if (k <= 2) TG_HEAD(2);
    else if (k <= 4) TG_HEAD(4);
    else if (k <= 5) TG_HEAD(5);
    else if (k <= 8) TG_HEAD(8);
    else if (k <= 9) TG_HEAD(9);
    else TG_HEAD(16);
#undef TG_HEAD
}

void launch_argmax_rows(const float *logits, int nrows, int k, unsigned long long *best, hipStream_t st) {
    hipLaunchKernelGGL(k_argmax_rows, dim3(k), dim3(256), 0, st, logits, nrows, best);
}

void launch_argmax_finish(const unsigned long long *best, int k, int32_t *idx, float *val, hipStream_t st) {
    hipLaunchKernelGGL(k_argmax_finish, dim3(1), dim3(64), 0, st, best, k, idx, val);
}

}  // namespace tg
