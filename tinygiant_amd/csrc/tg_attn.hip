/*
 * tg_attn.hip -- decode attention for one row on the device: the part of
 * tg_attention_v2 (csrc/libtinygiant.c:939-983) between the Q/K/V
 * projections and the output projection (those are the library's q8 + GEMV
 * kernels).
 *
 *   k_attn_partial  split over the sequence: one workgroup per (KV head,
 *                   32 positions) stages those K and V rows and the GQA query
 *                   heads that share them in LDS, so each cache byte is read
 *                   once; per query head it writes the chunk's max score,
 *                   sum of exponentials and unnormalised V sum.  It also does
 *                   the heads' preparation: the optional QK RMS norm
 *                   (tg_rms_norm, :680-698) and RoPE at pos
 *                   (apply_rope_inplace, :702-719) of its query heads, and, in
 *                   the chunk that ends at kv_len, of the new K row, which it
 *                   stores with the new V row at kv_len of the cache
 *   k_attn_combine  one workgroup per query head merges the chunks with the
 *                   optional sink logit (head_task, :862-904);
 *                   k_attn_combine_q8 does the same for the heads of one
 *                   256-value block and quantizes the block for the output
 *                   projection
 *
 * The scores, exponentials and sums follow head_task's formulas (scale by
 * 1/sqrt(head_dim), max seeded with the sink, sum seeded with exp(sink -
 * max)); the chunked f32 grouping differs from its sequential sum, within
 * the f32 bar.
 */
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "tg_attn.h"
#include "tg_device.hpp"

namespace tg {

namespace {

constexpr int CHUNK = ATTN_CHUNK;       /* positions per workgroup */
constexpr int MAXHD = ATTN_MAX_HEAD_DIM;
constexpr int MAXR = ATTN_MAX_GQA;

}  // namespace

/* One head of head_dim values from src: the optional RMS norm (tg_rms_norm,
 * :680-698; weight nw, none when null) and RoPE at pos (apply_rope_inplace,
 * :702-719) into dst, by one wave; lane holds pairs (i, i + half) for
 * i = lane, lane + 64. */
__device__ inline void prep_head(const float *src, const float *nw, const float *__restrict__ rc,
                                 const float *__restrict__ rs, int head_dim, float eps, int lane, float *dst) {
    const int half = head_dim / 2;
    float x1[MAXHD / 128], x2[MAXHD / 128];
#pragma unroll
    for (int j = 0; j < MAXHD / 128; j++) {
        const int i = lane + 64 * j;
        x1[j] = i < half ? src[i] : 0.f;
        x2[j] = i < half ? src[half + i] : 0.f;
    }
    if (nw) {
        /* tg_rms_norm: scale = 1/sqrt(ss/dim + eps), out = x*scale*w */
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < MAXHD / 128; j++) ss += x1[j] * x1[j] + x2[j] * x2[j];
        ss = wave_sum(ss);
        const float scale = 1.f / sqrtf(ss / (float)head_dim + eps);
#pragma unroll
        for (int j = 0; j < MAXHD / 128; j++) {
            const int i = lane + 64 * j;
            if (i < half) {
                x1[j] = (x1[j] * scale) * nw[i];
                x2[j] = (x2[j] * scale) * nw[half + i];
            }
        }
    }
    /* RoPE: x1' = x1*c - x2*s, x2' = x2*c + x1*s */
#pragma unroll
    for (int j = 0; j < MAXHD / 128; j++) {
        const int i = lane + 64 * j;
        if (i < half) {
            const float c = rc[i], s = rs[i];
            const float p = x2[j] * s;
            dst[i] = x1[j] * c - p;
            dst[half + i] = fmaf(x1[j], s, x2[j] * c);
        }
    }
}

/* grid (chunks, n_kv): part[(h * nchunks + c) * (head_dim + 2)] =
 * {max, sum, o[head_dim]} for every query head h of KV head blockIdx.y.
 * Each workgroup prepares the query heads of its group from the projections
 * (qkv: q | k | v) in LDS; the chunk that ends at kv_len also prepares the
 * new K row and copies the new V row, stores both at kv_len of the cache
 * and uses them from LDS.  Every other row comes from the cache. */
__global__ __launch_bounds__(256) void k_attn_partial(const float *__restrict__ qkv, const float *__restrict__ q_norm_w,
                                                      const float *__restrict__ k_norm_w, const float *__restrict__ rc,
                                                      const float *__restrict__ rs, float *kv_k, float *kv_v,
                                                      float *part, int n_heads, int n_kv, int head_dim, int kv_len,
                                                      int kv_max, int start, int seq_len, float inv_sqrt, float eps) {
    __shared__ float ks[CHUNK][MAXHD + 1];
    __shared__ float vs[CHUNK][MAXHD];
    __shared__ float qs[MAXR][MAXHD];
    __shared__ float sc[MAXR][CHUNK];
    const int kh = blockIdx.y, c = blockIdx.x, nchunks = gridDim.x;
    const int ratio = n_heads / n_kv;
    const int t0 = start + c * CHUNK, np = min(CHUNK, seq_len - t0);
    const bool last = t0 + np - 1 == kv_len;   /* uniform: this chunk holds the new row */
    const int npc = last ? np - 1 : np;       /* rows read from the cache */
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int q_dim = n_heads * head_dim, kv_dim = n_kv * head_dim;
    const float *kb = kv_k + ((size_t)kh * kv_max + t0) * head_dim;
    const float *vb = kv_v + ((size_t)kh * kv_max + t0) * head_dim;
    /* K and V rows of the chunk (contiguous in the cache): every 16-byte load
     * of the thread issued before the first LDS store */
    constexpr int NV = CHUNK * MAXHD / 4 / 256;   /* float4 per thread and matrix */
    float4 kr[NV], vr[NV];
    const int n4 = npc * head_dim / 4;
#pragma unroll
    for (int r = 0; r < NV; r++) {
        const int i = tid + 256 * r;
        if (i < n4) {
            kr[r] = ((const float4 *)kb)[i];
            vr[r] = ((const float4 *)vb)[i];
        }
    }
    /* query heads (one wave each), then the new K/V row */
    for (int j = w; j < ratio + (last ? 1 : 0); j += 4) {
        if (j < ratio) {
            prep_head(qkv + (size_t)(kh * ratio + j) * head_dim, q_norm_w, rc, rs, head_dim, eps, lane, qs[j]);
        } else {
            prep_head(qkv + q_dim + (size_t)kh * head_dim, q_norm_w ? k_norm_w : nullptr, rc, rs, head_dim, eps,
                      lane, ks[np - 1]);
            const float *vsrc = qkv + q_dim + kv_dim + (size_t)kh * head_dim;
            float *kd = kv_k + ((size_t)kh * kv_max + kv_len) * head_dim;
            float *vd = kv_v + ((size_t)kh * kv_max + kv_len) * head_dim;
            __builtin_amdgcn_wave_barrier();
            for (int i = lane; i < head_dim; i += 64) {
                const float v = vsrc[i];
                vs[np - 1][i] = v;
                vd[i] = v;
                kd[i] = ks[np - 1][i];
            }
        }
    }
#pragma unroll
    for (int r = 0; r < NV; r++) {
        const int i = tid + 256 * r;
        if (i < n4) {
            const int p = (4 * i) / head_dim, d = 4 * i - p * head_dim;
            ks[p][d] = kr[r].x;
            ks[p][d + 1] = kr[r].y;
            ks[p][d + 2] = kr[r].z;
            ks[p][d + 3] = kr[r].w;
            *(float4 *)&vs[p][d] = vr[r];
        }
    }
    __syncthreads();
    /* scores of (head j, position p) */
    for (int i = tid; i < ratio * CHUNK; i += 256) {
        const int j = i / CHUNK, p = i - j * CHUNK;
        float s = -INFINITY;
        if (p < np) {
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
            for (int d = 0; d < head_dim; d += 4) {
                a0 = fmaf(qs[j][d], ks[p][d], a0);
                a1 = fmaf(qs[j][d + 1], ks[p][d + 1], a1);
                a2 = fmaf(qs[j][d + 2], ks[p][d + 2], a2);
                a3 = fmaf(qs[j][d + 3], ks[p][d + 3], a3);
            }
            s = ((a0 + a1) + (a2 + a3)) * inv_sqrt;
        }
        sc[j][p] = s;
    }
    __syncthreads();
    /* per head: max, exponentials, sum (one wave per head, lane = position) */
    __shared__ float mls[MAXR][2];
    for (int j = w; j < ratio; j += 4) {
        const float s = lane < CHUNK ? sc[j][lane] : -INFINITY;
        const float m = wave_max(s);
        const float e = lane < np ? expf(s - m) : 0.f;
        if (lane < CHUNK) sc[j][lane] = e;
        const float l = wave_sum(e);
        if (lane == 0) {
            mls[j][0] = m;
            mls[j][1] = l;
        }
    }
    __syncthreads();
    /* o[j][d] = sum_p e[j][p] * v[p][d] */
    for (int i = tid; i < ratio * head_dim; i += 256) {
        const int j = i / head_dim, d = i - j * head_dim;
        float o = 0.f;
        for (int p = 0; p < np; p++) o = fmaf(sc[j][p], vs[p][d], o);
        float *dst = part + ((size_t)(kh * ratio + j) * nchunks + c) * (head_dim + 2);
        dst[2 + d] = o;
        if (d == 0) {
            dst[0] = mls[j][0];
            dst[1] = mls[j][1];
        }
    }
}

/* max / sum over the 256 threads of a workgroup (4 waves) */
__device__ inline float block_max(float v, float *red) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float r = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    return r;
}
__device__ inline float block_sum(float v, float *red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float r = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return r;
}

/* one workgroup per query head: att[h] = (sum_c o_c exp(m_c - M)) / L with
 * M = max(sink, m_c), L = exp(sink - M) + sum_c l_c exp(m_c - M); the chunk
 * scales go to LDS, the V sums are split over 256 / head_dim thread groups */
__global__ __launch_bounds__(256) void k_attn_combine(const float *__restrict__ part, const float *__restrict__ sinks,
                                                      float *att, int n_heads, int head_dim, int nchunks) {
    __shared__ float scale[ATTN_MAX_CHUNKS];
    __shared__ float red[4];
    __shared__ float osum[256];
    const int h = blockIdx.x, tid = threadIdx.x;
    const size_t stride = (size_t)head_dim + 2;
    const float *ph = part + (size_t)h * nchunks * stride;
    float m = -INFINITY;
    for (int c = tid; c < nchunks; c += 256) m = fmaxf(m, ph[c * stride]);
    float M = block_max(m, red);
    if (sinks) M = fmaxf(M, sinks[h]);
    float l = 0.f;
    for (int c = tid; c < nchunks; c += 256) {
        const float sc = expf(ph[c * stride] - M);
        scale[c] = sc;
        l = fmaf(ph[c * stride + 1], sc, l);
    }
    float L = block_sum(l, red);   /* also orders the scale writes before their reads */
    if (sinks) L += expf(sinks[h] - M);
    const int groups = 256 / head_dim, g = tid / head_dim, d = tid - g * head_dim;
    float o = 0.f;
    if (g < groups) {
#pragma unroll 8
        for (int c = g; c < nchunks; c += groups) o = fmaf(ph[c * stride + 2 + d], scale[c], o);
    }
    osum[tid] = o;
    __syncthreads();
    if (tid < head_dim) {
        float r = osum[tid];
        for (int k = 1; k < groups; k++) r += osum[k * head_dim + tid];
        att[(size_t)h * head_dim + tid] = r * (1.f / L);
    }
}

/* k_attn_combine for the 256 / head_dim query heads of one 256-value q8
 * block per workgroup (heads in turn, the same arithmetic), then q8 of the
 * block (the arithmetic of k_quantize_q8) into aq. */
__global__ __launch_bounds__(256) void k_attn_combine_q8(const float *__restrict__ part,
                                                         const float *__restrict__ sinks, float *att, int n_heads,
                                                         int head_dim, int nchunks, Q8Rows aq) {
    __shared__ float scale[ATTN_MAX_CHUNKS];
    __shared__ float red[4];
    __shared__ float osum[256];
    __shared__ __attribute__((aligned(16))) float blk[256];
    const int tid = threadIdx.x, hpb = 256 / head_dim;
    const size_t stride = (size_t)head_dim + 2;
    for (int jh = 0; jh < hpb; jh++) {
        const int h = blockIdx.x * hpb + jh;
        const float *ph = part + (size_t)h * nchunks * stride;
        float m = -INFINITY;
        for (int c = tid; c < nchunks; c += 256) m = fmaxf(m, ph[c * stride]);
        float M = block_max(m, red);
        if (sinks) M = fmaxf(M, sinks[h]);
        float l = 0.f;
        for (int c = tid; c < nchunks; c += 256) {
            const float sc = expf(ph[c * stride] - M);
            scale[c] = sc;
            l = fmaf(ph[c * stride + 1], sc, l);
        }
        float L = block_sum(l, red);
        if (sinks) L += expf(sinks[h] - M);
        const int groups = 256 / head_dim, g = tid / head_dim, d = tid - g * head_dim;
        float o = 0.f;
        if (g < groups) {
#pragma unroll 8
            for (int c = g; c < nchunks; c += groups) o = fmaf(ph[c * stride + 2 + d], scale[c], o);
        }
        osum[tid] = o;
        __syncthreads();
        if (tid < head_dim) {
            float r = osum[tid];
            for (int k = 1; k < groups; k++) r += osum[k * head_dim + tid];
            const float v = r * (1.f / L);
            att[(size_t)h * head_dim + tid] = v;
            blk[jh * head_dim + tid] = v;
        }
        __syncthreads();
    }
    if (tid < 64) {
        const float4 v = reinterpret_cast<const float4 *>(blk)[tid];
        q8_block_store(v.x, v.y, v.z, v.w, tid, aq, 0, blockIdx.x);
    }
}

void launch_attention_core(const float *qkv, const float *q_norm_w, const float *k_norm_w, const float *sinks,
                           float *kv_k, float *kv_v, int kv_len, int kv_max, int window, const float *rope_cos_row,
                           const float *rope_sin_row, int n_heads, int n_kv, int head_dim, float eps, float *part,
                           float *att, const Q8Rows *aq, hipStream_t st) {
    const int seq_len = kv_len + 1;
    const int start = (window > 0 && seq_len > window) ? seq_len - window : 0;
    const int nchunks = (seq_len - start + CHUNK - 1) / CHUNK;
    hipLaunchKernelGGL(k_attn_partial, dim3(nchunks, n_kv), dim3(256), 0, st, qkv, q_norm_w, k_norm_w, rope_cos_row,
                       rope_sin_row, kv_k, kv_v, part, n_heads, n_kv, head_dim, kv_len, kv_max, start, seq_len,
                       1.f / sqrtf((float)head_dim), eps);
    if (aq) {
        hipLaunchKernelGGL(k_attn_combine_q8, dim3(n_heads * head_dim / 256), dim3(256), 0, st, part, sinks, att,
                           n_heads, head_dim, nchunks, *aq);
    } else {
        hipLaunchKernelGGL(k_attn_combine, dim3(n_heads), dim3(256), 0, st, part, sinks, att, n_heads, head_dim,
                           nchunks);
    }
}

bool attention_combine_q8_ok(int n_heads, int head_dim) {
    return 256 % head_dim == 0 && (n_heads * head_dim) % 256 == 0;
}

}  // namespace tg
