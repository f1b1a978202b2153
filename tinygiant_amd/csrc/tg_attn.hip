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
 *                   stores with the new V row at kv_len of the cache.
 *                   For short spans (attention_fuse_ok) the same kernel also
 *                   combines: the last workgroup of each KV head, by a
 *                   ticket counter, merges its query heads (combine_group)
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
#include "tg_xchg.hpp"

namespace tg {

namespace {

constexpr int CHUNK = ATTN_CHUNK;       /* positions per workgroup */
constexpr int MAXHD = ATTN_MAX_HEAD_DIM;
constexpr int MAXR = ATTN_MAX_GQA;

}  // namespace

/* One head of head_dim (<= 128) values: the optional RMS norm (tg_rms_norm,
 * :680-698) and RoPE at pos (apply_rope_inplace, :702-719), by one wave;
 * lane i holds the pair (i, i + head_dim / 2).  head_in loads a lane's
 * inputs (so the loads can be issued early), head_out computes and stores. */
struct HeadIn {
    float x1, x2, w1, w2, c, s;
};
__device__ inline HeadIn head_in(const float *src, const float *nw, const float *__restrict__ rc,
                                 const float *__restrict__ rs, int head_dim, int lane) {
    const int half = head_dim / 2;
    const bool on = lane < half;
    HeadIn r;
    r.x1 = on ? src[lane] : 0.f;
    r.x2 = on ? src[half + lane] : 0.f;
    r.w1 = on && nw ? nw[lane] : 0.f;
    r.w2 = on && nw ? nw[half + lane] : 0.f;
    r.c = on ? rc[lane] : 0.f;
    r.s = on ? rs[lane] : 0.f;
    return r;
}
__device__ inline void head_out(const HeadIn &in, bool norm, int head_dim, float eps, int lane, float *dst) {
    const int half = head_dim / 2;
    float x1 = in.x1, x2 = in.x2;
    if (norm) {
        /* tg_rms_norm: scale = 1/sqrt(ss/dim + eps), out = x*scale*w */
        float ss = 0.f;
        ss += x1 * x1 + x2 * x2;
        ss = wave_sum(ss);
        const float scale = 1.f / sqrtf(ss / (float)head_dim + eps);
        if (lane < half) {
            x1 = (x1 * scale) * in.w1;
            x2 = (x2 * scale) * in.w2;
        }
    }
    /* RoPE: x1' = x1*c - x2*s, x2' = x2*c + x1*s */
    if (lane < half) {
        const float p = x2 * in.s;
        dst[lane] = x1 * in.c - p;
        dst[half + lane] = fmaf(x1, in.s, x2 * in.c);
    }
}

/* The combine (head_task's merge of the chunks with the optional sink,
 * :862-904) of the `ratio` query heads of KV head kh, by one workgroup,
 * from partials written through to memory (read with sc1, so no stale line
 * of another XCD's L2 is seen), then q8 of the group's 256-value blocks:
 *   lane c of 32-lane half j: chunk c of head j -> M_j, exp(m_c - M_j), L_j
 *   thread t: head t / (head_dim / 4), values 4 (t % (head_dim / 4)) .. + 3,
 *             so wave w holds values 4 lane .. 4 lane + 3 of block w.
 * Needs nchunks <= ATTN_FUSE_MAX_CHUNKS, ratio <= 8 and ratio * head_dim a
 * multiple of 256 (attention_fuse_ok). */
__device__ inline void combine_group(const Buf pb, const AttnFuse &fz, int kh, int ratio, int head_dim,
                                     int nchunks) {
    __shared__ float scl[ATTN_MAX_GQA][ATTN_FUSE_MAX_CHUNKS];
    __shared__ float linv[ATTN_MAX_GQA];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t stride = (uint32_t)head_dim + 2u;
    {
        const int j = tid >> 5, c = tid & 31;
        const bool hv = j < ratio, on = hv && c < nchunks;
        const int h = kh * ratio + (hv ? j : 0);
        const uint32_t off = ((uint32_t)h * (uint32_t)nchunks + (uint32_t)(on ? c : 0)) * stride * 4u;
        float m = -INFINITY, l = 0.f;
        if (on) {
            const u32x2 ml = __builtin_amdgcn_raw_buffer_load_b64(pb.r, (int)off, 0, CPOL_SC1);
            m = __uint_as_float(ml.x);
            l = __uint_as_float(ml.y);
        }
        float M = m;
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
        if (fz.sinks && hv) M = fmaxf(M, fz.sinks[h]);
        const float e = on ? expf(m - M) : 0.f;
        float L = l * e;
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) L += __shfl_xor(L, o, 64);
        if (fz.sinks && hv) L += expf(fz.sinks[h] - M);
        if (hv) {
            scl[j][c] = e;
            if (c == 0) linv[j] = 1.f / L;
        }
    }
    __syncthreads();
    const int tph = head_dim / 4;
    const int j = tid / tph, d = 4 * (tid - j * tph);
    float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
    if (j < ratio) {
        const int h = kh * ratio + j;
#pragma unroll 8
        for (int c = 0; c < nchunks; c++) {
            const uint32_t off = (((uint32_t)h * (uint32_t)nchunks + (uint32_t)c) * stride + 2u + (uint32_t)d) * 4u;
            const u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(pb.r, (int)off, 0, CPOL_SC1);
            const u32x2 b = __builtin_amdgcn_raw_buffer_load_b64(pb.r, (int)(off + 8u), 0, CPOL_SC1);
            const float s = scl[j][c];
            o0 = fmaf(__uint_as_float(a.x), s, o0);
            o1 = fmaf(__uint_as_float(a.y), s, o1);
            o2 = fmaf(__uint_as_float(b.x), s, o2);
            o3 = fmaf(__uint_as_float(b.y), s, o3);
        }
        const float li = linv[j];
        o0 *= li;
        o1 *= li;
        o2 *= li;
        o3 *= li;
        float *dst = fz.att + (size_t)h * head_dim + d;
        dst[0] = o0;
        dst[1] = o1;
        dst[2] = o2;
        dst[3] = o3;
    }
    const int nblk = ratio * head_dim / 256;
    if (wave < nblk) q8_block_store(o0, o1, o2, o3, lane, fz.aq, 0, kh * nblk + wave);
}

/* grid (chunks, n_kv): part[(h * nchunks + c) * (head_dim + 2)] =
 * {max, sum, o[head_dim]} for every query head h of KV head blockIdx.y.
 * Each workgroup prepares the query heads of its group from the projections
 * (qkv: q | k | v) in LDS; the chunk that ends at kv_len also prepares the
 * new K row and copies the new V row, stores both at kv_len of the cache
 * and uses them from LDS.  Every other row comes from the cache. */
template <bool FUSE>
__global__ __launch_bounds__(256) void k_attn_partial(const float *__restrict__ qkv, const float *__restrict__ q_norm_w,
                                                      const float *__restrict__ k_norm_w, const float *__restrict__ rc,
                                                      const float *__restrict__ rs, float *kv_k, float *kv_v,
                                                      float *part, int n_heads, int n_kv, int head_dim, int kv_len,
                                                      int kv_max, int start, int seq_len, float inv_sqrt, float eps,
                                                      AttnFuse fz) {
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
    /* the inputs of this wave's heads first (query heads w, w + 4, ..., then
     * the new K row as head `ratio`, with the new V row), so their
     * preparation below waits only for them and not for the chunk */
    const bool norm = q_norm_w != nullptr;
    HeadIn hin[3];
    float vnew[2] = {0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 3; k++) {
        const int j = w + 4 * k;
        if (j < ratio) {
            hin[k] = head_in(qkv + (size_t)(kh * ratio + j) * head_dim, q_norm_w, rc, rs, head_dim, lane);
        } else if (j == ratio && last) {
            hin[k] = head_in(qkv + q_dim + (size_t)kh * head_dim, norm ? k_norm_w : nullptr, rc, rs, head_dim,
                             lane);
            const float *vsrc = qkv + q_dim + kv_dim + (size_t)kh * head_dim;
#pragma unroll
            for (int u = 0; u < 2; u++)
                if (lane + 64 * u < head_dim) vnew[u] = vsrc[lane + 64 * u];
        }
    }
    /* K and V rows of the chunk (contiguous in the cache): every 16-byte load
     * of the thread issued before the first LDS store; past the rows read
     * from the cache the buffers return zeros */
    constexpr int NV = CHUNK * MAXHD / 4 / 256;   /* float4 per thread and matrix */
    const int n4 = npc * head_dim / 4;
    const Buf kbb = make_buf(kb, (uint32_t)n4 * 16u), vbb = make_buf(vb, (uint32_t)n4 * 16u);
    u32x4 kr[NV], vr[NV];
#pragma unroll
    for (int r = 0; r < NV; r++) {
        kr[r] = ld16(kbb, (uint32_t)(tid + 256 * r) * 16u);
        vr[r] = ld16(vbb, (uint32_t)(tid + 256 * r) * 16u);
    }
    /* query heads, then the new K/V row */
#pragma unroll
    for (int k = 0; k < 3; k++) {
        const int j = w + 4 * k;
        if (j < ratio) {
            head_out(hin[k], norm, head_dim, eps, lane, qs[j]);
        } else if (j == ratio && last) {
            head_out(hin[k], norm, head_dim, eps, lane, ks[np - 1]);
            float *kd = kv_k + ((size_t)kh * kv_max + kv_len) * head_dim;
            float *vd = kv_v + ((size_t)kh * kv_max + kv_len) * head_dim;
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int i = lane + 64 * u;
                if (i < head_dim) {
                    vs[np - 1][i] = vnew[u];
                    vd[i] = vnew[u];
                    kd[i] = ks[np - 1][i];
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < NV; r++) {
        const int i = tid + 256 * r;
        if (i < n4) {
            const int p = (4 * i) / head_dim, d = 4 * i - p * head_dim;
            ks[p][d] = __uint_as_float(kr[r].x);
            ks[p][d + 1] = __uint_as_float(kr[r].y);
            ks[p][d + 2] = __uint_as_float(kr[r].z);
            ks[p][d + 3] = __uint_as_float(kr[r].w);
            *(u32x4 *)&vs[p][d] = vr[r];
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
    const Buf pb = make_buf(part, (uint32_t)((size_t)n_heads * nchunks * (head_dim + 2) * 4));
    for (int i = tid; i < ratio * head_dim; i += 256) {
        const int j = i / head_dim, d = i - j * head_dim;
        float o = 0.f;
        for (int p = 0; p < np; p++) o = fmaf(sc[j][p], vs[p][d], o);
        const size_t rec = ((size_t)(kh * ratio + j) * nchunks + c) * (head_dim + 2);
        if (FUSE) {
            /* written through to memory: the combining workgroup may sit on
             * another XCD */
            const uint32_t off = (uint32_t)rec * 4u;
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(o), pb.r, (int)(off + 4u * (2 + d)), 0, CPOL_SC1);
            if (d == 0) {
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(mls[j][0]), pb.r, (int)off, 0, CPOL_SC1);
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(mls[j][1]), pb.r, (int)(off + 4u), 0, CPOL_SC1);
            }
        } else {
            float *dst = part + rec;
            dst[2 + d] = o;
            if (d == 0) {
                dst[0] = mls[j][0];
                dst[1] = mls[j][1];
            }
        }
    }
    if constexpr (FUSE) {
        /* every write of this workgroup has completed before it takes a
         * ticket; the workgroup with the last ticket of its KV head sees all
         * chunks' partials and combines the head group (no waiting anywhere) */
        __shared__ unsigned ticket;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        /* system scope: performed at memory (sc1), not in one XCD's L2 */
        if (tid == 0) ticket = __hip_atomic_fetch_add(fz.ctr + kh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __syncthreads();
        if (ticket != (unsigned)(nchunks - 1)) return;
        combine_group(pb, fz, kh, ratio, head_dim, nchunks);
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
 * block per workgroup of 512 threads, then q8 of the block (the arithmetic
 * of k_quantize_q8) into aq.  Wave g takes the chunks c = g (mod 8); lane p
 * takes values 4p .. 4p + 3 of the block (head p / (head_dim / 4)), so the
 * chunk loads of a thread are independent and go out together.  The eight
 * wave partials are added in wave order. */
constexpr int CQ_WAVES = 8;
__global__ __launch_bounds__(CQ_WAVES * 64) void k_attn_combine_q8(const float *__restrict__ part,
                                                                   const float *__restrict__ sinks, float *att,
                                                                   int n_heads, int head_dim, int nchunks,
                                                                   Q8Rows aq) {
    __shared__ float scale[4 * ATTN_MAX_CHUNKS];   /* [head][chunk]: hpb <= 4 (head_dim >= 64) */
    __shared__ float redm[CQ_WAVES][4], redl[CQ_WAVES][4];
    __shared__ float hm[4], hl[4];
    __shared__ __attribute__((aligned(16))) float osum[CQ_WAVES][256];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int hpb = 256 / head_dim, h0 = blockIdx.x * hpb;
    const size_t stride = (size_t)head_dim + 2;
    float *sc = scale;   /* sc[j * nchunks + c] */
    /* maxima, per head over all chunks */
    for (int j = 0; j < hpb; j++) {
        const float *ph = part + (size_t)(h0 + j) * nchunks * stride;
        float m = -INFINITY;
        for (int c = tid; c < nchunks; c += CQ_WAVES * 64) m = fmaxf(m, ph[c * stride]);
        m = wave_max(m);
        if (lane == 0) redm[wave][j] = m;
    }
    __syncthreads();
    if (tid < hpb) {
        float M = redm[0][tid];
        for (int w = 1; w < CQ_WAVES; w++) M = fmaxf(M, redm[w][tid]);
        if (sinks) M = fmaxf(M, sinks[h0 + tid]);
        hm[tid] = M;
    }
    __syncthreads();
    /* chunk scales and the sums of exponentials */
    for (int j = 0; j < hpb; j++) {
        const float *ph = part + (size_t)(h0 + j) * nchunks * stride;
        const float M = hm[j];
        float l = 0.f;
        for (int c = tid; c < nchunks; c += CQ_WAVES * 64) {
            const float e = expf(ph[c * stride] - M);
            sc[j * nchunks + c] = e;
            l = fmaf(ph[c * stride + 1], e, l);
        }
        l = wave_sum(l);
        if (lane == 0) redl[wave][j] = l;
    }
    __syncthreads();
    if (tid < hpb) {
        float L = redl[0][tid];
        for (int w = 1; w < CQ_WAVES; w++) L += redl[w][tid];
        if (sinks) L += expf(sinks[h0 + tid] - hm[tid]);
        hl[tid] = 1.f / L;
    }
    /* V sums: lane p, chunks c = wave (mod 8) */
    const int tph = head_dim / 4;
    const int j = lane / tph, d = 4 * (lane - j * tph);
    const float *ph = part + (size_t)(h0 + j) * nchunks * stride + 2 + d;
    const float *sj = sc + j * nchunks;
    float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
#pragma unroll 8
    for (int c = wave; c < nchunks; c += CQ_WAVES) {
        const float2 a = *reinterpret_cast<const float2 *>(ph + c * stride);
        const float2 b = *reinterpret_cast<const float2 *>(ph + c * stride + 2);
        const float e = sj[c];
        o0 = fmaf(a.x, e, o0);
        o1 = fmaf(a.y, e, o1);
        o2 = fmaf(b.x, e, o2);
        o3 = fmaf(b.y, e, o3);
    }
    reinterpret_cast<float4 *>(osum[wave])[lane] = make_float4(o0, o1, o2, o3);
    __syncthreads();
    if (wave == 0) {
        float4 r = reinterpret_cast<const float4 *>(osum[0])[lane];
        for (int w = 1; w < CQ_WAVES; w++) {
            const float4 t = reinterpret_cast<const float4 *>(osum[w])[lane];
            r.x += t.x;
            r.y += t.y;
            r.z += t.z;
            r.w += t.w;
        }
        const float li = hl[j];
        r.x *= li;
        r.y *= li;
        r.z *= li;
        r.w *= li;
        reinterpret_cast<float4 *>(att + (size_t)h0 * head_dim)[lane] = r;
        q8_block_store(r.x, r.y, r.z, r.w, lane, aq, 0, blockIdx.x);
    }
}

void launch_attention_core(const float *qkv, const float *q_norm_w, const float *k_norm_w, const float *sinks,
                           float *kv_k, float *kv_v, int kv_len, int kv_max, int window, const float *rope_cos_row,
                           const float *rope_sin_row, int n_heads, int n_kv, int head_dim, float eps, float *part,
                           float *att, const Q8Rows *aq, hipStream_t st, unsigned *ctr) {
    const int seq_len = kv_len + 1;
    const int start = (window > 0 && seq_len > window) ? seq_len - window : 0;
    const int nchunks = (seq_len - start + CHUNK - 1) / CHUNK;
    const float inv_sqrt = 1.f / sqrtf((float)head_dim);
    if (aq && ctr && attention_fuse_ok(n_heads, n_kv, head_dim, kv_len, window)) {
        const AttnFuse fz = {ctr, sinks, att, *aq};
        hipLaunchKernelGGL(k_attn_partial<true>, dim3(nchunks, n_kv), dim3(256), 0, st, qkv, q_norm_w, k_norm_w,
                           rope_cos_row, rope_sin_row, kv_k, kv_v, part, n_heads, n_kv, head_dim, kv_len, kv_max,
                           start, seq_len, inv_sqrt, eps, fz);
        return;
    }
    const AttnFuse none = {};
    hipLaunchKernelGGL(k_attn_partial<false>, dim3(nchunks, n_kv), dim3(256), 0, st, qkv, q_norm_w, k_norm_w,
                       rope_cos_row, rope_sin_row, kv_k, kv_v, part, n_heads, n_kv, head_dim, kv_len, kv_max, start,
                       seq_len, inv_sqrt, eps, none);
    if (aq) {
        hipLaunchKernelGGL(k_attn_combine_q8, dim3(n_heads * head_dim / 256), dim3(CQ_WAVES * 64), 0, st, part, sinks,
                           att, n_heads, head_dim, nchunks, *aq);
    } else {
        hipLaunchKernelGGL(k_attn_combine, dim3(n_heads), dim3(256), 0, st, part, sinks, att, n_heads, head_dim,
                           nchunks);
    }
}

bool attention_combine_q8_ok(int n_heads, int head_dim) {
    /* k_attn_combine_q8 holds at most 4 heads per block */
    return head_dim >= 64 && 256 % head_dim == 0 && (n_heads * head_dim) % 256 == 0;
}

bool attention_fuse_ok(int n_heads, int n_kv, int head_dim, int kv_len, int window) {
    const int seq_len = kv_len + 1;
    const int span = (window > 0 && seq_len > window) ? window : seq_len;
    const int nchunks = (span + CHUNK - 1) / CHUNK;
    const int ratio = n_heads / n_kv;
    return attention_combine_q8_ok(n_heads, head_dim) && nchunks <= ATTN_FUSE_MAX_CHUNKS && ratio <= 8 &&
           (ratio * head_dim) % 256 == 0;
}

}  // namespace tg
