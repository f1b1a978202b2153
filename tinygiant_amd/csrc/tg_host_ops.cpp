/*
 * tg_host_ops.cpp -- the reference ABI symbols that are outside the fused
 * MoE expert path: RMSNorm, f32/f16 matvecs, the three decode-attention
 * entry points, the full transformer layer and the page-cache hints.
 *
 * They exist so that tinygiant/_lib.py (which binds every symbol at load
 * time) and tinygiant/engine.py run unchanged against libtinygiant_hip.
 * tg_attention_v2 runs on the GPU (tg_api.hip, tg_attn.hip); the f32-weight
 * attention entry point here keeps its small arithmetic on the host,
 * single-threaded, and tg_attention_decode_q4 forwards to tg_attention_v2.
 * Semantics follow csrc/libtinygiant.c line for line where cited.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>
#include <sys/mman.h>

#include <vector>

#define TG_API extern "C" __attribute__((visibility("default")))

extern "C" void tg_matmul(int fmt, const void *mat, const float *bias, const float *input, float *output,
                          int nrows, int ncols);
/* on the GPU (tg_api.hip) */
extern "C" void tg_attention_v2(int fmt_q, int fmt_k, int fmt_v, int fmt_o, const void *wq, const void *wk,
                                const void *wv, const void *wo, const float *bq, const float *bk, const float *bv,
                                const float *bo, const float *q_norm_w, const float *k_norm_w, const float *sinks,
                                float *kv_k, float *kv_v, int kv_len, int kv_max, int window, const float *rope_cos,
                                const float *rope_sin, const float *input, float *output, int embed_dim, int n_heads,
                                int n_kv_heads, int head_dim, int pos, float eps);
extern "C" void tg_expert_forward_mixed(const uint8_t *gate_q4, const uint8_t *up_q4, const void *down_data,
                                        int down_format, const float *input, float *output, float weight,
                                        int embed_dim, int inter_dim);

namespace {

float half_to_float(uint16_t h) {
    uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t f;
    if (e == 0) {
        if (m == 0) {
            f = s;
        } else {
            int sh = 0;
            while (!(m & 0x400u)) {
                m <<= 1;
                sh++;
            }
            m &= 0x3FFu;
            f = s | ((uint32_t)(113 - sh) << 23) | (m << 13);
        }
    } else if (e == 31) {
        f = s | 0x7F800000u | (m << 13);
    } else {
        f = s | ((e + 112u) << 23) | (m << 13);
    }
    float r;
    memcpy(&r, &f, 4);
    return r;
}

void rope(float *x, int n_heads, int head_dim, const float *cos_t, const float *sin_t, int pos) {
    /* apply_rope_inplace (csrc/libtinygiant.c:702-719): NeoX halves */
    int half = head_dim / 2;
    const float *c = cos_t + (size_t)pos * half, *s = sin_t + (size_t)pos * half;
    for (int h = 0; h < n_heads; h++) {
        float *xh = x + (size_t)h * head_dim;
        for (int i = 0; i < half; i++) {
            float x1 = xh[i], x2 = xh[half + i];
            xh[i] = x1 * c[i] - x2 * s[i];
            xh[half + i] = x2 * c[i] + x1 * s[i];
        }
    }
}

/* one head of GQA decode attention over positions [start, seq_len)
 * (head_task, csrc/libtinygiant.c:862-904) */
void attend(const float *q_h, const float *k_cache, const float *v_cache, float *out_h, int start, int seq_len,
            int head_dim, float inv_sqrt, const float *sink) {
    std::vector<float> sc((size_t)(seq_len - start));
    float mx = sink ? *sink : -1e30f;
    for (int t = start; t < seq_len; t++) {
        const float *kt = k_cache + (size_t)t * head_dim;
        float dot = 0.f;
        for (int d = 0; d < head_dim; d++) dot += q_h[d] * kt[d];
        sc[t - start] = dot * inv_sqrt;
        if (sc[t - start] > mx) mx = sc[t - start];
    }
    float sum = sink ? expf(*sink - mx) : 0.f;
    for (int t = start; t < seq_len; t++) {
        sc[t - start] = expf(sc[t - start] - mx);
        sum += sc[t - start];
    }
    float inv = 1.f / sum;
    memset(out_h, 0, (size_t)head_dim * sizeof(float));
    for (int t = start; t < seq_len; t++) {
        float w = sc[t - start] * inv;
        const float *vt = v_cache + (size_t)t * head_dim;
        for (int d = 0; d < head_dim; d++) out_h[d] += w * vt[d];
    }
}

}  // namespace

TG_API void tg_rms_norm(const float *x, const float *weight, float *out, int dim, float eps) {
    float ss = 0.f;
    for (int i = 0; i < dim; i++) ss += x[i] * x[i];
    float scale = 1.f / sqrtf(ss / dim + eps);
    for (int i = 0; i < dim; i++) out[i] = (x[i] * scale) * weight[i];
}

TG_API void tg_f32_matvec(const float *A, const float *x, float *out, int nrows, int ncols) {
    for (int r = 0; r < nrows; r++) {
        const float *row = A + (size_t)r * ncols;
        float s = 0.f;
        for (int i = 0; i < ncols; i++) s += row[i] * x[i];
        out[r] = s;
    }
}

TG_API void tg_f16_matvec(const uint16_t *A, const float *x, float *out, int nrows, int ncols) {
    for (int r = 0; r < nrows; r++) {
        const uint16_t *row = A + (size_t)r * ncols;
        float s = 0.f;
        for (int i = 0; i < ncols; i++) s += half_to_float(row[i]) * x[i];
        out[r] = s;
    }
}

/* tg_attention_decode (csrc/libtinygiant.c:723-814): f32 projections */
TG_API void tg_attention_decode(const float *wq, const float *wk, const float *wv, const float *wo,
                                const float *q_norm_w, const float *k_norm_w, float *kv_k, float *kv_v, int kv_len,
                                int kv_max, const float *rope_cos, const float *rope_sin, const float *input,
                                float *output, int embed_dim, int n_heads, int n_kv_heads, int head_dim, int pos) {
    int q_dim = n_heads * head_dim, kv_dim = n_kv_heads * head_dim, ratio = n_heads / n_kv_heads;
    std::vector<float> q(q_dim), k(kv_dim), v(kv_dim), att(q_dim);
    tg_f32_matvec(wq, input, q.data(), q_dim, embed_dim);
    tg_f32_matvec(wk, input, k.data(), kv_dim, embed_dim);
    tg_f32_matvec(wv, input, v.data(), kv_dim, embed_dim);
    for (int h = 0; h < n_heads; h++) tg_rms_norm(&q[(size_t)h * head_dim], q_norm_w, &q[(size_t)h * head_dim], head_dim, 1e-6f);
    for (int h = 0; h < n_kv_heads; h++) tg_rms_norm(&k[(size_t)h * head_dim], k_norm_w, &k[(size_t)h * head_dim], head_dim, 1e-6f);
    rope(q.data(), n_heads, head_dim, rope_cos, rope_sin, pos);
    rope(k.data(), n_kv_heads, head_dim, rope_cos, rope_sin, pos);
    for (int h = 0; h < n_kv_heads; h++) {
        memcpy(kv_k + ((size_t)h * kv_max + kv_len) * head_dim, &k[(size_t)h * head_dim], head_dim * 4);
        memcpy(kv_v + ((size_t)h * kv_max + kv_len) * head_dim, &v[(size_t)h * head_dim], head_dim * 4);
    }
    float inv_sqrt = 1.f / sqrtf((float)head_dim);
    for (int h = 0; h < n_heads; h++) {
        int kh = h / ratio;
        attend(&q[(size_t)h * head_dim], kv_k + (size_t)kh * kv_max * head_dim, kv_v + (size_t)kh * kv_max * head_dim,
               &att[(size_t)h * head_dim], 0, kv_len + 1, head_dim, inv_sqrt, nullptr);
    }
    tg_f32_matvec(wo, att.data(), output, embed_dim, q_dim);
}

/* tg_attention_decode_q4 (csrc/libtinygiant.c:985-1036): Q4_K q/k/o, f16 v */
TG_API void tg_attention_decode_q4(const uint8_t *wq_q4, const uint8_t *wk_q4, const uint16_t *wv_f16,
                                   const uint8_t *wo_q4, const float *q_norm_w, const float *k_norm_w, float *kv_k,
                                   float *kv_v, int kv_len, int kv_max, const float *rope_cos, const float *rope_sin,
                                   const float *input, float *output, int embed_dim, int n_heads, int n_kv_heads,
                                   int head_dim, int pos) {
    tg_attention_v2(0, 0, 1, 0, wq_q4, wk_q4, wv_f16, wo_q4, nullptr, nullptr, nullptr, nullptr, q_norm_w, k_norm_w,
                    nullptr, kv_k, kv_v, kv_len, kv_max, 0, rope_cos, rope_sin, input, output, embed_dim, n_heads,
                    n_kv_heads, head_dim, pos, 1e-6f);
}

/* tg_transformer_layer (csrc/libtinygiant.c:1467-1507) */
TG_API void tg_transformer_layer(const float *wq, const float *wk, const float *wv, const float *wo,
                                 const float *attn_norm_w, const float *q_norm_w, const float *k_norm_w,
                                 const float *ffn_norm_w, float *kv_k, float *kv_v, int kv_len, int kv_max,
                                 const float *rope_cos, const float *rope_sin, const uint8_t **gate_ptrs,
                                 const uint8_t **up_ptrs, const void **down_ptrs, const int *down_is_f16,
                                 const float *expert_weights, int n_active, float *x, int embed_dim, int inter_dim,
                                 int n_heads, int n_kv_heads, int head_dim, int pos) {
    std::vector<float> normed(embed_dim), attn(embed_dim), moe(embed_dim, 0.f);
    tg_rms_norm(x, attn_norm_w, normed.data(), embed_dim, 1e-6f);
    tg_attention_decode(wq, wk, wv, wo, q_norm_w, k_norm_w, kv_k, kv_v, kv_len, kv_max, rope_cos, rope_sin,
                        normed.data(), attn.data(), embed_dim, n_heads, n_kv_heads, head_dim, pos);
    for (int i = 0; i < embed_dim; i++) x[i] += attn[i];
    tg_rms_norm(x, ffn_norm_w, normed.data(), embed_dim, 1e-6f);
    for (int e = 0; e < n_active; e++)
        tg_expert_forward_mixed(gate_ptrs[e], up_ptrs[e], down_ptrs[e], down_is_f16[e], normed.data(), moe.data(),
                                expert_weights[e], embed_dim, inter_dim);
    for (int i = 0; i < embed_dim; i++) x[i] += moe[i];
}

/* posix_madvise(WILLNEED) over 16 KiB pages (csrc/libtinygiant.c:1550-1564) */
TG_API void tg_prefetch(const void *addr, size_t len) {
    uintptr_t mask = ~((uintptr_t)16384 - 1);
    void *a = (void *)((uintptr_t)addr & mask);
    posix_madvise(a, len + ((uintptr_t)addr - (uintptr_t)a), POSIX_MADV_WILLNEED);
}

TG_API void tg_prefetch_batch(const void **addrs, const size_t *lens, int count) {
    for (int i = 0; i < count; i++) tg_prefetch(addrs[i], lens[i]);
}
