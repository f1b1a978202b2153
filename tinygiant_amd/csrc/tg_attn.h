/*
 * tg_attn.h -- device decode attention (internal launch interface).
 */
#ifndef TG_ATTN_H
#define TG_ATTN_H
#include <hip/hip_runtime.h>

#include "tg_device.hpp"

#define ATTN_CHUNK 32          /* sequence positions per workgroup */
#define ATTN_MAX_HEAD_DIM 128  /* head_dim: even, multiple of 4, at most this */
#define ATTN_MAX_GQA 8         /* query heads per KV head, at most this */
#define ATTN_MAX_CHUNKS 2048   /* kv_max <= ATTN_CHUNK * ATTN_MAX_CHUNKS */

namespace tg {

/* qkv: [q_dim | kv_dim | kv_dim] projection outputs; rope rows are the
 * cos/sin tables at pos; part [n_heads][ceil(span / ATTN_CHUNK)][head_dim + 2];
 * att [q_dim].  With aq given (attention_combine_q8_ok), q8 of att is also
 * written to row 0 of aq. */
void launch_attention_core(const float *qkv, const float *q_norm_w, const float *k_norm_w, const float *sinks,
                           float *kv_k, float *kv_v, int kv_len, int kv_max, int window, const float *rope_cos_row,
                           const float *rope_sin_row, int n_heads, int n_kv, int head_dim, float eps, float *part,
                           float *att, const Q8Rows *aq, hipStream_t st);
bool attention_combine_q8_ok(int n_heads, int head_dim);

}  // namespace tg
#endif
