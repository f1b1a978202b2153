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
#define ATTN_FUSE_MAX_CHUNKS 32  /* chunks up to which the partial kernel also combines */

namespace tg {

/* The combine folded into the partial kernel (attention_fuse_ok): the last
 * workgroup of each KV head, by a ticket from ctr[kh], merges the chunks of
 * its query heads, writes att and q8 of it into row 0 of aq. */
struct AttnFuse {
    unsigned *ctr;        /* n_kv counters, zero when the kernel starts */
    const float *sinks;
    float *att;
    Q8Rows aq;
};

/* qkv: [q_dim | kv_dim | kv_dim] projection outputs; rope rows are the
 * cos/sin tables at pos; part [n_heads][ceil(span / ATTN_CHUNK)][head_dim + 2];
 * att [q_dim].  With aq given (attention_combine_q8_ok), q8 of att is also
 * written to row 0 of aq.  With ctr also given and attention_fuse_ok, the
 * combine runs inside the partial kernel (two launches become one); ctr
 * holds n_kv counters that must be zero (launch_gemv_q8x clears them). */
void launch_attention_core(const float *qkv, const float *q_norm_w, const float *k_norm_w, const float *sinks,
                           float *kv_k, float *kv_v, int kv_len, int kv_max, int window, const float *rope_cos_row,
                           const float *rope_sin_row, int n_heads, int n_kv, int head_dim, float eps, float *part,
                           float *att, const Q8Rows *aq, hipStream_t st, unsigned *ctr = nullptr);
bool attention_combine_q8_ok(int n_heads, int head_dim);
/* whether the combine folds into the partial kernel for this shape and span
 * (then launch_attention_core needs aq and ctr) */
bool attention_fuse_ok(int n_heads, int n_kv, int head_dim, int kv_len, int window);

}  // namespace tg
#endif
