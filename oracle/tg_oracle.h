/*
 * tg_oracle.h -- CPU restatement of the reference arithmetic of the fused
 * quantized MoE expert path (csrc/libtinygiant.c of andrew-the-drawer/tinygiant).
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the HIP product is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links or calls it.
 *
 * Every function cites the reference function it restates.  The restatement
 * is written from the reference's semantics in portable scalar C (no NEON):
 * integer parts are exact, float parts follow the reference's grouping and
 * are compiled with -ffp-contract=off (no FMA contraction, no fast-math).
 */
#ifndef TG_ORACLE_H
#define TG_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_FMT_Q4K = 0, OR_FMT_F16 = 1, OR_FMT_Q6K = 2, OR_FMT_MXFP4 = 3, OR_FMT_Q80 = 4 };
enum { OR_ACT_SILU = 0, OR_ACT_GPTOSS = 1 };

/* Activation quant block, byte-identical to the reference's q8_block
 * (csrc/libtinygiant.c:159-164): 4 + 4 + 32 + 256 = 296 bytes. */
typedef struct {
    float   scale;
    int32_t sum;
    int32_t bsums[8];
    int8_t  qs[256];
} or_q8_block;

int      or_q8_nblocks(int ncols);
float    or_f16_to_f32(uint16_t h);
void     or_get_scale_min_k4(int j, const uint8_t *scales, uint8_t *sc, uint8_t *m);
float    or_e8m0_half(uint8_t e);
size_t   or_row_bytes(int fmt, int ncols);

void     or_quantize_q8(const float *x, or_q8_block *out, int ncols);

float    or_dot_q4k_q8(const uint8_t *row, const or_q8_block *xq, int bpr);
void     or_dot_q4k_q8_x4(const uint8_t *row, const or_q8_block *const xq[4], int bpr, float out[4]);
float    or_dot_q6k_q8(const uint8_t *row, const or_q8_block *xq, int bpr);
void     or_dot_q6k_q8_x4(const uint8_t *row, const or_q8_block *const xq[4], int bpr, float out[4]);
float    or_dot_mxfp4_q8(const uint8_t *row, const or_q8_block *xq, int ncols);
void     or_dot_mxfp4_q8_x4(const uint8_t *row, const or_q8_block *const xq[4], int ncols, float out[4]);
float    or_dot_q80_q8(const uint8_t *row, const or_q8_block *xq, int ncols);
float    or_dot_f16(const uint16_t *row, const float *x, int ncols);

/* Per-sub-block integer dot sums of one weight row against one q8 row:
 * Q4K: 8 sums of 32 per 256-block; Q6K: 16 sums of 16 per 256-block (with the
 * -32 offset applied); MXFP4 and Q80: one sum of 32 per 32-block.
 * Returns the number of sums written. */
int      or_isums(int fmt, const uint8_t *row, const or_q8_block *xq, int ncols, int32_t *out);

void     or_set_threads(int n);
int      or_get_threads(void);

void     or_matmul(int fmt, const void *mat, const float *bias, const float *input,
                   float *output, int nrows, int ncols);
void     or_matmul_q4k_scalar(const uint8_t *mat, const float *input, float *output,
                              int nrows, int ncols);
void     or_rms_norm(const float *x, const float *weight, float *out, int dim, float eps);

void     or_moe_forward_rows_v2(const uint8_t *const *gate_ptrs, const uint8_t *const *up_ptrs,
                                const void *const *down_ptrs, int gate_fmt, const int *down_fmts,
                                const float *const *gate_bias, const float *const *up_bias,
                                const float *const *down_bias, int act, int n_experts,
                                const float *row_weights, const float *inputs, float *output,
                                int k, int embed_dim, int inter_dim);
void     or_moe_forward_rows_v2_ex(const uint8_t *const *gate_ptrs, const uint8_t *const *up_ptrs,
                                   const void *const *down_ptrs, int gate_fmt, const int *down_fmts,
                                   const float *const *gate_bias, const float *const *up_bias,
                                   const float *const *down_bias, int act, int n_experts,
                                   const float *row_weights, const float *inputs, float *output,
                                   int k, int embed_dim, int inter_dim,
                                   const float *hidden_in, float *hidden_out);
/* Decode attention for one row (tg_attention_v2).  att_out, when not NULL,
 * receives the per-head attention output [n_heads * head_dim] before the
 * output projection. */
void     or_attention_v2(int fmt_q, int fmt_k, int fmt_v, int fmt_o,
                         const void *wq, const void *wk, const void *wv, const void *wo,
                         const float *bq, const float *bk, const float *bv, const float *bo,
                         const float *q_norm_w, const float *k_norm_w, const float *sinks,
                         float *kv_k, float *kv_v, int kv_len, int kv_max, int window,
                         const float *rope_cos, const float *rope_sin,
                         const float *input, float *output,
                         int embed_dim, int n_heads, int n_kv_heads, int head_dim, int pos, float eps,
                         float *att_out);
void     or_expert_forward(const uint8_t *q4_data, const float *input, float *output,
                           float weight, int embed_dim, int inter_dim);
void     or_expert_forward_mixed(const uint8_t *gate, const uint8_t *up, const void *down,
                                 int down_format, const float *input, float *output,
                                 float weight, int embed_dim, int inter_dim);

#ifdef __cplusplus
}
#endif
#endif
