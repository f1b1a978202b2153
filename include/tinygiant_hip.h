/*
 * tinygiant_hip.h -- C ABI of libtinygiant_hip.so, the MI355X (gfx950)
 * implementation of TinyGiant's fused quantized MoE expert path.
 *
 * Part 1 declares the 21 symbols that tinygiant/_lib.py:39-93 binds with
 * ctypes, with the reference's exact C signatures (csrc/libtinygiant.c), so
 * the library is a drop-in for libtinygiant.{so,dylib}.  Part 2 declares the
 * device-resident extensions (tg_hip_*), which have no reference counterpart.
 *
 * Conventions shared with the reference:
 *   formats   0 = Q4_K (144-byte 256-blocks), 1 = F16, 2 = Q6_K (210-byte
 *             256-blocks), 3 = MXFP4 (17-byte 32-blocks), 4 = Q8_0 (34-byte
 *             32-blocks)                        (csrc/libtinygiant.c:594)
 *   act       0 = SiLU(g)*u, 1 = gpt-oss clamp/sigmoid(1.702 g)*(u+1) (:1248)
 *   outputs of the MoE entry points are accumulated (+=), not overwritten
 *   every call is synchronous: outputs are complete on return
 *   all pointers in Part 1 are host pointers; a pointer inside a range given
 *   to tg_mlock resolves to that range's copy in HBM, any other weight
 *   pointer is staged to the device for the duration of the call
 *   activation widths (embed_dim, inter_dim, ncols) are multiples of 32
 */
#ifndef TINYGIANT_HIP_H
#define TINYGIANT_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ======================= Part 1: reference ABI ======================= */

/* Fused top-k expert FFN over k rows (replaces csrc/libtinygiant.c:1386-1437,
 * bound at tinygiant/_lib.py:74-75, called at tinygiant/engine.py:336-340).
 * row_weights[e*k + r] == 0 excludes row r from expert e. */
void tg_moe_forward_rows_v2(const uint8_t *const *gate_ptrs, const uint8_t *const *up_ptrs,
                            const void *const *down_ptrs, int gate_fmt, const int *down_fmts,
                            const float *const *gate_bias, const float *const *up_bias,
                            const float *const *down_bias, int act, int n_experts,
                            const float *row_weights, const float *inputs, float *output, int k,
                            int embed_dim, int inter_dim);

/* v2 with Q4_K gate/up, no biases, SiLU (replaces :1439-1448; _lib.py:90) */
void tg_moe_forward_rows(const uint8_t *const *gate_ptrs, const uint8_t *const *up_ptrs,
                         const void *const *down_ptrs, const int *down_fmts, int n_experts,
                         const float *row_weights, const float *inputs, float *output, int k,
                         int embed_dim, int inter_dim);

/* Sum over experts of weight * all-Q4_K expert [gate|up|down]; zeroes output
 * first (replaces :1452-1460; exported, not bound by _lib.py). */
void tg_moe_forward(const uint8_t **expert_ptrs, const float *weights, int n_experts,
                    const float *input, float *output, int embed_dim, int inter_dim);

/* output += weight * expert(input), all-Q4_K [gate|up|down] buffer
 * (replaces :1040-1080; _lib.py:42) */
void tg_expert_forward(const uint8_t *q4_data, const float *input, float *output, float weight,
                       int embed_dim, int inter_dim);

/* down_format 1 = f16, 2 = q6_K, else q4_K (replaces :1084-1128; _lib.py:43-44) */
void tg_expert_forward_mixed(const uint8_t *gate_q4, const uint8_t *up_q4, const void *down_data,
                             int down_format, const float *input, float *output, float weight,
                             int embed_dim, int inter_dim);

/* output[r] += weights[r] * expert(inputs[r]) for k rows (replaces :1182-1231; _lib.py:89) */
void tg_expert_forward_rows(const uint8_t *gate_q4, const uint8_t *up_q4, const void *down_data,
                            int down_format, const float *inputs, float *output, const float *weights,
                            int k, int embed_dim, int inter_dim);

/* output[r] = dot(mat row r, q8(input)) + bias[r] (replaces :925-931; _lib.py:76,
 * called at tinygiant/engine.py:352) */
void tg_matmul(int fmt, const void *mat, const float *bias, const float *input, float *output,
               int nrows, int ncols);
void tg_matmul_q4k(const uint8_t *q4_matrix, const float *input, float *output, int nrows,
                   int ncols);                                   /* :375-378; _lib.py:45 */
void tg_matmul_q6k(const uint8_t *q6_matrix, const float *input, float *output, int nrows,
                   int ncols);                                   /* :498-501; _lib.py:46 */
size_t tg_row_bytes(int fmt, int ncols);                         /* :606; _lib.py:77-78 */

/* The reference sizes its CPU pool (:85-104); here the count sizes nothing on
 * the GPU path and is returned by tg_get_threads.  _lib.py:79-81 */
void tg_set_threads(int n);
int tg_get_threads(void);

/* The reference mlocks host pages (:1566-1571; _lib.py:65-66, called by
 * tinygiant/cache.py:153-162 for every pinned expert view).  Here the range
 * is copied into HBM once and later pointers into it use the copy.
 * Returns 0, or -1 if HBM is exhausted. */
int tg_mlock(const void *addr, size_t len);

/* Out of the hot path; served so the engine runs unchanged (tg_host_ops.cpp). */
void tg_rms_norm(const float *x, const float *weight, float *out, int dim, float eps); /* :680; _lib.py:47 */
void tg_f32_matvec(const float *A, const float *x, float *out, int nrows, int ncols); /* :662; _lib.py:48 */
void tg_f16_matvec(const uint16_t *A, const float *x, float *out, int nrows, int ncols); /* :655; _lib.py:49 */
void tg_attention_decode(const float *wq, const float *wk, const float *wv, const float *wo,
                         const float *q_norm_w, const float *k_norm_w, float *kv_k, float *kv_v,
                         int kv_len, int kv_max, const float *rope_cos, const float *rope_sin,
                         const float *input, float *output, int embed_dim, int n_heads,
                         int n_kv_heads, int head_dim, int pos);          /* :723; _lib.py:50-56 */
void tg_attention_decode_q4(const uint8_t *wq_q4, const uint8_t *wk_q4, const uint16_t *wv_f16,
                            const uint8_t *wo_q4, const float *q_norm_w, const float *k_norm_w,
                            float *kv_k, float *kv_v, int kv_len, int kv_max, const float *rope_cos,
                            const float *rope_sin, const float *input, float *output, int embed_dim,
                            int n_heads, int n_kv_heads, int head_dim, int pos); /* :985; _lib.py:57-63 */
void tg_attention_v2(int fmt_q, int fmt_k, int fmt_v, int fmt_o, const void *wq, const void *wk,
                     const void *wv, const void *wo, const float *bq, const float *bk, const float *bv,
                     const float *bo, const float *q_norm_w, const float *k_norm_w, const float *sinks,
                     float *kv_k, float *kv_v, int kv_len, int kv_max, int window,
                     const float *rope_cos, const float *rope_sin, const float *input, float *output,
                     int embed_dim, int n_heads, int n_kv_heads, int head_dim, int pos,
                     float eps);                                          /* :939; _lib.py:67-73 */
void tg_transformer_layer(const float *wq, const float *wk, const float *wv, const float *wo,
                          const float *attn_norm_w, const float *q_norm_w, const float *k_norm_w,
                          const float *ffn_norm_w, float *kv_k, float *kv_v, int kv_len, int kv_max,
                          const float *rope_cos, const float *rope_sin, const uint8_t **gate_ptrs,
                          const uint8_t **up_ptrs, const void **down_ptrs, const int *down_is_f16,
                          const float *expert_weights, int n_active, float *x, int embed_dim,
                          int inter_dim, int n_heads, int n_kv_heads, int head_dim,
                          int pos);                                       /* :1467; _lib.py:91-92 */
void tg_prefetch(const void *addr, size_t len);                         /* :1550; _lib.py:64 */
void tg_prefetch_batch(const void **addrs, const size_t *lens, int count); /* :1557; _lib.py:64 */

/* ================ Part 2: device-resident extensions ================ */
/* No reference counterpart.  Pointers named *_dev are device pointers;
 * `stream` is a hipStream_t (NULL = the library's stream).  These only queue
 * work (except where noted) and never allocate inside *_run/*_dev calls. */

const char *tg_hip_last_error(void);           /* last argument error, "" if none */
void tg_hip_clear_error(void);
int tg_hip_register(const void *addr, size_t len);   /* = tg_mlock */
int tg_hip_unregister(const void *addr);             /* frees the HBM copy; 0 or -1 */
size_t tg_hip_registered_bytes(void);
const void *tg_hip_device_ptr(const void *host, size_t n);  /* HBM copy of a registered range */
void *tg_hip_stream(void);
void *tg_hip_malloc(size_t n);
void tg_hip_free(void *p);
void tg_hip_memcpy_h2d(void *dst_dev, const void *src, size_t n);   /* synchronous */
void tg_hip_memcpy_d2h(void *dst, const void *src_dev, size_t n);   /* synchronous */
void tg_hip_memcpy_d2d(void *dst_dev, const void *src_dev, size_t n, void *stream);
void tg_hip_synchronize(void);
/* No counterpart in the reference (its CPU library holds no device state).
 * Waits for the device, then releases the library's stream, arena, pinned
 * rows, upload buffers and timing marks; a later call re-initialises.  Plans,
 * decode steps and device arrays are the caller's to destroy first. */
void tg_hip_shutdown(void);

/* Seeded synthetic tensors: kind -1 raw bytes, 0 Q4_K, 2 Q6_K, 3 MXFP4, 4 Q8_0
 * (block scale fields drawn as documented in tg_synth.h). */
void tg_hip_synth_fill(int kind, uint64_t seed, void *dst_dev, uint64_t nbytes, void *stream);
void tg_hip_synth_fill_host(int kind, uint64_t seed, void *dst, uint64_t nbytes);

/* Parity probes (synchronous, host pointers). */
void tg_hip_quantize_q8(const float *x, int ncols, int nrows, void *out_blocks /* 296 B each */);
int tg_hip_isums(int fmt, const void *mat, int nrows, int ncols, const float *x, int32_t *out);

/* tg_moe_forward_rows_v2 plus its stage outputs (stage-wise parity): the
 * hidden rows [pairs][inter_dim] f32, pairs numbered expert-major in gather
 * order, and their q8 blocks [pairs][ceil(inter_dim/256)] (296 B each). */
void tg_hip_moe_forward_stages(const uint8_t *const *gate_ptrs, const uint8_t *const *up_ptrs,
                               const void *const *down_ptrs, int gate_fmt, const int *down_fmts,
                               const float *const *gate_bias, const float *const *up_bias,
                               const float *const *down_bias, int act, int n_experts,
                               const float *row_weights, const float *inputs, float *output, int k,
                               int embed_dim, int inter_dim, float *hidden_out, void *hq_blocks_out);

/* A MoE layer whose weights are already in HBM, planned once and replayed. */
typedef struct tg_hip_moe_plan tg_hip_moe_plan;
tg_hip_moe_plan *tg_hip_moe_plan_create(const void *const *gate_dev, const void *const *up_dev,
                                        const void *const *down_dev, int gate_fmt, const int *down_fmts,
                                        const float *const *gate_bias_dev, const float *const *up_bias_dev,
                                        const float *const *down_bias_dev, int act, int n_experts,
                                        const float *row_weights, int k, int embed_dim, int inter_dim);
void tg_hip_moe_plan_run(tg_hip_moe_plan *plan, const float *inputs_dev, float *output_dev, void *stream);
int tg_hip_moe_plan_pairs(const tg_hip_moe_plan *plan);
void tg_hip_moe_plan_destroy(tg_hip_moe_plan *plan);

/* k-row device GEMV: y[j][r] = dot(mat row r, q8(x_j)) + bias[r];
 * scratch_dev holds tg_hip_matmul_scratch_bytes(k, ncols) bytes. */
void tg_hip_matmul_dev(int fmt, const void *mat_dev, const float *bias_dev, const float *inputs_dev,
                       float *outputs_dev, int nrows, int ncols, int k, void *scratch_dev, void *stream);
size_t tg_hip_matmul_scratch_bytes(int k, int ncols);
/* No counterpart in the reference.  For callers that cannot allocate (code
 * under HIP graph capture, tight serving loops): tg_hip_matmul_dev with the
 * q8 rows of the inputs in the library's fixed device scratch instead of a
 * workspace argument; allocates nothing.  tg_hip_init() must have run on the
 * device first.  k * ceil(ncols / 256) * 360 bytes must fit in
 * tg_hip_matmul_noalloc_max_bytes() (384 KiB), else it sets
 * tg_hip_last_error() and leaves the outputs untouched.  Calls on one GPU
 * share the scratch: calls that overlap in time on one GPU race. */
void tg_hip_init(void);
void tg_hip_matmul_dev_noalloc(int fmt, const void *mat_dev, const float *bias_dev, const float *inputs_dev,
                               float *outputs_dev, int nrows, int ncols, int k, void *stream);
size_t tg_hip_matmul_noalloc_max_bytes(void);
void tg_hip_rms_norm_dev(const float *x_dev, const float *w_dev, float *out_dev, int nrows, int n,
                         float eps, void *stream);

/* MoE router over k device-resident rows x_j (normalized hidden states):
 * logits = router (n_experts x dim f32) . x_j (+ bias), the top_k experts by
 * descending logit into idx_dev [k][top_k], and their weights, a softmax over
 * the selected logits only, into w_dev [k][top_k] (replaces Router.logits,
 * _topk and _weights, tinygiant/router.py:29-42, for selection without cache
 * bias; n_experts <= 256, top_k <= 64).  scratch_dev holds
 * tg_hip_route_scratch_bytes(k, n_experts) bytes (the logits). */
void tg_hip_route_dev(const float *router_dev, const float *bias_dev, const float *x_dev, int k,
                      int n_experts, int dim, int top_k, int32_t *idx_dev, float *w_dev,
                      void *scratch_dev, void *stream);
size_t tg_hip_route_scratch_bytes(int k, int n_experts);
/* The same with the selection restricted to the resident experts
 * (resident_dev: one byte per expert, nonzero = resident), as
 * Router.select(restrict=True) does for a draft pass (tinygiant/router.py:
 * 46-54, called from engine.py:287 with mode="draft"): the other experts'
 * logits count as -inf for the top-k, the weights are the softmax of the
 * selected experts' own logits, and when fewer than top_k experts are
 * resident the selection is the unrestricted one. */
void tg_hip_route_restricted_dev(const float *router_dev, const float *bias_dev, const float *x_dev, int k,
                                 int n_experts, int dim, int top_k, const uint8_t *resident_dev,
                                 int32_t *idx_dev, float *w_dev, void *scratch_dev, void *stream);

/* Copies nbytes of the file at path, from file_offset on, into device
 * memory at dev_dst: pread into two pinned staging buffers of chunk_bytes
 * (at least 1 MiB) while the previous chunk's host-to-device copy runs.
 * Returns the bytes copied, or -1 with tg_hip_last_error() set (missing
 * file, short file, no pinned memory).  The native part of the expert-cache
 * loader (tinygiant_amd/loader.py), which uploads the reference's on-disk
 * expert cache (index.json + layer_NNN.q4.bin, tinygiant/relayout.py:147-162,
 * 287-300, read by tinygiant/cache.py:29-54) whole into HBM. */
int64_t tg_hip_upload_file(const char *path, uint64_t file_offset, uint64_t nbytes, void *dev_dst,
                           uint64_t chunk_bytes);

/* Decode attention for one row with every pointer on the device (replaces
 * tg_attention_v2, csrc/libtinygiant.c:939-983, with the same arguments and
 * meaning): q8 of input, Q/K/V projections (+ biases), the optional per-head
 * QK RMS norm, RoPE at pos, K/V rows stored at kv_len of kv_k / kv_v
 * [n_kv_heads][kv_max][head_dim], GQA softmax attention over the last
 * `window` positions (0: all) with optional per-head sink logits, and the
 * output projection into output (overwritten).  att_out, when not NULL,
 * receives the per-head attention output [n_heads * head_dim] before the
 * output projection.  scratch holds tg_hip_attention_scratch_bytes(...)
 * bytes.  Shapes: embed_dim % 32 == 0, head_dim % 4 == 0 and <= 128,
 * n_heads / n_kv_heads integral and <= 8, kv_len < kv_max <= 65536;
 * kv_k and kv_v 16-byte aligned. */
void tg_hip_attention_dev(int fmt_q, int fmt_k, int fmt_v, int fmt_o, const void *wq, const void *wk,
                          const void *wv, const void *wo, const float *bq, const float *bk, const float *bv,
                          const float *bo, const float *q_norm_w, const float *k_norm_w, const float *sinks,
                          float *kv_k, float *kv_v, int kv_len, int kv_max, int window, const float *rope_cos,
                          const float *rope_sin, const float *input, float *output, int embed_dim, int n_heads,
                          int n_kv_heads, int head_dim, int pos, float eps, float *att_out, void *scratch,
                          void *stream);
size_t tg_hip_attention_scratch_bytes(int embed_dim, int n_heads, int n_kv_heads, int head_dim, int kv_max);

/* Output head over k (1..16) device-resident rows with the argmax fused in:
 * x_j = RMSNorm(inputs_j) * norm_w (skipped when norm_w_dev is NULL),
 * logits[j][r] = dot(mat row r, q8(x_j)) and argmax_dev[j] = the first r
 * with the largest logit, maxval_dev[j] its logit (may be NULL).  Replaces
 * the reference's per-row tg_rms_norm + tg_matmul over the head
 * (tinygiant/engine.py:347-354) and numpy.argmax over each row
 * (tinygiant/specdec.py:77,90); Q6_K heads of 2048 columns read the head
 * once for all rows.  logits_dev (k x nrows) may be NULL; scratch_dev holds
 * tg_hip_head_scratch_bytes(k, nrows, ncols) bytes. */
void tg_hip_head_argmax_dev(int fmt, const void *mat_dev, const float *inputs_dev,
                            const float *norm_w_dev, float eps, int k, int nrows, int ncols,
                            float *logits_dev, int32_t *argmax_dev, float *maxval_dev,
                            void *scratch_dev, void *stream);
size_t tg_hip_head_scratch_bytes(int k, int nrows, int ncols);

/* Device-resident decode step over L planned layers sharing one hidden
 * state h_dev [k][embed_dim]: h <- h + MoE_l(RMSNorm_l(h)) for each layer
 * (tinygiant/engine.py:281-282,335-341).  norm_w_dev may be NULL (weight 1).
 * mode 0 queues the per-layer kernels, 1 replays them as one HIP graph,
 * 2 runs the whole step as one persistent cooperative kernel on 256
 * co-resident workgroups.  For k = 2..16 rows (a verify pass of K + 1 rows,
 * tinygiant/specdec.py:66, or a prefill chunk, engine.py:213-217) that is
 * the multi-row kernel: any number of layers of the Qwen3-30B-A3B expert
 * shape (D = 2048, I = 768, Q4_K gate/up, Q6_K down, SiLU, no biases), up to
 * 128 active experts and 256 pairs per layer, the bits of mode 0.  For
 * k = 1, <= 64 layers of one of two expert shapes:
 *   Qwen3-30B-A3B: D = 2048, I = 768, Q4_K gate/up, Q6_K down, SiLU, no
 *     biases, exactly 8 active experts per layer;
 *   gpt-oss-120b: D = I = 2880, MXFP4 gate/up/down, the clamped SwiGLU,
 *     optional biases, exactly 4 active experts per layer (MXFP4 dots on
 *     block-scaled MFMA: the reference's per-block integer sums, f32
 *     additions grouped differently);
 * (mode 2 launches it as the one cooperative node of a HIP graph, rebuilt
 * when a setter below changes its arguments);
 * 3 launches the same kernel with a plain launch (for tools that do not
 * follow cooperative launches; needs an otherwise idle device, and a step
 * whose workgroups are not all resident ends with status 1).  The persistent
 * kernels keep their launch epoch on the device, so a caller may capture a
 * mode-3 tg_hip_decode_run into a graph of its own and replay it. */
typedef struct tg_hip_decode tg_hip_decode;
tg_hip_decode *tg_hip_decode_create(tg_hip_moe_plan *const *plans, int n_layers,
                                    const float *const *norm_w_dev, float eps, float *h_dev,
                                    int mode);
/* 0 ok; 1 if a persistent step's exchange wait timed out; 2 if a launch split
 * a class of workgroups g % 8 over several XCDs, which its intra-XCD
 * exchanges assume they share -- the step then stores every slot
 * device-coherently from the next launch on */
int tg_hip_decode_status(tg_hip_decode *step);
/* Persistent steps: exchange-slot policy 0 (intra-XCD slots stay in the
 * writer's L2; the default) or 1 (every slot device-coherent, correct under
 * any placement; same bits).  Returns the previous policy, -1 otherwise. */
int tg_hip_decode_set_policy(tg_hip_decode *step, int policy);
/* Persistent steps: HW_REG_XCC_ID of each of its 256 workgroups in the last
 * launch into out[256]; returns the count written (0 if none). */
int tg_hip_decode_placement(tg_hip_decode *step, unsigned *out);
/* Stage-wise parity probe of the persistent step: while set, each layer
 * writes a record of tg_hip_decode_record_bytes(step) bytes into
 * debug_dev[layer]: for the Qwen3 kernel (tg_hip_decode_debug_bytes()) h in,
 * RMSNorm x, q8(x), hidden, q8(hidden); for the gpt-oss kernel h in, x and
 * each expert slot's hidden vector (f32). */
void tg_hip_decode_set_debug(tg_hip_decode *step, void *debug_dev);
size_t tg_hip_decode_debug_bytes(void);
size_t tg_hip_decode_record_bytes(tg_hip_decode *step);
/* Phase timing of the persistent step: while set, times_dev [256][L][24]
 * uint64 receives up to 24 words per layer of every workgroup (timestamps of
 * the 100 MHz device clock and exchange poll round counts). */
void tg_hip_decode_set_timing(tg_hip_decode *step, void *times_dev);
void tg_hip_decode_run(tg_hip_decode *step, void *stream);
float tg_hip_decode_time(tg_hip_decode *step, int iters);   /* ms for iters steps, HIP events */
void tg_hip_decode_kernel_times(tg_hip_decode *step, float *ms_out /*[6]*/, int *n_out /*[6]*/);
void tg_hip_decode_destroy(tg_hip_decode *step);
void tg_hip_device_name(char *buf, int n);
/* MXFP4 expert layers whose busiest expert holds at least `rows` pairs run
 * their gate/up and down phases on block-scaled MFMA (each weight block read
 * once per 64 pairs; the per-block integer sums of dot_mxfp4_q8,
 * csrc/libtinygiant.c:533-547, with the f32 additions grouped differently);
 * 0 keeps every layer on the per-pair kernels.
 * Default 4.  Returns the previous setting.  No counterpart in the
 * reference, which has one CPU kernel for every row count. */
int tg_hip_set_moe_grouped_min_rows(int rows);
/* Q4_K gate/up + Q6_K down expert layers whose busiest expert holds at
 * least `rows` pairs run both phases on int8 MFMA (each weight byte read
 * once per 16 pairs; the integer sums of dot_q4k_q8 / dot_q6k_q8,
 * csrc/libtinygiant.c:223-272, :384-443, with the f32 additions grouped
 * differently); 0 keeps every such layer on the v_dot4 phases.  A negative
 * value (the default) picks by shape: 17 where both persistent ring phases
 * run (D = 2048 gate/up rows, I = 768 down rows, no down bias), 40 for the
 * other shapes.  Returns the previous setting.  No counterpart in the
 * reference. */
int tg_hip_set_moe_qk_min_rows(int rows);
/* The fused q6_K head (tg_hip_head_argmax_dev) reads the head on int8 MFMA
 * from `k` input rows on: each block's integer sum is exact and its term
 * d * d_x * sum is added in block order, as dot_q6k_q8 does
 * (csrc/libtinygiant.c:403-443); below `k` the v_dot4 kernel runs (its work
 * grows with the row count); 0 keeps every call on the v_dot4 kernel.
 * Default 8.  Returns the previous setting.  No counterpart in the
 * reference. */
int tg_hip_set_head_mfma_min_k(int k);
/* Q4_K / Q6_K expert layers, and MXFP4 ones below the MFMA threshold, run
 * expert-major (bit 1): each weight row is
 * read once and dotted with the q8 row of every pair of its expert, as
 * moe_phase_a / moe_phase_b do with dot_fmt_x4 (csrc/libtinygiant.c:
 * 1279-1384, :622-628).  For a layer with at most two pairs per expert:
 * bit 2, the two phases quantize their rows themselves instead of q8
 * launches (rows of at most 2048 values); bit 4, the down phase also adds the partials into the output
 * rows (the last workgroup of each row tile, in expert order) instead of a
 * combine launch.  Bit 8: bits 2 and 4 whatever the pair count.  0 runs one
 * workgroup column per pair with the q8 and combine launches.  Every mode
 * gives the same bits.  Default 7; a negative mode
 * restores it.  Returns the previous mode.  A switch with no counterpart in
 * the reference. */
int tg_hip_set_moe_expert_major(int mode);
/* Event marks (slots 0..7) on the library stream; tg_hip_marks_ms waits for
 * mark b and returns the milliseconds between marks a and b. */
void tg_hip_mark(int slot);
float tg_hip_marks_ms(int a, int b);
/* nbytes (multiple of 16) device-to-device `iters` times with a plain copy
 * kernel; returns milliseconds (HIP events): measured HBM reference point. */
float tg_hip_copy_time(const void *src_dev, void *dst_dev, uint64_t nbytes, int iters);

#ifdef __cplusplus
}
#endif
#endif
