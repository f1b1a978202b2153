/*
 * tg_head.h -- output head with fused argmax (internal launch interface).
 */
#ifndef TG_HEAD_H
#define TG_HEAD_H
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tg_device.hpp"

namespace tg {

/* The fused kernel covers Q6_K heads of 2048 columns, up to 2^20 vocab rows
 * and 1..16 input rows. */
bool head_fast_ok(int fmt, int ncols, int nrows, int k);
/* best[0..k) receive packed argmax keys and best[16] counts finished
 * workgroups: all 17 words must be zero at launch (launch_rms_norm_q8 and
 * launch_quantize clear them); the last workgroup writes idx[k] and val[k]
 * (val may be null); logits may be null. */
constexpr int HEAD_KEY_WORDS = 17;
void launch_head_q6k(const uint8_t *W, int nrows, const Q8Rows &x, int k, float *logits, unsigned long long *best,
                     int32_t *idx, float *val, hipStream_t st);
/* k at which launch_head_q6k switches to the int8 MFMA kernel (0: never);
 * returns the previous setting */
int set_head_mfma_min_k(int k);
/* argmax keys of materialized logits [k][nrows] */
void launch_argmax_rows(const float *logits, int nrows, int k, unsigned long long *best, hipStream_t st);
/* keys -> row index and logit */
void launch_argmax_finish(const unsigned long long *best, int k, int32_t *idx, float *val, hipStream_t st);

}  // namespace tg
#endif
