/*
 * tg_head.h -- output head with fused argmax (internal launch interface).
 */
#ifndef TG_HEAD_H
#define TG_HEAD_H
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tg_device.hpp"

namespace tg {

/* The fused kernel covers Q6_K heads of 2048 columns and 1..16 rows. */
bool head_fast_ok(int fmt, int ncols, int k);
/* best[k] receives packed argmax keys (reset first); logits may be null. */
void launch_head_q6k(const uint8_t *W, int nrows, const Q8Rows &x, int k, float *logits, unsigned long long *best,
                     hipStream_t st);
/* argmax keys of materialized logits [k][nrows] */
void launch_argmax_rows(const float *logits, int nrows, int k, unsigned long long *best, hipStream_t st);
/* keys -> row index and logit */
void launch_argmax_finish(const unsigned long long *best, int k, int32_t *idx, float *val, hipStream_t st);

}  // namespace tg
#endif
