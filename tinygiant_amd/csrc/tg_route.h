/*
 * tg_route.h -- the device router (internal launch interface).
 */
#ifndef TG_ROUTE_H
#define TG_ROUTE_H
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tg {

/* logits [k][n_experts] (scratch), idx/w [k][k_top]; k_top <= 64,
 * n_experts <= 256; resident (may be NULL): one byte per expert, nonzero
 * for the experts the selection is restricted to */
void launch_route(const float *router, const float *bias, const float *x, int k, int n_experts, int dim, int k_top,
                  const uint8_t *resident, float *logits, int32_t *idx, float *w, hipStream_t st);

}  // namespace tg
#endif
