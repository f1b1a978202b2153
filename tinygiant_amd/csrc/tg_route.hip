/*
 * tg_route.hip -- the MoE router on the device: per input row, logits over
 * the experts, the top-k experts by descending logit and their weights as a
 * softmax over the selected logits only (Router.logits/_topk/_weights,
 * tinygiant/router.py:29-42; selection without cache bias, router.py:62-63).
 *
 *   k_route_logits   one wave per (expert, input row): f32 router row . x_j
 *                    (+ bias), lanes accumulating in fixed order and a
 *                    fixed DPP tree
 *   k_route_topk     one wave per input row: top-k by repeated wave argmax
 *                    (larger logit first, lower expert index on equal
 *                    logits), then exp(l - max) / sum with the sum grouped
 *                    as numpy's float32 pairwise sum groups 8 values;
 *                    optionally restricted to a resident set of experts
 *                    (Router.select(restrict=True), router.py:46-54: the
 *                    others take -inf before the top-k, the weights come
 *                    from the same logits, and with fewer than k resident
 *                    experts the selection is unrestricted)
 */
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "tg_device.hpp"
#include "tg_route.h"

namespace tg {

/* logits[j][e] = router[e] . x_j (+ bias[e]); one wave per (expert, input
 * row) pair, so every row's logits are independent waves (k x n_experts of
 * them); lanes read 16-byte pieces of the two rows when they are 16-byte
 * aligned and dim a multiple of 256, and accumulate in a fixed order. */
__global__ __launch_bounds__(256) void k_route_logits(const float *__restrict__ router, const float *__restrict__ bias,
                                                      const float *__restrict__ x, int k, int n_experts, int dim,
                                                      int vec, float *logits) {
    const int lane = threadIdx.x & 63;
    const int p = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (p >= n_experts * k) return;   /* uniform per wave */
    const int e = p % n_experts, j = p / n_experts;
    const float *w = router + (size_t)e * dim;
    const float *xr = x + (size_t)j * dim;
    float acc = 0.f;
    if (vec) {
#pragma unroll 4
        for (int i = 4 * lane; i < dim; i += 256) {
            const float4 a = *reinterpret_cast<const float4 *>(w + i);
            const float4 b = *reinterpret_cast<const float4 *>(xr + i);
            acc = fmaf(a.x, b.x, acc);
            acc = fmaf(a.y, b.y, acc);
            acc = fmaf(a.z, b.z, acc);
            acc = fmaf(a.w, b.w, acc);
        }
    } else {
        for (int i = lane; i < dim; i += 64) acc = fmaf(w[i], xr[i], acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) logits[(size_t)j * n_experts + e] = bias ? acc + bias[e] : acc;
}

/* top-k + softmax over the selected, one wave per input row (k_top <= 64,
 * n_experts <= 256) */
__global__ __launch_bounds__(64) void k_route_topk(const float *__restrict__ logits, int n_experts, int k_top,
                                                   const uint8_t *__restrict__ resident, int32_t *idx_out,
                                                   float *w_out) {
    const int lane = threadIdx.x;
    const int j = blockIdx.x;
    const float *lg = logits + (size_t)j * n_experts;
    /* every load first (clamped indices, no branches), so the row costs one
     * memory latency */
    float lv[4];
    uint32_t rv[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int ec = min(lane + 64 * t, n_experts - 1);
        lv[t] = lg[ec];
        rv[t] = resident ? resident[ec] : 1u;
    }
    /* the mask applies only when at least k_top experts are resident */
    int cnt = 0;
#pragma unroll
    for (int t = 0; t < 4; t++) cnt += __popcll(__ballot(lane + 64 * t < n_experts && rv[t] != 0));
    const bool masked = resident != nullptr && cnt >= k_top;
    float v[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int e = lane + 64 * t;
        if (e >= n_experts) lv[t] = -INFINITY;
        v[t] = e < n_experts && (!masked || rv[t] != 0) ? lv[t] : -INFINITY;
    }
    /* top-k by repeated wave argmax: larger logit first, lower expert index
     * on equal logits; lane s keeps the s-th selected (its own, unmasked,
     * logit) */
    float sel_l = 0.f;
    int sel_e = 0;
    for (int s = 0; s < k_top; s++) {
        float bv = v[0];
        int be = lane;
#pragma unroll
        for (int t = 1; t < 4; t++)
            if (v[t] > bv) {
                bv = v[t];
                be = lane + 64 * t;
            }
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oe = __shfl_xor(be, o, 64);
            if (ov > bv || (ov == bv && oe < be)) {
                bv = ov;
                be = oe;
            }
        }
        float own = lv[0];
#pragma unroll
        for (int t = 1; t < 4; t++)
            if (t == (be >> 6)) own = lv[t];
        own = __shfl(own, be & 63, 64);
        if (lane == s) {
            sel_l = own;
            sel_e = be;
        }
        if ((be & 63) == lane) {
#pragma unroll
            for (int t = 0; t < 4; t++)
                if (t == (be >> 6)) v[t] = -INFINITY;
        }
    }
    /* softmax over the selected (descending order, so the max is the first) */
    const float mx = __shfl(sel_l, 0, 64);
    const float ex = lane < k_top ? expf(sel_l - mx) : 0.f;
    float sum;
    if (k_top >= 8) {
        /* numpy's pairwise float32 sum for 8 <= n <= 128: eight running sums
         * over whole groups of 8, ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)), then
         * the n % 8 leftovers one by one */
        float r[8];
#pragma unroll
        for (int q = 0; q < 8; q++) r[q] = __shfl(ex, q, 64);
        int i = 8;
        for (; i + 8 <= k_top; i += 8)
#pragma unroll
            for (int q = 0; q < 8; q++) r[q] += __shfl(ex, i + q, 64);
        sum = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        for (; i < k_top; i++) sum += __shfl(ex, i, 64);
    } else {
        sum = 0.f;
        for (int q = 0; q < k_top; q++) sum += __shfl(ex, q, 64);
    }
    if (lane < k_top) {
        idx_out[(size_t)j * k_top + lane] = sel_e;
        w_out[(size_t)j * k_top + lane] = ex / sum;
    }
}

void launch_route(const float *router, const float *bias, const float *x, int k, int n_experts, int dim, int k_top,
                  const uint8_t *resident, float *logits, int32_t *idx, float *w, hipStream_t st) {
    const int vec = dim % 256 == 0 && ((uintptr_t)router & 15) == 0 && ((uintptr_t)x & 15) == 0;
    hipLaunchKernelGGL(k_route_logits, dim3((n_experts * k + 3) / 4), dim3(256), 0, st, router, bias, x, k, n_experts,
                       dim, vec, logits);
    hipLaunchKernelGGL(k_route_topk, dim3(k), dim3(64), 0, st, logits, n_experts, k_top, resident, idx, w);
}

}  // namespace tg
