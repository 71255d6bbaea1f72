// Softmax and top-k routing of one token by one wave64, restating src/engine.zig:527-540 and
// topK (:670-687): probabilities, the k largest in descending order with ties to the lower
// index, weights divided by their k-ordered sum clamped at 6.103515625e-5, then the optional
// expert_weights_scale. Every lane ends with the same ids and weights.
#pragma once
#include "gd_kernel.h"

#define ROUTE_MAX_EXPERTS 512
#define ROUTE_MAX_USED 16

__device__ __forceinline__ void route_better(float v, uint32_t i, float &bv, uint32_t &bi) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

__device__ __forceinline__ void wave_route(const float *__restrict__ logits, uint32_t NE, uint32_t U,
                                           float scale, uint32_t ids[ROUTE_MAX_USED],
                                           float wts[ROUTE_MAX_USED]) {
    const uint32_t lane = threadIdx.x & 63u;
    float p[8];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t i = lane + 64u * j;
        p[j] = i < NE ? logits[i] : -INFINITY;
        m = fmaxf(m, p[j]);
    }
    m = gd_wave_max(m);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t i = lane + 64u * j;
        p[j] = i < NE ? expf(p[j] - m) : 0.f;
        s += p[j];
    }
    s = gd_wave_sum(s);
#pragma unroll
    for (int j = 0; j < 8; ++j) p[j] = lane + 64u * j < NE ? p[j] / s : -1.f;
    float total = 0.f;
    for (uint32_t k = 0; k < U; ++k) {
        float bv = p[0];
        uint32_t bi = lane;
#pragma unroll
        for (int j = 1; j < 8; ++j)
            if (p[j] > bv) {  // indices ascend with j: strict > keeps the lower index on ties
                bv = p[j];
                bi = lane + 64u * j;
            }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const uint32_t oi = (uint32_t)__shfl_xor((int)bi, o, 64);
            route_better(ov, oi, bv, bi);
        }
        ids[k] = bi;
        wts[k] = bv;
        total += bv;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (lane + 64u * j == bi) p[j] = -1.f;
    }
    const float denom = fmaxf(total, 6.103515625e-5f);
    for (uint32_t k = 0; k < U; ++k) {
        float w = wts[k] / denom;
        if (scale != 0.f && scale != 1.f) w *= scale;
        wts[k] = w;
    }
}
