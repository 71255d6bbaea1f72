// Top-k routing of one token by one wave64 without LDS traffic.
//
// Selection: the k largest router logits, ties to the lower index. Softmax is monotonic, so
// this is the top-k of the probabilities of src/engine.zig:527-540 and :670-687 except where
// two distinct logits round to the same probability (a sub-ulp near-tie). Each candidate is a
// 64-bit key (order-preserving logit bits << 32 | ~index); the wave maximum of the lane heads
// is found with DPP row shifts and row broadcasts and read from lane 63.
// Weights: w_k = exp(l_k - l_max) / sum_j exp(l_j - l_max) over the selected experts, which is
// p_k / sum_j p_j of the reference; its clamp at 6.103515625e-5 cannot bind because the top-k
// of at most 512 probabilities sum to at least k / 512.
#pragma once
#include "gd_kernel.h"


__device__ __forceinline__ uint32_t rf_order(float f) {
    const uint32_t u = gd_f32_bits(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float rf_unorder(uint32_t k) {
    return gd_bits_f32((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

template <int CTRL, int ROWS>
__device__ __forceinline__ uint64_t rf_step(uint64_t key) {
    const uint32_t hi = (uint32_t)(key >> 32), lo = (uint32_t)key;
    const uint64_t o = ((uint64_t)(uint32_t)__builtin_amdgcn_update_dpp(0, (int)hi, CTRL, ROWS, 0xf, true) << 32) |
                       (uint32_t)__builtin_amdgcn_update_dpp(0, (int)lo, CTRL, ROWS, 0xf, true);
    return o > key ? o : key;
}

// Wave maximum of 64-bit keys; every lane receives it (as a scalar).
__device__ __forceinline__ uint64_t rf_wave_max(uint64_t key) {
    key = rf_step<0x111, 0xf>(key);  // row_shr:1
    key = rf_step<0x112, 0xf>(key);  // row_shr:2
    key = rf_step<0x114, 0xf>(key);  // row_shr:4
    key = rf_step<0x118, 0xf>(key);  // row_shr:8  -> lane 15 of each row holds the row maximum
    key = rf_step<0x142, 0xa>(key);  // row_bcast:15 into rows 1 and 3
    key = rf_step<0x143, 0xc>(key);  // row_bcast:31 into rows 2 and 3 -> lane 63 holds the maximum
    return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(key >> 32), 63) << 32) |
           (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key, 63);
}

// Loads the lane's PER logits (n_expert <= 64 * PER) without branches; invalid slots get the
// key 0, below every real key.
template <int PER>
__device__ __forceinline__ void rf_load(const float *__restrict__ logits, uint32_t NE, float v[PER]) {
    const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const uint32_t i = lane + 64u * j;
        v[j] = logits[i < NE ? i : NE - 1u];
    }
}

// Top-U of the logits loaded by rf_load. Returns ids and weights (uniform across the wave).
// U is a compile-time count (the number of experts used per token).
template <int PER, int U>
__device__ __forceinline__ void wave_route_fast(const float v[PER], uint32_t NE, float scale, uint32_t ids[U],
                                                float wts[U]) {
    const uint32_t lane = threadIdx.x & 63u;
    uint64_t key[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const uint32_t i = lane + 64u * j;
        key[j] = i < NE ? ((uint64_t)rf_order(v[j]) << 32) | (uint32_t)~i : 0ull;
    }
    // Sort the lane's candidates in descending key order (insertion network).
#pragma unroll
    for (int a = 1; a < PER; ++a)
#pragma unroll
        for (int b = a; b > 0; --b) {
            const uint64_t hi = key[b] > key[b - 1] ? key[b] : key[b - 1];
            const uint64_t lo = key[b] > key[b - 1] ? key[b - 1] : key[b];
            key[b - 1] = hi;
            key[b] = lo;
        }
    float top[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
        const uint64_t m = rf_wave_max(key[0]);
        ids[k] = ~(uint32_t)m;
        top[k] = rf_unorder((uint32_t)(m >> 32));
        const bool mine = key[0] == m;
#pragma unroll
        for (int j = 0; j + 1 < PER; ++j) key[j] = mine ? key[j + 1] : key[j];
        key[PER - 1] = mine ? 0ull : key[PER - 1];
    }
    float total = 0.f;
#pragma unroll
    for (int k = 0; k < U; ++k) {
        wts[k] = expf(top[k] - top[0]);
        total += wts[k];
    }
    const float inv = 1.0f / total;
#pragma unroll
    for (int k = 0; k < U; ++k) {
        float w = wts[k] * inv;
        if (scale != 0.f && scale != 1.f) w *= scale;
        wts[k] = w;
    }
}
