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

#define RF_MAX_USED 16

__device__ __forceinline__ uint32_t rf_order(float f) {
    const uint32_t u = gd_f32_bits(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float rf_unorder(uint32_t k) {
    return gd_bits_f32((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

template <int CTRL, int ROWS>
__device__ __forceinline__ void rf_step(uint32_t &hi, uint32_t &lo) {
    const uint32_t ohi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hi, CTRL, ROWS, 0xf, true);
    const uint32_t olo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)lo, CTRL, ROWS, 0xf, true);
    const bool take = ohi > hi || (ohi == hi && olo > lo);
    hi = take ? ohi : hi;
    lo = take ? olo : lo;
}

// Wave maximum of 64-bit keys; every lane receives it (as scalars).
__device__ __forceinline__ void rf_wave_max(uint32_t hi, uint32_t lo, uint32_t &mhi, uint32_t &mlo) {
    rf_step<0x111, 0xf>(hi, lo);  // row_shr:1
    rf_step<0x112, 0xf>(hi, lo);  // row_shr:2
    rf_step<0x114, 0xf>(hi, lo);  // row_shr:4
    rf_step<0x118, 0xf>(hi, lo);  // row_shr:8  -> lane 15 of each row holds the row maximum
    rf_step<0x142, 0xa>(hi, lo);  // row_bcast:15 into rows 1 and 3
    rf_step<0x143, 0xc>(hi, lo);  // row_bcast:31 into rows 2 and 3 -> lane 63 holds the maximum
    mhi = __builtin_amdgcn_readlane(hi, 63);
    mlo = __builtin_amdgcn_readlane(lo, 63);
}

// logits: the token's n_expert (<= 256 * PER / 4 ... <= 64 * PER) values. Returns ids and
// weights (uniform across the wave).
template <int PER>
__device__ __forceinline__ void wave_route_fast(const float *__restrict__ logits, uint32_t NE, uint32_t U, float scale,
                                                uint32_t ids[RF_MAX_USED], float wts[RF_MAX_USED]) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t khi[PER], klo[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const uint32_t i = lane + 64u * j;
        khi[j] = i < NE ? rf_order(logits[i]) : 0u;
        klo[j] = i < NE ? ~i : 0u;
    }
    // Sort the lane's candidates in descending key order (insertion network).
#pragma unroll
    for (int a = 1; a < PER; ++a)
#pragma unroll
        for (int b = a; b > 0; --b) {
            const bool sw = khi[b] > khi[b - 1] || (khi[b] == khi[b - 1] && klo[b] > klo[b - 1]);
            const uint32_t th = khi[b], tl = klo[b];
            khi[b] = sw ? khi[b - 1] : khi[b];
            klo[b] = sw ? klo[b - 1] : klo[b];
            khi[b - 1] = sw ? th : khi[b - 1];
            klo[b - 1] = sw ? tl : klo[b - 1];
        }
    float top[RF_MAX_USED];
    for (uint32_t k = 0; k < U; ++k) {
        uint32_t mhi, mlo;
        rf_wave_max(khi[0], klo[0], mhi, mlo);
        ids[k] = ~mlo;
        top[k] = rf_unorder(mhi);
        const bool mine = khi[0] == mhi && klo[0] == mlo;
#pragma unroll
        for (int j = 0; j + 1 < PER; ++j) {
            khi[j] = mine ? khi[j + 1] : khi[j];
            klo[j] = mine ? klo[j + 1] : klo[j];
        }
        khi[PER - 1] = mine ? 0u : khi[PER - 1];
        klo[PER - 1] = mine ? 0u : klo[PER - 1];
    }
    float total = 0.f;
    for (uint32_t k = 0; k < U; ++k) {
        wts[k] = expf(top[k] - top[0]);
        total += wts[k];
    }
    for (uint32_t k = 0; k < U; ++k) {
        float w = wts[k] / total;
        if (scale != 0.f && scale != 1.f) w *= scale;
        wts[k] = w;
    }
}
