// Top-k routing of one token by one wave64 without LDS traffic.
//
// Selection: the k largest router logits, ties to the lower index. Softmax is monotonic, so
// this is the top-k of the probabilities of src/engine.zig:527-540 and :670-687 except where
// two distinct logits round to the same probability (a sub-ulp near-tie). Each lane holds its
// candidates sorted by (order-preserving logit bits, lower index first); a round takes the wave
// maximum of the lanes' head bits (32-bit DPP row shifts and row broadcasts, read from lane 63),
// the ballot of the lanes whose head holds it, and the winner's index from the single such lane,
// or on an exact tie the smallest index among them (a second, 32-bit minimum).
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

// Loads the lane's PER logits (n_expert <= 64 * PER) without branches; invalid slots get the
// key 0, below every real key.
template <int PER>
__device__ __forceinline__ void rf_load(const float *__restrict__ logits, uint32_t NE, float v[PER]) {
    const uint32_t lane = threadIdx.x & 63u;
    gd_guint *g = gd_global(reinterpret_cast<const uint32_t *>(logits));  // global_load: no LDS aliasing
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const uint32_t i = lane + 64u * j;
        v[j] = gd_bits_f32(g[i < NE ? i : NE - 1u]);
    }
}

// Wave maximum (MAX) or minimum of 32-bit values; every lane receives it (as a scalar). Lanes
// outside a DPP source range or row mask contribute the operation's identity.
template <int CTRL, int ROWS, bool MAX>
__device__ __forceinline__ uint32_t rf_step32(uint32_t v) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(MAX ? 0 : -1, (int)v, CTRL, ROWS, 0xf, false);
    return MAX ? (o > v ? o : v) : (o < v ? o : v);
}
template <bool MAX>
__device__ __forceinline__ uint32_t rf_wave_reduce32(uint32_t v) {
    v = rf_step32<0x111, 0xf, MAX>(v);  // row_shr:1
    v = rf_step32<0x112, 0xf, MAX>(v);  // row_shr:2
    v = rf_step32<0x114, 0xf, MAX>(v);  // row_shr:4
    v = rf_step32<0x118, 0xf, MAX>(v);  // row_shr:8  -> lane 15 of each row holds the row result
    v = rf_step32<0x142, 0xa, MAX>(v);  // row_bcast:15 into rows 1 and 3
    v = rf_step32<0x143, 0xc, MAX>(v);  // row_bcast:31 into rows 2 and 3 -> lane 63 holds the result
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Round-by-round form of the selection, for callers that need only the first ranks (a decode
// group needs the expert of its own slot, rank k) or want to overlap the weights with loads.
// rf_init: the lane's candidate keys (logit order << 32 | ~index, 0 past NE), sorted.
template <int PER>
__device__ __forceinline__ void rf_init(const float v[PER], uint32_t NE, uint64_t key[PER]) {
    const uint32_t lane = threadIdx.x & 63u;
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
}

// rf_next: the next rank's expert id (uniform) and its logit; removes it from the candidates.
template <int PER>
__device__ __forceinline__ uint32_t rf_next(uint64_t key[PER], float &logit) {
    const uint32_t h = (uint32_t)(key[0] >> 32), my = ~(uint32_t)key[0];
    const uint32_t m = rf_wave_reduce32<true>(h);
    const uint64_t at_max = __ballot(h == m);
    uint32_t id;
    if (__builtin_popcountll(at_max) == 1) id = (uint32_t)__builtin_amdgcn_readlane((int)my, (int)__builtin_ctzll(at_max));
    else id = rf_wave_reduce32<false>(h == m ? my : 0xffffffffu);
    logit = rf_unorder(m);
    const bool mine = my == id;
#pragma unroll
    for (int j = 0; j + 1 < PER; ++j) key[j] = mine ? key[j + 1] : key[j];
    key[PER - 1] = mine ? 0ull : key[PER - 1];
    return id;
}

// rf_weights: w_k = exp(l_k - l_0) / sum_j exp(l_j - l_0) over the selected logits (descending),
// times the layer's scale unless it is 0 or 1.
template <int U>
__device__ __forceinline__ void rf_weights(const float top[U], float scale, float wts[U]) {
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

// Top-U of the logits loaded by rf_load. Returns ids and weights (uniform across the wave).
// U is a compile-time count (the number of experts used per token).
template <int PER, int U>
__device__ __forceinline__ void wave_route_fast(const float v[PER], uint32_t NE, float scale, uint32_t ids[U],
                                                float wts[U]) {
    uint64_t key[PER];
    rf_init<PER>(v, NE, key);
    float top[U];
#pragma unroll
    for (int k = 0; k < U; ++k) ids[k] = rf_next<PER>(key, top[k]);
    rf_weights<U>(top, scale, wts);
}
