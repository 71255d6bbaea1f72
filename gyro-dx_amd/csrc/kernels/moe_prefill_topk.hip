// Prefill path, step 2: top-U routing of every token (U = n_used <= 16), one wave per token.
// Softmax, top-k with ties to the lower index, and the renormalised weights of
// src/engine.zig:527-540 and :670-687, computed on the logits as route_fast.h describes.
// The logits are the sum of S planes (the router's K split), added in plane order.
// Grid: ceil(n / 4); 256 threads (four tokens per group). Requires n_expert <= 256,
// 1 <= n_used <= 16.
// Constants: 0 logits_uav 1 logits_off 2 n_expert 3 n_tok 4 scale (fp32 bits) 5 ids_uav
// 6 ids_off 7 weights_uav 8 weights_off 9 S (0 or 1: one plane) 10 plane stride (floats)
// 11 n_used (0: 8, so that a caller passing 11 constants gets top-8) 12 hist_uav (0: none) 13 hist_off
// (words): every selected slot s = t n_used + k adds 1 to hist[s / 256][id] (device-scope
// atomics; the chunk histogram moe_prefill_sort places from, zeroed beforehand by the router).
#include "route_fast.h"

GD_PIPELINE_NAMED(moe_prefill_topk, 256) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t NE = a.c[2], n = a.c[3];
    const uint32_t t = blockIdx.x * 4u + wave;
    if (t >= n) return;
    const uint32_t S = a.c[9] > 1u ? a.c[9] : 1u;
    const float *lg = gd_buf<const float>(a, a.c[0]) + a.c[1] + (size_t)t * NE;
    float v[4];
    rf_load<4>(lg, NE, v);
    // Planes 1 .. 15 (the router's K split is at most 16): every load issued before the first
    // add, then the sum in plane order.
    float p[15][4];
#pragma unroll
    for (int z = 1; z < 16; ++z)
        if ((uint32_t)z < S) rf_load<4>(lg + (size_t)z * a.c[10], NE, p[z - 1]);
#pragma unroll
    for (int z = 1; z < 16; ++z)
        if ((uint32_t)z < S) {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] += p[z - 1][j];
        }
    for (uint32_t z = 16; z < S; ++z) {
        float q[4];
        rf_load<4>(lg + (size_t)z * a.c[10], NE, q);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] += q[j];
    }
    const uint32_t U = a.c[11] ? a.c[11] : 8u;  // uniform, <= 16
    uint32_t ids[16];
    float wts[16];
    if (U == 8u) {
        wave_route_fast<4, 8>(v, NE, gd_bits_f32(a.c[4]), ids, wts);
    } else {
        // Ranks 0 .. U - 1 in order, then the softmax over them in rank order (rf_weights).
        uint64_t key[4];
        rf_init<4>(v, NE, key);
        float top[16];
#pragma unroll
        for (int k = 0; k < 16; ++k)
            if ((uint32_t)k < U) ids[k] = rf_next<4>(key, top[k]);
        float total = 0.f;
#pragma unroll
        for (int k = 0; k < 16; ++k)
            if ((uint32_t)k < U) {
                wts[k] = expf(top[k] - top[0]);
                total += wts[k];
            }
        const float inv = 1.0f / total, scale = gd_bits_f32(a.c[4]);
#pragma unroll
        for (int k = 0; k < 16; ++k)
            if ((uint32_t)k < U) {
                float w = wts[k] * inv;
                if (scale != 0.f && scale != 1.f) w *= scale;
                wts[k] = w;
            }
    }
    if (lane < U) {
        uint32_t id = ids[0];
        float w = wts[0];
#pragma unroll
        for (int j = 1; j < 16; ++j) {
            if ((uint32_t)j >= U) break;
            id = lane == (uint32_t)j ? ids[j] : id;
            w = lane == (uint32_t)j ? wts[j] : w;
        }
        gd_buf<uint32_t>(a, a.c[5])[a.c[6] + t * U + lane] = id;
        gd_buf<float>(a, a.c[7])[a.c[8] + t * U + lane] = w;
        if (a.c[12]) {
            const uint32_t s = t * U + lane;
            __hip_atomic_fetch_add(gd_buf<uint32_t>(a, a.c[12]) + a.c[13] + (s >> 8) * NE + min(id, NE - 1u), 1u,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}
