// Per token: softmax over the router logits, top-k of the probabilities (ties to the lower
// index), weights renormalised by their k-ordered sum clamped at 6.103515625e-5, then the
// optional expert_weights_scale. Replaces moe_route of shaders/engine/moe.hlsl:8-80; the CPU
// semantics are src/engine.zig:527-540 and :670-687. Grid: x = tokens; 256 threads (<= 512
// experts). Constants (RouteC): 0 logits_uav 1 logits_off 2 n_expert 3 n_used 4 ids_uav
// 5 ids_off 6 weights_uav 7 weights_off 8 host_uav (0xffffffff: none) 9 host_off
// 10 scale (fp32 bits) 11 n_tok.
#include "gd_kernel.h"

__device__ __forceinline__ void arg_better(float v, uint32_t i, float &bv, uint32_t &bi) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

GD_PIPELINE_NAMED(moe_route, 256) {
    __shared__ float p[512];
    __shared__ float red[4];
    __shared__ uint32_t redi[4];
    __shared__ float chosen[64];
    const uint32_t t = blockIdx.x, i = threadIdx.x, lane = i & 63u, wave = i >> 6;
    const uint32_t NE = a.c[2], U = a.c[3] < 64u ? a.c[3] : 64u;
    const float *L = gd_buf<const float>(a, a.c[0]) + a.c[1] + t * NE;
    const float v0 = i < NE ? L[i] : -INFINITY;
    const float v1 = i + 256u < NE ? L[i + 256u] : -INFINITY;
    float m = gd_wave_max(fmaxf(v0, v1));
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    const float e0 = i < NE ? expf(v0 - m) : 0.f;
    const float e1 = i + 256u < NE ? expf(v1 - m) : 0.f;
    float s = gd_wave_sum(e0 + e1);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    s = (red[0] + red[1]) + (red[2] + red[3]);
    p[i] = i < NE ? e0 / s : -1.f;
    p[i + 256u] = i + 256u < NE ? e1 / s : -1.f;
    __syncthreads();

    uint32_t *ids = gd_buf<uint32_t>(a, a.c[4]) + a.c[5] + t * a.c[3];
    float *weights = gd_buf<float>(a, a.c[6]) + a.c[7] + t * a.c[3];
    const bool host = a.c[8] != 0xffffffffu;
    float total = 0.f;
    for (uint32_t k = 0; k < U; ++k) {
        float bv = p[i];
        uint32_t bi = i;
        arg_better(p[i + 256u], i + 256u, bv, bi);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const uint32_t oi = (uint32_t)__shfl_xor((int)bi, o, 64);
            arg_better(ov, oi, bv, bi);
        }
        if (lane == 0) {
            red[wave] = bv;
            redi[wave] = bi;
        }
        __syncthreads();
        float gb = red[0];
        uint32_t gi = redi[0];
        for (uint32_t q = 1; q < 4; ++q) arg_better(red[q], redi[q], gb, gi);
        total += gb;
        if (i == 0) {
            ids[k] = gi;
            chosen[k] = gb;
            if (host) gd_buf<uint32_t>(a, a.c[8])[a.c[9] + t * a.c[3] + k] = gi;
        }
        __syncthreads();
        if (i == gi) p[i] = -1.f;
        if (i + 256u == gi) p[i + 256u] = -1.f;
        __syncthreads();
    }
    if (i < U) {
        const float scale = gd_bits_f32(a.c[10]);
        float w = chosen[i] / fmaxf(total, 6.103515625e-5f);
        if (scale != 0.f && scale != 1.f) w *= scale;
        weights[i] = w;
    }
}
