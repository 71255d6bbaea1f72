// Residual step and RMSNorm between the MoE layers of a stack (x <- x + MoE(RMSNorm(x)); rmsNorm
// of src/kernels.zig:281-291):
//   v     = x[t] + add[t]                (add: the previous layer's MoE output, when given)
//   xo[t] = v                            (when given: the residual stream after the add)
//   h[t]  = v / sqrt(mean(v^2) + eps) * w
// One group per token, 256 threads, up to 16 values per thread (E <= 4096). The sum of squares
// is reduced per wave with DPP, then over the four waves in order. xo may alias x: every
// load of a thread comes before its first store, so the loads need not wait for the stores.
// Grid: n tokens; 256 threads.
// Constants: 0 x_uav 1 x_off 2 add_uav (0xffffffff: none) 3 add_off 4 w_srv (0xffffffff: none)
// 5 w_off 6 h_uav 7 h_off 8 E 9 eps (fp32 bits) 10 xo_uav (0xffffffff: none) 11 xo_off.
#include "gd_kernel.h"

#define SN_PER 16

GD_PIPELINE_NAMED(moe_stack_norm, 256) {
    __shared__ float part[4];
    const uint32_t t = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t E = a.c[8];
    const size_t row = (size_t)t * E;
    const float *X = gd_buf<const float>(a, a.c[0]) + a.c[1] + row;
    const bool add = a.c[2] != 0xffffffffu, has_w = a.c[4] != 0xffffffffu, keep = a.c[10] != 0xffffffffu;
    const float *A = add ? gd_buf<const float>(a, a.c[2]) + a.c[3] + row : nullptr;
    float *XO = keep ? gd_buf<float>(a, a.c[10]) + a.c[11] + row : nullptr;
    float v[SN_PER];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < SN_PER; ++j) {
        const uint32_t i = tid + 256u * j;
        v[j] = 0.f;
        if (i < E) v[j] = add ? X[i] + A[i] : X[i];
    }
#pragma unroll
    for (int j = 0; j < SN_PER; ++j) ss += v[j] * v[j];
    if (keep) {
#pragma unroll
        for (int j = 0; j < SN_PER; ++j) {
            const uint32_t i = tid + 256u * j;
            if (i < E) XO[i] = v[j];
        }
    }
    // The norm weights are loaded before the barrier, so their latency overlaps it.
    float wv[SN_PER];
    const float *W = has_w ? gd_buf<const float>(a, a.c[4]) + a.c[5] : nullptr;
#pragma unroll
    for (int j = 0; j < SN_PER; ++j) {
        const uint32_t i = tid + 256u * j;
        wv[j] = has_w && i < E ? W[i] : 1.f;
    }
    ss = gd_wave_sum_dpp(ss);
    if (lane == 0) part[wave] = ss;
    __syncthreads();
    const float total = (part[0] + part[1]) + (part[2] + part[3]);
    const float scale = 1.0f / sqrtf(total / (float)E + gd_bits_f32(a.c[9]));
    float *H = gd_buf<float>(a, a.c[6]) + a.c[7] + row;
#pragma unroll
    for (int j = 0; j < SN_PER; ++j) {
        const uint32_t i = tid + 256u * j;
        if (i < E) H[i] = has_w ? v[j] * scale * wv[j] : v[j] * scale;
    }
}
