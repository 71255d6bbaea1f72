// Router logits and the rotated expert input for up to 8 tokens, one launch.
//   logits[t][r] = W_r[r] . x[t] (+ bias[r])          src/engine.zig:526 (kernels.matmul)
//   xh[t] = H_128 (gate_signs * x[t]) per 128-block    src/engine.zig:547-551
// Grid: x = max(n_expert, E / 128); 256 threads. Group r < n_expert computes router row r;
// groups r < E / 128 also rotate block r of every token (wave 0).
// Constants: 0 x_uav 1 x_off 2 x_stride 3 n_tok 4 router_srv 5 router_off 6 n_expert 7 E
// 8 bias_srv (0xffffffff: none) 9 bias_off 10 logits_uav 11 logits_off 12 signs_srv
// (0xffffffff: copy) 13 signs_off 14 xh_uav 15 xh_off.
#include "fwht.h"

#define ROUTER_MAX_TOK 8

GD_PIPELINE(256) {
    __shared__ float red[4][ROUTER_MAX_TOK];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, row = blockIdx.x;
    const uint32_t x_off = a.c[1], x_stride = a.c[2], E = a.c[7], NE = a.c[6];
    const uint32_t n_tok = a.c[3] < ROUTER_MAX_TOK ? a.c[3] : ROUTER_MAX_TOK;
    const float *X = gd_buf<const float>(a, a.c[0]);
    const float *W = gd_buf<const float>(a, a.c[4]) + a.c[5] + (size_t)row * E;
    float acc[ROUTER_MAX_TOK];
#pragma unroll
    for (int t = 0; t < ROUTER_MAX_TOK; ++t) acc[t] = 0.f;
    const uint32_t c_end = row < NE ? E : 0u;  // uniform per group
    for (uint32_t c = tid * 4u; c < c_end; c += 1024u) {
        const float4 w = *reinterpret_cast<const float4 *>(W + c);
#pragma unroll
        for (int t = 0; t < ROUTER_MAX_TOK; ++t) {
            if ((uint32_t)t < n_tok) {
                const float4 v = *reinterpret_cast<const float4 *>(X + x_off + t * x_stride + c);
                acc[t] += (w.x * v.x + w.y * v.y) + (w.z * v.z + w.w * v.w);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < ROUTER_MAX_TOK; ++t) {
        if ((uint32_t)t < n_tok) {
            const float s = gd_wave_sum(acc[t]);
            if (lane == 0) red[wave][t] = s;
        }
    }
    __syncthreads();
    if (tid < n_tok && row < NE) {
        float v = (red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid]);
        if (a.c[8] != 0xffffffffu) v += gd_buf<const float>(a, a.c[8])[a.c[9] + row];
        gd_buf<float>(a, a.c[10])[a.c[11] + tid * NE + row] = v;
    }
    if (wave == 0 && row < E / 128u) {
        const float *S = a.c[12] != 0xffffffffu ? gd_buf<const float>(a, a.c[12]) + a.c[13] : nullptr;
        float *XH = gd_buf<float>(a, a.c[14]) + a.c[15];
        const uint32_t i = row * 128u + 2u * lane;
        for (uint32_t t = 0; t < n_tok; ++t) {
            float x0 = X[x_off + t * x_stride + i], x1 = X[x_off + t * x_stride + i + 1u];
            if (S) {
                x0 *= S[i];
                x1 *= S[i + 1u];
                gd_fwht128_wave(x0, x1);
                x0 *= GD_INV_SQRT128;
                x1 *= GD_INV_SQRT128;
            }
            XH[t * E + i] = x0;
            XH[t * E + i + 1u] = x1;
        }
    }
}
