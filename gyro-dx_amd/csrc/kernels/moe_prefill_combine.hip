// Prefill path, step 6: route-weighted combine of every token's n_used expert outputs,
// accumulated in k order from zero as src/engine.zig:634-642 does.
//   out[t][c] = sum_k w[t][k] * down32[t * n_used + k][c]  (+ res[t][c] afterwards, when given:
//   the residual step of a stack; res may alias out)
// Grid: (ceil(E / 1024), n); 256 threads, four columns per thread.
// Constants: 0 down32_uav 1 down32_off 2 weights_uav 3 weights_off 4 out_uav 5 out_off
// 6 E 7 n_used 8 residual (0: none, 1: add; zero when the caller passes 8 constants) 9 res_uav
// 10 res_off.
#include "gd_kernel.h"

GD_PIPELINE_NAMED(moe_prefill_combine, 256) {
    const uint32_t E = a.c[6], U = a.c[7], t = blockIdx.y;
    const uint32_t c = (blockIdx.x * 256u + threadIdx.x) * 4u;
    if (c >= E) return;
    const float *D = gd_buf<const float>(a, a.c[0]) + a.c[1] + (size_t)t * U * E + c;
    const float *W = gd_buf<const float>(a, a.c[2]) + a.c[3] + t * U;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (uint32_t k = 0; k < U; ++k) {
        const float w = W[k];
        const float4 d = *reinterpret_cast<const float4 *>(D + (size_t)k * E);
        acc.x += w * d.x;
        acc.y += w * d.y;
        acc.z += w * d.z;
        acc.w += w * d.w;
    }
    if (a.c[8]) {
        const float4 r = *reinterpret_cast<const float4 *>(gd_buf<const float>(a, a.c[9]) + a.c[10] + (size_t)t * E + c);
        acc = make_float4(r.x + acc.x, r.y + acc.y, r.z + acc.z, r.w + acc.w);
    }
    *reinterpret_cast<float4 *>(gd_buf<float>(a, a.c[4]) + a.c[5] + (size_t)t * E + c) = acc;
}
