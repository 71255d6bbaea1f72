// Prefill path, step 6: route-weighted combine of every token's n_used expert outputs,
// accumulated in k order from zero as src/engine.zig:634-642 does, plus the shared expert's
// gated output (src/engine.zig:644-653) when the layer has one.
//   out[t][c] = sum_k w[t][k] * down32[t * n_used + k][c]
//               (+ sigmoid(g[t]) * sh[t][c], g[t] = x[t] . shared_gate, when given)
//               (+ res[t][c] afterwards, when given: the residual step of a stack; res may
//               alias out)
// Every group of a token computes the gate dot over all of x[t] itself (fp32, a fixed order:
// four-element partials per thread, a wave tree, then the waves in order), so no group waits
// for another.
// Grid: (ceil(E / 1024), n); 256 threads, four columns per thread. Requires E % 4 == 0.
// Constants: 0 down32_uav 1 down32_off 2 weights_uav 3 weights_off 4 out_uav 5 out_off
// 6 E 7 n_used 8 residual (0: none, 1: add; zero when the caller passes 8 constants) 9 res_uav
// 10 res_off 11 shared (0: none, 1: add; zero when the caller passes 11 constants) 12 sh_uav
// 13 sh_off 14 x_uav 15 x_off (rows of E floats) 16 shared_gate_srv.
#include "gd_kernel.h"

GD_PIPELINE_NAMED(moe_prefill_combine, 256) {
    __shared__ float part[4];
    const uint32_t E = a.c[6], U = a.c[7], t = blockIdx.y;
    const uint32_t c = (blockIdx.x * 256u + threadIdx.x) * 4u;
    float gate = 0.f;
    if (a.c[11]) {  // uniform
        const float *X = gd_buf<const float>(a, a.c[14]) + a.c[15] + (size_t)t * E;
        const float *G = gd_buf<const float>(a, a.c[16]);
        float s = 0.f;
        for (uint32_t i = threadIdx.x * 4u; i < E; i += 1024u) {
            const float4 xv = *reinterpret_cast<const float4 *>(X + i);
            const float4 gv = *reinterpret_cast<const float4 *>(G + i);
            s += xv.x * gv.x + xv.y * gv.y + xv.z * gv.z + xv.w * gv.w;
        }
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) s += __shfl_xor(s, d, 64);
        if ((threadIdx.x & 63u) == 0u) part[threadIdx.x >> 6] = s;
        __syncthreads();
        gate = gd_sigmoid_accurate(((part[0] + part[1]) + part[2]) + part[3]);
    }
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
    if (a.c[11]) {
        const float4 sh = *reinterpret_cast<const float4 *>(gd_buf<const float>(a, a.c[12]) + a.c[13] + (size_t)t * E + c);
        acc = make_float4(acc.x + gate * sh.x, acc.y + gate * sh.y, acc.z + gate * sh.z, acc.w + gate * sh.w);
    }
    if (a.c[8]) {
        const float4 r = *reinterpret_cast<const float4 *>(gd_buf<const float>(a, a.c[9]) + a.c[10] + (size_t)t * E + c);
        acc = make_float4(r.x + acc.x, r.y + acc.y, r.z + acc.z, r.w + acc.w);
    }
    *reinterpret_cast<float4 *>(gd_buf<float>(a, a.c[4]) + a.c[5] + (size_t)t * E + c) = acc;
}
