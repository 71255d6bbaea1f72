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
// Grid: (ceil(E / 1024), n); 256 threads, four columns per thread. Requires E % 4 == 0,
// n_used <= 16 and, with the shared expert, E <= 4096.
// Constants: 0 down32_uav 1 down32_off 2 weights_uav 3 weights_off 4 out_uav 5 out_off
// 6 E 7 n_used 8 residual (0: none, 1: add; zero when the caller passes 8 constants) 9 res_uav
// 10 res_off 11 shared (0: none, 1: add; zero when the caller passes 11 constants) 12 sh_uav
// 13 sh_off 14 x_uav 15 x_off (rows of E floats) 16 shared_gate_srv.
#include "gyro_fast.h"

#define CB_MAX_U 16
#define CB_MAX_E 4096  // with the shared expert

GD_PIPELINE_NAMED(moe_prefill_combine, 256) {
    __shared__ float part[4];
    const uint32_t E = a.c[6], U = a.c[7], t = blockIdx.y;
    const uint32_t c = (blockIdx.x * 256u + threadIdx.x) * 4u;
    float gate = 0.f;
    if (a.c[11]) {  // uniform
        const float *X = gd_buf<const float>(a, a.c[14]) + a.c[15] + (size_t)t * E;
        const float *G = gd_buf<const float>(a, a.c[16]);
        // Up to 4096 columns: all of a thread's loads in flight together, then the sum in order.
        gd_u32x4 xv[CB_MAX_E / 1024], gv[CB_MAX_E / 1024];
#pragma unroll
        for (int j = 0; j < CB_MAX_E / 1024; ++j) {
            const uint32_t i = threadIdx.x * 4u + 1024u * j;
            if (i < E) {
                xv[j] = *gd_global4(reinterpret_cast<const uint32_t *>(X + i));
                gv[j] = *gd_global4(reinterpret_cast<const uint32_t *>(G + i));
            }
        }
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < CB_MAX_E / 1024; ++j) {
            if (threadIdx.x * 4u + 1024u * j < E)
                s += gd_bits_f32(xv[j][0]) * gd_bits_f32(gv[j][0]) + gd_bits_f32(xv[j][1]) * gd_bits_f32(gv[j][1]) +
                     gd_bits_f32(xv[j][2]) * gd_bits_f32(gv[j][2]) + gd_bits_f32(xv[j][3]) * gd_bits_f32(gv[j][3]);
        }
        s = gd_wave_sum_dpp(s);
        if ((threadIdx.x & 63u) == 0u) part[threadIdx.x >> 6] = s;
        __syncthreads();
        gate = gd_sigmoid_accurate(((part[0] + part[1]) + part[2]) + part[3]);
    }
    if (c >= E) return;
    const uint32_t *D = gd_buf<const uint32_t>(a, a.c[0]) + a.c[1] + (size_t)t * U * E + c;
    cfloat *W = as_const(gd_buf<const float>(a, a.c[2]) + a.c[3] + t * U);
    // All n_used (<= 16) rows in flight together, then the k-ordered sum.
    gd_u32x4 dv[CB_MAX_U];
#pragma unroll
    for (int k = 0; k < CB_MAX_U; ++k)
        if ((uint32_t)k < U) dv[k] = *gd_global4(D + (size_t)k * E);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < CB_MAX_U; ++k) {
        if ((uint32_t)k < U) {
            const float w = W[k];
            acc.x += w * gd_bits_f32(dv[k][0]);
            acc.y += w * gd_bits_f32(dv[k][1]);
            acc.z += w * gd_bits_f32(dv[k][2]);
            acc.w += w * gd_bits_f32(dv[k][3]);
        }
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
