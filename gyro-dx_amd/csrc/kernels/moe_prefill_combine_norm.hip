// Prefill path inside a stack: the route-weighted combine of layer l (moe_prefill_combine, with
// the residual and, when given, the shared expert) and the RMSNorm of layer l + 1 (moe_stack_norm:
// rmsNorm of src/kernels.zig:281-291) in one launch, one group per token:
//   out[t] = res[t] + sum_k w[t][k] * down32[t * n_used + k] (+ sigmoid(g[t]) * sh[t])
//   h[t]   = out[t] / sqrt(mean(out[t]^2) + eps) * nw        (nw: the next layer's norm weight)
// Each column's sum is formed as moe_prefill_combine forms it, and the norm reduces the row as
// moe_stack_norm does (thread i of the first 256 sums columns i, i + 256, ... in that order, DPP
// wave sums, then (w0 + w1) + (w2 + w3)), so both outputs equal those of the two launches bit for
// bit. The row passes through LDS between the two orders. x (the gate-dot input) may alias h: a
// group reads its row of x before its first barrier and writes its row of h after its last.
// Grid: n tokens; 1024 threads, four columns per thread. Requires E % 4 == 0, E <= 4096,
// n_used <= 16.
// Constants: 0 down32_uav 1 down32_off 2 weights_uav 3 weights_off 4 out_uav 5 out_off 6 E
// 7 n_used 8 residual (0: none, 1: add) 9 res_uav 10 res_off 11 shared (0: none, 1: add)
// 12 sh_uav 13 sh_off 14 x_uav 15 x_off 16 shared_gate_srv (as moe_prefill_combine)
// 17 norm weight srv (0xffffffff: none) 18 h_uav 19 h_off 20 eps (fp32 bits).
#include "gyro_fast.h"

#define CN_MAX_U 16
#define CN_MAX_E 4096
#define CN_PER (CN_MAX_E / 256)

GD_PIPELINE_NAMED(moe_prefill_combine_norm, 1024) {
    __shared__ float part[4], npart[4];
    __shared__ float row[CN_MAX_E];
    const uint32_t E = a.c[6], U = a.c[7], t = blockIdx.x, tid = threadIdx.x;
    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const size_t ro = (size_t)t * E;
    const uint32_t c = tid * 4u;
    // The next layer's norm weights of this thread's columns, and, for the first 256 threads,
    // of the columns it reduces: loaded first, so their latency overlaps the combine.
    const bool has_w = a.c[17] != 0xffffffffu;
    const float *NW = has_w ? gd_buf<const float>(a, a.c[17]) : nullptr;
    float4 wv = make_float4(1.f, 1.f, 1.f, 1.f);
    if (has_w && c < E) wv = *reinterpret_cast<const float4 *>(NW + c);
    float gate = 0.f;
    if (a.c[11]) {  // the shared expert's gate, in moe_prefill_combine's order (threads 0..255)
        float s = 0.f;
        if (tid < 256u) {
            const float *X = gd_buf<const float>(a, a.c[14]) + a.c[15] + ro;
            const float *G = gd_buf<const float>(a, a.c[16]);
            gd_u32x4 xv[CN_MAX_E / 1024], gv[CN_MAX_E / 1024];
#pragma unroll
            for (int j = 0; j < CN_MAX_E / 1024; ++j) {
                const uint32_t i = tid * 4u + 1024u * j;
                if (i < E) {
                    xv[j] = *gd_global4(reinterpret_cast<const uint32_t *>(X + i));
                    gv[j] = *gd_global4(reinterpret_cast<const uint32_t *>(G + i));
                }
            }
#pragma unroll
            for (int j = 0; j < CN_MAX_E / 1024; ++j) {
                if (tid * 4u + 1024u * j < E)
                    s += gd_bits_f32(xv[j][0]) * gd_bits_f32(gv[j][0]) + gd_bits_f32(xv[j][1]) * gd_bits_f32(gv[j][1]) +
                         gd_bits_f32(xv[j][2]) * gd_bits_f32(gv[j][2]) + gd_bits_f32(xv[j][3]) * gd_bits_f32(gv[j][3]);
            }
            s = gd_wave_sum_dpp(s);
            if (lane == 0u) part[wave] = s;
        }
        __syncthreads();
        gate = gd_sigmoid_accurate(((part[0] + part[1]) + part[2]) + part[3]);
    }
    if (c < E) {
        const uint32_t *D = gd_buf<const uint32_t>(a, a.c[0]) + a.c[1] + (size_t)t * U * E + c;
        cfloat *W = as_const(gd_buf<const float>(a, a.c[2]) + a.c[3] + t * U);
        gd_u32x4 dv[CN_MAX_U];
#pragma unroll
        for (int k = 0; k < CN_MAX_U; ++k)
            if ((uint32_t)k < U) dv[k] = *gd_global4(D + (size_t)k * E);
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int k = 0; k < CN_MAX_U; ++k) {
            if ((uint32_t)k < U) {
                const float w = W[k];
                acc.x += w * gd_bits_f32(dv[k][0]);
                acc.y += w * gd_bits_f32(dv[k][1]);
                acc.z += w * gd_bits_f32(dv[k][2]);
                acc.w += w * gd_bits_f32(dv[k][3]);
            }
        }
        if (a.c[11]) {
            const float4 sh = *reinterpret_cast<const float4 *>(gd_buf<const float>(a, a.c[12]) + a.c[13] + ro + c);
            acc = make_float4(acc.x + gate * sh.x, acc.y + gate * sh.y, acc.z + gate * sh.z, acc.w + gate * sh.w);
        }
        if (a.c[8]) {
            const float4 r = *reinterpret_cast<const float4 *>(gd_buf<const float>(a, a.c[9]) + a.c[10] + ro + c);
            acc = make_float4(r.x + acc.x, r.y + acc.y, r.z + acc.z, r.w + acc.w);
        }
        *reinterpret_cast<float4 *>(gd_buf<float>(a, a.c[4]) + a.c[5] + ro + c) = acc;
        *reinterpret_cast<float4 *>(row + c) = acc;
    }
    __syncthreads();
    if (tid < 256u) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < CN_PER; ++j) {
            const uint32_t i = tid + 256u * j;
            const float v = i < E ? row[i] : 0.f;
            ss += v * v;
        }
        ss = gd_wave_sum_dpp(ss);
        if (lane == 0u) npart[wave] = ss;
    }
    __syncthreads();
    if (c >= E) return;
    const float total = (npart[0] + npart[1]) + (npart[2] + npart[3]);
    const float scale = 1.0f / sqrtf(total / (float)E + gd_bits_f32(a.c[20]));
    const float4 v = *reinterpret_cast<const float4 *>(row + c);
    float4 h;
    if (has_w)
        h = make_float4(v.x * scale * wv.x, v.y * scale * wv.y, v.z * scale * wv.z, v.w * scale * wv.w);
    else
        h = make_float4(v.x * scale, v.y * scale, v.z * scale, v.w * scale);
    *reinterpret_cast<float4 *>(gd_buf<float>(a, a.c[18]) + a.c[19] + ro + c) = h;
}
