// Decode path, step 1: router logits and the rotated expert input for up to 8 tokens.
//   logits[t][r] = W_r[r] . x[t] (+ bias[r])          src/engine.zig:526 (kernels.matmul)
//   xh[t] = H_128 (gate_signs * x[t]) per 128-block    src/engine.zig:547-551
// The rotated input is written as binary16 pairs (xh16[t][i/2] = x[i] | x[i+1] << 16), the
// form the gate/up kernel keeps in scalar registers; |xh| must stay below 65504.
// Grid: x = max(n_expert, E / 128); 256 threads. Group r < n_expert computes router row r;
// groups r < E / 128 also rotate block r of every token (wave 0).
// Constants: 0 x_uav 1 x_off 2 x_stride 3 n_tok 4 router_srv 5 router_off 6 n_expert 7 E
// 8 bias_srv (0xffffffff: none) 9 bias_off 10 logits_uav 11 logits_off 12 signs_srv
// (0xffffffff: copy) 13 signs_off 14 xh16_uav 15 xh16_off (words).
#include "fwht.h"

#define ROUTER_MAX_TOK 8
#define ROUTER_MAX_E 4096

GD_PIPELINE_NAMED(moe_router, 256) {
    __shared__ float red[4][ROUTER_MAX_TOK];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, row = blockIdx.x;
    const uint32_t x_off = a.c[1], x_stride = a.c[2], E = a.c[7], NE = a.c[6];
    const uint32_t n_tok = a.c[3] < ROUTER_MAX_TOK ? a.c[3] : ROUTER_MAX_TOK;
    const float *X = gd_buf<const float>(a, a.c[0]);
    const bool rotate_here = wave == 0 && row < E / 128u;

    // Rotation inputs first (independent of the router row).
    float rx[ROUTER_MAX_TOK][2], rs[2] = {1.f, 1.f};
    const uint32_t ri = row * 128u + 2u * lane;
    const bool has_signs = a.c[12] != 0xffffffffu;
    if (rotate_here) {
        if (has_signs) {
            const float2 sv = *reinterpret_cast<const float2 *>(gd_buf<const float>(a, a.c[12]) + a.c[13] + ri);
            rs[0] = sv.x;
            rs[1] = sv.y;
        }
#pragma unroll
        for (int t = 0; t < ROUTER_MAX_TOK; ++t)
            if ((uint32_t)t < n_tok) {
                const float2 xv = *reinterpret_cast<const float2 *>(X + x_off + t * x_stride + ri);
                rx[t][0] = xv.x;
                rx[t][1] = xv.y;
            }
    }
    if (row < NE) {  // uniform per group
        const float *W = gd_buf<const float>(a, a.c[4]) + a.c[5] + (size_t)row * E;
        constexpr int PER = ROUTER_MAX_E / 1024;
        float4 w[PER];
#pragma unroll
        for (int j = 0; j < PER; ++j)
            if (tid * 4u + 1024u * j < E) w[j] = *reinterpret_cast<const float4 *>(W + tid * 4u + 1024u * j);
#pragma unroll
        for (int t = 0; t < ROUTER_MAX_TOK; ++t) {
            if ((uint32_t)t < n_tok) {
                float acc = 0.f;
#pragma unroll
                for (int j = 0; j < PER; ++j)
                    if (tid * 4u + 1024u * j < E) {
                        const float4 v = *reinterpret_cast<const float4 *>(X + x_off + t * x_stride + tid * 4u + 1024u * j);
                        acc += (w[j].x * v.x + w[j].y * v.y) + (w[j].z * v.z + w[j].w * v.w);
                    }
                const float s = gd_wave_sum(acc);
                if (lane == 0) red[wave][t] = s;
            }
        }
    }
    __syncthreads();
    if (tid < n_tok && row < NE) {
        float v = (red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid]);
        if (a.c[8] != 0xffffffffu) v += gd_buf<const float>(a, a.c[8])[a.c[9] + row];
        gd_buf<float>(a, a.c[10])[a.c[11] + tid * NE + row] = v;
    }
    if (rotate_here) {
        uint32_t *XH = gd_buf<uint32_t>(a, a.c[14]) + a.c[15];
#pragma unroll
        for (int t = 0; t < ROUTER_MAX_TOK; ++t) {
            if ((uint32_t)t >= n_tok) break;
            float x0 = rx[t][0], x1 = rx[t][1];
            if (has_signs) {
                x0 *= rs[0];
                x1 *= rs[1];
                gd_fwht128_wave(x0, x1);
                x0 *= GD_INV_SQRT128;
                x1 *= GD_INV_SQRT128;
            }
            const uint32_t h0 = __builtin_bit_cast(uint16_t, (_Float16)x0);
            const uint32_t h1 = __builtin_bit_cast(uint16_t, (_Float16)x1);
            XH[t * (E / 2u) + row * 64u + lane] = h0 | (h1 << 16);
        }
    }
}
