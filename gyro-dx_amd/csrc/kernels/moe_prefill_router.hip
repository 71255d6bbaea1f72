// Prefill path, step 1: router logits of many tokens on fp32 MFMA, and the rotated expert
// input in binary16.
//   logits[t][r] = W_r[r] . x[t] (+ bias[r])          src/engine.zig:526 (kernels.matmul)
//   xh16[t]      = H_128 (gate_signs * x[t]) per 128-block, as binary16 pairs
//                                                      src/engine.zig:547-551
// Group (bx, by) computes the 32 x 32 logit tile of tokens 32 bx.. and experts 32 by.. with
// v_mfma_f32_32x32x2_f32; its eight waves split K = E into eighths and their partial tiles
// are added in wave order through LDS. Each lane half feeds four consecutive k per 16-byte
// load (lane half h takes k + 4h .. k + 4h + 3 of every 8), the same k for A and B, so every
// product x[t][k] W[r][k] enters the sum once. The rotation of all n * E/128 blocks is spread
// over every wave of the grid, one block per wave at a time.
// Grid: (ceil(n / 32), ceil(n_expert / 32)); 512 threads. Requires E % 128 == 0.
// Constants: 0 x_uav 1 x_off (words; rows of E floats) 2 n_tok 3 E 4 router_srv 5 router_off
// 6 n_expert 7 bias_srv (0xffffffff: none) 8 bias_off 9 logits_uav 10 logits_off
// 11 signs_srv (0xffffffff: no rotation, plain conversion) 12 signs_off 13 xh16_uav
// 14 xh16_off (words).
#include "fwht.h"

typedef float f32x16 __attribute__((ext_vector_type(16)));

GD_PIPELINE_NAMED(moe_prefill_router, 512) {
    __shared__ float red[8][32 * 32];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t n = a.c[2], E = a.c[3], NE = a.c[6];
    const float *X = gd_buf<const float>(a, a.c[0]) + a.c[1];

    // Rotation share of this group.
    {
        const uint32_t nblk = E / 128u, total = n * nblk;
        const uint32_t waves = gridDim.x * gridDim.y * 8u;
        const uint32_t first = (blockIdx.y * gridDim.x + blockIdx.x) * 8u + wave;
        const bool has_signs = a.c[11] != 0xffffffffu;
        const float *S = has_signs ? gd_buf<const float>(a, a.c[11]) + a.c[12] : nullptr;
        uint32_t *XH = gd_buf<uint32_t>(a, a.c[13]) + a.c[14];
        for (uint32_t b = first; b < total; b += waves) {
            const uint32_t t = b / nblk, blk = b - t * nblk, i = blk * 128u + 2u * lane;
            const float2 xv = *reinterpret_cast<const float2 *>(X + (size_t)t * E + i);
            float x0 = xv.x, x1 = xv.y;
            if (has_signs) {
                const float2 sv = *reinterpret_cast<const float2 *>(S + i);
                x0 *= sv.x;
                x1 *= sv.y;
                gd_fwht128_wave(x0, x1);
                x0 *= GD_INV_SQRT128;
                x1 *= GD_INV_SQRT128;
            }
            const uint32_t h0 = __builtin_bit_cast(uint16_t, (_Float16)x0);
            const uint32_t h1 = __builtin_bit_cast(uint16_t, (_Float16)x1);
            XH[(size_t)t * (E / 2u) + blk * 64u + lane] = h0 | (h1 << 16);
        }
    }

    // Router tile.
    const uint32_t t0 = blockIdx.x * 32u, r0 = blockIdx.y * 32u;
    const uint32_t m = lane & 31u, h = lane >> 5;
    const bool tv = t0 + m < n, rv = r0 + m < NE;
    const float *xa = X + (size_t)(tv ? t0 + m : 0u) * E + 4u * h;
    const float *wb = gd_buf<const float>(a, a.c[4]) + a.c[5] + (size_t)(rv ? r0 + m : 0u) * E + 4u * h;
    const uint32_t kpw = E / 8u, k0 = wave * kpw;
    f32x16 acc = {};
#pragma unroll 4
    for (uint32_t k = k0; k < k0 + kpw; k += 8u) {
        float4 av = *reinterpret_cast<const float4 *>(xa + k);
        float4 bv = *reinterpret_cast<const float4 *>(wb + k);
        if (!tv) av = make_float4(0.f, 0.f, 0.f, 0.f);
        if (!rv) bv = make_float4(0.f, 0.f, 0.f, 0.f);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, bv.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, bv.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, bv.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, bv.w, acc, 0, 0, 0);
    }
    // Accumulator register r holds tile row 8 (r / 4) + 4 h + r % 4, column m.
#pragma unroll
    for (int r = 0; r < 16; ++r) red[wave][((r / 4) * 8 + h * 4 + (r % 4)) * 32 + m] = acc[r];
    __syncthreads();
    const bool has_bias = a.c[7] != 0xffffffffu;
    float *L = gd_buf<float>(a, a.c[9]) + a.c[10];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint32_t idx = tid + 512u * q, i = idx >> 5, j = idx & 31u;
        const uint32_t t = t0 + i, r = r0 + j;
        if (t < n && r < NE) {
            float v = red[0][idx];
#pragma unroll
            for (int w = 1; w < 8; ++w) v += red[w][idx];
            if (has_bias) v += gd_buf<const float>(a, a.c[7])[a.c[8] + r];
            L[(size_t)t * NE + r] = v;
        }
    }
}
