// Matrix-vector products for up to 8 token rows: y[t][r] = act(scale * W[r] . x[t]) (+= y with
// mode 1). Replaces mv_f32, mv_bf16 and mv_q8 of shaders/engine/mv.hlsl:4-92,123-182 with the same
// constants (C): 0 w_srv, 1 w_off (bytes), 2 rows, 3 cols, 4 x_uav, 5 x_off, 6 x_stride,
// 7 n_tok, 8 y_uav, 9 y_off, 10 y_stride, 11 mode, 12 act, 13 scale (fp32 bits), 14 row_bytes,
// 15 rows_per_wave.
//
// The host sizes the grid as ceil(rows / (8 * rows_per_wave)) (src/gpu_engine.zig:851-853),
// i.e. for eight 32-lane waves per group. Here a group is four 64-lane waves; wave w covers the
// rows the reference gives to its waves 2w and 2w+1, so the grid covers the same rows.
#pragma once
#include "gd_kernel.h"

#define MV_MAX_TOK 8
#define MV_STAGED 16384

// Row formats: fp32; bf16; Q8_0 repacked as `cols` int8 quants followed by cols / 32 binary16
// scales (q8_repack), row_bytes = cols + cols / 16.
enum { MV_F32 = 0, MV_BF16 = 1, MV_Q8 = 2 };

template <int KIND>
__device__ __forceinline__ void mv_body(const GdArgs &a) {
    __shared__ float gx[MV_STAGED];
    const uint32_t rows = a.c[2], cols = a.c[3], n_tok = a.c[7] < MV_MAX_TOK ? a.c[7] : MV_MAX_TOK;
    const uint32_t x_off = a.c[5], x_stride = a.c[6], y_off = a.c[9], y_stride = a.c[10];
    const uint32_t mode = a.c[11], act = a.c[12], row_bytes = a.c[14], rpw = a.c[15];
    const float scale = gd_bits_f32(a.c[13]);
    const uint8_t *W = gd_buf<const uint8_t>(a, a.c[0]) + a.c[1];
    const float *X = gd_buf<const float>(a, a.c[4]);
    float *Y = gd_buf<float>(a, a.c[8]);
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;

    const bool staged = n_tok * cols <= MV_STAGED;
    if (staged) {
        for (uint32_t i = tid; i < n_tok * cols; i += 256u) {
            const uint32_t t = i / cols;
            gx[i] = X[x_off + t * x_stride + (i - t * cols)];
        }
        __syncthreads();
    }
    // Values per lane per step: 16 bytes of the row (a Q8 lane's 16 quants lie in one 32-block).
    constexpr uint32_t per = KIND == MV_Q8 ? 16u : KIND == MV_BF16 ? 8u : 4u;
    for (uint32_t half = 0; half < 2; ++half) {
        const uint32_t ref_wave = wave * 2u + half;
        for (uint32_t rr = 0; rr < rpw; ++rr) {
            const uint32_t row = (blockIdx.x * 8u + ref_wave) * rpw + rr;
            if (row >= rows) break;
            float acc[MV_MAX_TOK];
#pragma unroll
            for (int t = 0; t < MV_MAX_TOK; ++t) acc[t] = 0.f;
            const uint8_t *wr = W + (size_t)row * row_bytes;
            for (uint32_t c = lane * per; c < cols; c += 64u * per) {
                float v[per];
                if (KIND == MV_Q8) {
                    const uint4 raw = *reinterpret_cast<const uint4 *>(wr + c);
                    const float d = gd_half(*reinterpret_cast<const uint16_t *>(wr + cols + (c / 32u) * 2u));
                    const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j)
#pragma unroll
                        for (int b = 0; b < 4; ++b)
                            v[4 * j + b] = d * (float)((int32_t)(w4[j] << (24 - 8 * b)) >> 24);
                } else if (KIND == MV_BF16) {
                    const uint4 raw = *reinterpret_cast<const uint4 *>(wr + c * 2u);
                    const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        v[2 * j] = gd_bits_f32(w4[j] << 16);
                        v[2 * j + 1] = gd_bits_f32(w4[j] & 0xffff0000u);
                    }
                } else {
                    const float4 raw = *reinterpret_cast<const float4 *>(wr + c * 4u);
                    v[0] = raw.x; v[1] = raw.y; v[2] = raw.z; v[3] = raw.w;
                }
#pragma unroll
                for (int t = 0; t < MV_MAX_TOK; ++t) {
                    if ((uint32_t)t < n_tok) {
                        float s = 0.f;
#pragma unroll
                        for (uint32_t j = 0; j < per; ++j) {
                            const float xv = staged ? gx[t * cols + c + j] : X[x_off + t * x_stride + c + j];
                            s += v[j] * xv;
                        }
                        acc[t] += s;
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < MV_MAX_TOK; ++t) {
                if ((uint32_t)t < n_tok) {
                    const float total = gd_wave_sum(acc[t]);
                    if (lane == 0) {
                        const uint32_t idx = y_off + t * y_stride + row;
                        float v = total * scale;
                        if (act == 1u) v = gd_silu_accurate(v);
                        else if (act == 2u) v = gd_sigmoid_accurate(v);
                        if (mode == 1u) v += Y[idx];
                        Y[idx] = v;
                    }
                }
            }
        }
    }
}
