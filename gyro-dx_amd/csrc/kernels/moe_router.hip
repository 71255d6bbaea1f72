// Decode path, step 1: router logits and the rotated expert input for up to 8 tokens.
//   logits[t][r] = W_r[r] . x[t] (+ bias[r])          src/engine.zig:526 (kernels.matmul)
//   xh[t] = H_128 (gate_signs * x[t]) per 128-block    src/engine.zig:547-551
// Optionally the layer input is first normalised as in a stack (rmsNorm, src/kernels.zig:281-291):
// x[t] is replaced by h[t] = x[t] * s[t] * w with s[t] = 1 / sqrt(mean(x[t]^2) + eps). Every
// group accumulates mean(x[t]^2) beside its dot product from the same loads; the logit is then
// s[t] * ((W_r[r] * w) . x[t]).
// The rotated input is written as binary16 pairs (xh16[t][i/2] = x[i] | x[i+1] << 16), the
// form the gate/up kernel keeps in scalar registers; |xh| must stay below 65504.
// Grid: x = max(n_expert, E / 128); 256 threads. Group r < n_expert computes router row r;
// groups r < E / 128 also rotate block r of every token (wave 0).
// Constants: 0 x_uav 1 x_off 2 x_stride 3 n_tok 4 router_srv 5 router_off 6 n_expert 7 E
// 8 bias_srv (0xffffffff: none) 9 bias_off 10 logits_uav 11 logits_off 12 signs_srv
// (0xffffffff: copy) 13 signs_off 14 xh16_uav 15 xh16_off (words) 16 norm (0: none, 1: RMSNorm
// without weight, 2: with weight; zero when the caller passes 16 constants) 17 norm_w_srv
// 18 norm_w_off 19 eps (fp32 bits) 20 shared rows (2 SF; 0: no shared expert) 21 sh_w_srv (bf16
// [2 SF][E]: gate rows then up rows) 22 sh_h_uav (fp32 [n][2 SF]) 23 sh_gate_srv (fp32 [E])
// 24 sh_g_uav (fp32 [n]). With a shared expert (src/engine.zig:644-653) the grid has 2 SF / 16 + 1
// further groups after the max(n_expert, E / 128) above: each of the first computes 16 bf16 rows
// (4 per wave) of W_sg x and W_su x on the unrotated input, the last the gate dot g . x. The
// shared groups require E <= 2048.
#include "fwht.h"

#define ROUTER_MAX_TOK 8
#define ROUTER_MAX_E 4096

#define SH_ROWS_PER_GROUP 16
#define SH_MAX_E 2048  // hidden width covered by the fused shared-expert rows

// Shared expert rows of group sg: wave w takes rows 16 sg + 4 w .. + 3 of W_sh (bf16, E columns);
// lane l covers columns 8 l + 512 m (m < E / 512) of every row.
__device__ __forceinline__ void router_shared_rows(const GdArgs &a, uint32_t sg, uint32_t n_tok, uint32_t E) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t rows = a.c[20], r0 = sg * SH_ROWS_PER_GROUP + wave * 4u;
    const uint16_t *Wsh = gd_buf<const uint16_t>(a, a.c[21]);
    const float *X = gd_buf<const float>(a, a.c[0]);
    float *H = gd_buf<float>(a, a.c[22]);
    constexpr int MM = SH_MAX_E / 512;  // column chunks
    uint4 w[4][MM];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int m = 0; m < MM; ++m)
            if (r0 + (uint32_t)i < rows && 512u * m < E)
                w[i][m] = *reinterpret_cast<const uint4 *>(Wsh + (size_t)(r0 + i) * E + 8u * lane + 512u * m);
    for (uint32_t t = 0; t < n_tok; ++t) {
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            if (512u * m >= E) break;
            const float4 *xp = reinterpret_cast<const float4 *>(X + a.c[1] + t * a.c[2] + 8u * lane + 512u * m);
            const float4 x0 = xp[0], x1 = xp[1];
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t ww[4] = {w[i][m].x, w[i][m].y, w[i][m].z, w[i][m].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    acc[i] += gd_bits_f32(ww[q] << 16) * xv[2 * q];
                    acc[i] += gd_bits_f32(ww[q] & 0xffff0000u) * xv[2 * q + 1];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float v = gd_wave_sum(acc[i]);
            if (lane == 0 && r0 + (uint32_t)i < rows) H[t * rows + r0 + i] = v;
        }
    }
}

GD_PIPELINE_NAMED(moe_router, 256) {
    __shared__ float red[4][ROUTER_MAX_TOK], reds[4][ROUTER_MAX_TOK];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, row = blockIdx.x;
    const uint32_t x_off = a.c[1], x_stride = a.c[2], E = a.c[7], NE = a.c[6];
    const uint32_t n_tok = a.c[3] < ROUTER_MAX_TOK ? a.c[3] : ROUTER_MAX_TOK;
    const uint32_t norm = a.c[16];
    const float *X = gd_buf<const float>(a, a.c[0]);
    {
        // Shared-expert groups follow the router and rotation groups (uniform per group).
        const uint32_t first_sh = max(NE, E / 128u);
        if (a.c[20] && row >= first_sh) {
            const uint32_t sg = row - first_sh, n_sg = a.c[20] / SH_ROWS_PER_GROUP;
            if (sg < n_sg) {
                router_shared_rows(a, sg, n_tok, E);
            } else {
                // The gate dot g . x (fp32 row), one wave per token.
                const float *G = gd_buf<const float>(a, a.c[23]);
                for (uint32_t t = wave; t < n_tok; t += 4u) {
                    float acc = 0.f;
                    for (uint32_t i = lane; i < E; i += 64u) acc += G[i] * X[x_off + t * x_stride + i];
                    acc = gd_wave_sum(acc);
                    if (lane == 0) gd_buf<float>(a, a.c[24])[t] = acc;
                }
            }
            return;
        }
    }
    const float *NW = norm == 2u ? gd_buf<const float>(a, a.c[17]) + a.c[18] : nullptr;
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
        if (norm == 2u) {
            const float2 nv = *reinterpret_cast<const float2 *>(NW + ri);
            rs[0] *= nv.x;
            rs[1] *= nv.y;
        }
#pragma unroll
        for (int t = 0; t < ROUTER_MAX_TOK; ++t)
            if ((uint32_t)t < n_tok) {
                const float2 xv = *reinterpret_cast<const float2 *>(X + x_off + t * x_stride + ri);
                rx[t][0] = xv.x;
                rx[t][1] = xv.y;
            }
    }
    // Groups with a router row compute its dot products; with the norm, every group that has a
    // router row or a rotation block also needs the tokens' sums of squares.
    const bool dot = row < NE;  // uniform per group
    if (dot || (norm && row < E / 128u)) {
        const float *W = gd_buf<const float>(a, a.c[4]) + a.c[5] + (size_t)(dot ? row : 0u) * E;
        constexpr int PER = ROUTER_MAX_E / 1024;
        float4 w[PER];
#pragma unroll
        for (int j = 0; j < PER; ++j)
            if (dot && tid * 4u + 1024u * j < E) {
                w[j] = *reinterpret_cast<const float4 *>(W + tid * 4u + 1024u * j);
                if (norm == 2u) {
                    const float4 g = *reinterpret_cast<const float4 *>(NW + tid * 4u + 1024u * j);
                    w[j] = make_float4(w[j].x * g.x, w[j].y * g.y, w[j].z * g.z, w[j].w * g.w);
                }
            }
#pragma unroll
        for (int t = 0; t < ROUTER_MAX_TOK; ++t) {
            if ((uint32_t)t < n_tok) {
                float acc = 0.f, ss = 0.f;
#pragma unroll
                for (int j = 0; j < PER; ++j)
                    if (tid * 4u + 1024u * j < E) {
                        const float4 v = *reinterpret_cast<const float4 *>(X + x_off + t * x_stride + tid * 4u + 1024u * j);
                        if (dot) acc += (w[j].x * v.x + w[j].y * v.y) + (w[j].z * v.z + w[j].w * v.w);
                        if (norm) ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
                    }
                if (dot) {
                    const float s = gd_wave_sum(acc);
                    if (lane == 0) red[wave][t] = s;
                }
                if (norm) {
                    const float q = gd_wave_sum(ss);
                    if (lane == 0) reds[wave][t] = q;
                }
            }
        }
    }
    __syncthreads();
    if (tid < n_tok && row < NE) {
        float v = (red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid]);
        if (norm) {
            const float q = (reds[0][tid] + reds[1][tid]) + (reds[2][tid] + reds[3][tid]);
            v *= 1.0f / sqrtf(q / (float)E + gd_bits_f32(a.c[19]));
        }
        if (a.c[8] != 0xffffffffu) v += gd_buf<const float>(a, a.c[8])[a.c[9] + row];
        gd_buf<float>(a, a.c[10])[a.c[11] + tid * NE + row] = v;
    }
    if (rotate_here) {
        uint32_t *XH = gd_buf<uint32_t>(a, a.c[14]) + a.c[15];
#pragma unroll
        for (int t = 0; t < ROUTER_MAX_TOK; ++t) {
            if ((uint32_t)t >= n_tok) break;
            float x0 = rx[t][0], x1 = rx[t][1];
            if (norm) {
                const float q = (reds[0][t] + reds[1][t]) + (reds[2][t] + reds[3][t]);
                const float sc = 1.0f / sqrtf(q / (float)E + gd_bits_f32(a.c[19]));
                x0 *= sc;
                x1 *= sc;
            }
            if (has_signs || norm == 2u) {
                x0 *= rs[0];
                x1 *= rs[1];
            }
            if (has_signs) {
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
