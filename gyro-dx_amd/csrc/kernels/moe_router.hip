// Decode path, step 1: router logits and the rotated expert input for up to 8 tokens.
//   logits[t][r] = W_r[r] . x[t] (+ bias[r])          src/engine.zig:526 (kernels.matmul)
//   xh[t] = H_128 (gate_signs * x[t]) per 128-block    src/engine.zig:547-551
// Optionally the layer input is first normalised as in a stack (rmsNorm, src/kernels.zig:281-291):
// x[t] is replaced by h[t] = x[t] * s[t] * w with s[t] = 1 / sqrt(mean(x[t]^2) + eps). Every
// group accumulates mean(x[t]^2) beside its dot product from the same loads; the logit is then
// s[t] * ((W_r[r] * w) . x[t]).
// The rotated input is written in fp32 (xh[t][i]), the precision of src/engine.zig:547-551, which
// the gate/up kernels multiply by fp32 codebook values.
// Grid: x = n_expert + E / 128; 256 threads. Group r < n_expert computes router row r; group
// n_expert + b rotates block b of every token (wave 0), beside the router rows rather than after
// them in the same wave (with the norm, its four waves first sum the tokens' squares).
// Constants: 0 x_uav 1 x_off 2 x_stride 3 n_tok 4 router_srv 5 router_off 6 n_expert 7 E
// 8 bias_srv (0xffffffff: none) 9 bias_off 10 logits_uav 11 logits_off 12 signs_srv
// (0xffffffff: copy) 13 signs_off 14 xh_uav (fp32 [n_tok][E]) 15 xh_off (words) 16 norm (0: none, 1: RMSNorm
// without weight, 2: with weight; zero when the caller passes 16 constants) 17 norm_w_srv
// 18 norm_w_off 19 eps (fp32 bits) 20 shared rows (2 SF; 0: no shared expert) 21 sh_w_srv (bf16
// [2 SF][E]: gate rows then up rows) 22 sh_h_uav (fp32 [n][2 SF]) 23 sh_gate_srv (fp32 [E])
// 24 sh_g_uav (fp32 [n]). With a shared expert (src/engine.zig:644-653) the grid has 2 SF / 4 + 1
// further groups after the n_expert + E / 128 above: each of the first computes 4 bf16 rows
// (one per wave) of W_sg x and W_su x on the unrotated input, the last the gate dot g . x. The
// shared groups require E <= 2048.
// Every load is a global load issued ahead of its use, and the wave sums run on DPP.
#include "fwht.h"

#define ROUTER_MAX_TOK 8
#define ROUTER_MAX_E 4096

#define SH_ROWS_PER_GROUP 4
#define SH_MAX_E 2048  // hidden width covered by the fused shared-expert rows

// Shared expert row 4 sg + w of W_sh (bf16, E columns) on wave w; lane l covers columns
// 8 l + 512 m (m < E / 512).
__device__ __forceinline__ float4 rt_f4(gd_u32x4 v) {
    return make_float4(gd_bits_f32(v[0]), gd_bits_f32(v[1]), gd_bits_f32(v[2]), gd_bits_f32(v[3]));
}
__device__ __forceinline__ void router_shared_rows(const GdArgs &a, uint32_t sg, uint32_t n_tok, uint32_t E) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t rows = a.c[20], r = sg * SH_ROWS_PER_GROUP + wave;
    if (r >= rows) return;  // uniform per wave; no barrier follows
    const uint32_t *Wsh = gd_buf<const uint32_t>(a, a.c[21]) + ((size_t)r * E + 8u * lane) / 2u;
    const uint32_t *X = gd_buf<const uint32_t>(a, a.c[0]) + a.c[1] + 8u * lane;
    float *H = gd_buf<float>(a, a.c[22]);
    constexpr int MM = SH_MAX_E / 512;  // column chunks
    gd_u32x4 w[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m)
        if (512u * m < E) w[m] = *gd_global4(Wsh + 256u * m);
    for (uint32_t t = 0; t < n_tok; ++t) {
        float acc = 0.f;
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            if (512u * m >= E) break;
            gd_gu32x4 *xp = gd_global4(X + t * a.c[2] + 512u * m);
            const float4 x0 = rt_f4(xp[0]), x1 = rt_f4(xp[1]);
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc += gd_bits_f32(w[m][q] << 16) * xv[2 * q];
                acc += gd_bits_f32(w[m][q] & 0xffff0000u) * xv[2 * q + 1];
            }
        }
        const float v = gd_wave_sum_dpp(acc);
        if (lane == 0) H[t * rows + r] = v;
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
        const uint32_t first_sh = NE + E / 128u;
        if (a.c[20] && row >= first_sh) {
            const uint32_t sg = row - first_sh, n_sg = a.c[20] / SH_ROWS_PER_GROUP;
            if (sg < n_sg) {
                router_shared_rows(a, sg, n_tok, E);
            } else {
                // The gate dot g . x (fp32 row), one wave per token.
                // Wave w takes tokens w, w + 4, ...; lane l the 4 columns 4 l + 256 m of every
                // 256-column chunk m, all loads in flight together (E <= 2048).
                const uint32_t *G = gd_buf<const uint32_t>(a, a.c[23]) + 4u * lane;
                const uint32_t *XU = reinterpret_cast<const uint32_t *>(X) + x_off + 4u * lane;
                for (uint32_t t = wave; t < n_tok; t += 4u) {
                    float4 gv[SH_MAX_E / 256], xv[SH_MAX_E / 256];
#pragma unroll
                    for (int m = 0; m < SH_MAX_E / 256; ++m)
                        if (256u * m < E) {
                            gv[m] = rt_f4(*gd_global4(G + 256u * m));
                            xv[m] = rt_f4(*gd_global4(XU + t * x_stride + 256u * m));
                        }
                    float acc = 0.f;
#pragma unroll
                    for (int m = 0; m < SH_MAX_E / 256; ++m)
                        if (256u * m < E) acc += (gv[m].x * xv[m].x + gv[m].y * xv[m].y) + (gv[m].z * xv[m].z + gv[m].w * xv[m].w);
                    acc = gd_wave_sum_dpp(acc);
                    if (lane == 0) gd_buf<float>(a, a.c[24])[t] = acc;
                }
            }
            return;
        }
    }
    const float *NW = norm == 2u ? gd_buf<const float>(a, a.c[17]) + a.c[18] : nullptr;
    const bool dot = row < NE;  // uniform per group
    const bool rot = !dot && row < NE + E / 128u;  // a rotation group: block row - NE
    const bool rotate_here = rot && wave == 0;
    // Rotation inputs first: in pass p, lane l of wave 0 holds values 8 (l % 16) .. + 7 of the
    // group's block of token 4 p + l / 16.
    const uint32_t l16 = lane & 15u, blk = rot ? row - NE : 0u, ri = blk * 128u + l16 * 8u;
    const bool has_signs = a.c[12] != 0xffffffffu;
    // The row's bias, requested first so that its latency is not added after the barrier.
    const bool has_bias = a.c[8] != 0xffffffffu;
    float bias_v = 0.f;
    if (dot && has_bias && tid < n_tok) bias_v = gd_bits_f32(*gd_global(gd_buf<const uint32_t>(a, a.c[8]) + a.c[9] + row));
    float rx[2][8], rs[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) rs[j] = 1.f;
    if (rotate_here) {
        if (has_signs) {
            gd_gu32x4 *sv = gd_global4(gd_buf<const uint32_t>(a, a.c[12]) + a.c[13] + ri);
            const float4 s0 = rt_f4(sv[0]), s1 = rt_f4(sv[1]);
            rs[0] = s0.x; rs[1] = s0.y; rs[2] = s0.z; rs[3] = s0.w;
            rs[4] = s1.x; rs[5] = s1.y; rs[6] = s1.z; rs[7] = s1.w;
        }
        if (norm == 2u) {
            gd_gu32x4 *nv = gd_global4(reinterpret_cast<const uint32_t *>(NW) + ri);
            const float4 n0 = rt_f4(nv[0]), n1 = rt_f4(nv[1]);
            rs[0] *= n0.x; rs[1] *= n0.y; rs[2] *= n0.z; rs[3] *= n0.w;
            rs[4] *= n1.x; rs[5] *= n1.y; rs[6] *= n1.z; rs[7] *= n1.w;
        }
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const uint32_t t = 4u * (uint32_t)p + (lane >> 4);
            if (t < n_tok) {
                gd_gu32x4 *xv = gd_global4(reinterpret_cast<const uint32_t *>(X) + x_off + t * x_stride + ri);
                const float4 x0 = rt_f4(xv[0]), x1 = rt_f4(xv[1]);
                rx[p][0] = x0.x; rx[p][1] = x0.y; rx[p][2] = x0.z; rx[p][3] = x0.w;
                rx[p][4] = x1.x; rx[p][5] = x1.y; rx[p][6] = x1.z; rx[p][7] = x1.w;
            }
        }
    }
    // Groups with a router row compute its dot products; with the norm, every group that has a
    // router row or a rotation block also needs the tokens' sums of squares.
    if (dot || (norm && rot)) {
        const uint32_t *W = gd_buf<const uint32_t>(a, a.c[4]) + a.c[5] + (size_t)(dot ? row : 0u) * E;
        constexpr int PER = ROUTER_MAX_E / 1024;
        float4 w[PER];
#pragma unroll
        for (int j = 0; j < PER; ++j)
            if (dot && tid * 4u + 1024u * j < E) {
                w[j] = rt_f4(*gd_global4(W + tid * 4u + 1024u * j));
                if (norm == 2u) {
                    const float4 g = rt_f4(*gd_global4(reinterpret_cast<const uint32_t *>(NW) + tid * 4u + 1024u * j));
                    w[j] = make_float4(w[j].x * g.x, w[j].y * g.y, w[j].z * g.z, w[j].w * g.w);
                }
            }
        const uint32_t *XU = reinterpret_cast<const uint32_t *>(X) + x_off + tid * 4u;
        // Every token's inputs are loaded before the first token's sums, so the tokens' load
        // latencies overlap instead of following one another.
        float4 xt[ROUTER_MAX_TOK][PER];
#pragma unroll
        for (int t = 0; t < ROUTER_MAX_TOK; ++t)
            if ((uint32_t)t < n_tok) {
#pragma unroll
                for (int j = 0; j < PER; ++j)
                    if (tid * 4u + 1024u * j < E) xt[t][j] = rt_f4(*gd_global4(XU + t * x_stride + 1024u * j));
            }
#pragma unroll
        for (int t = 0; t < ROUTER_MAX_TOK; ++t) {
            if ((uint32_t)t < n_tok) {
                float acc = 0.f, ss = 0.f;
#pragma unroll
                for (int j = 0; j < PER; ++j)
                    if (tid * 4u + 1024u * j < E) {
                        const float4 v = xt[t][j];
                        if (dot) acc += (w[j].x * v.x + w[j].y * v.y) + (w[j].z * v.z + w[j].w * v.w);
                        if (norm) ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
                    }
                if (dot) {
                    const float s = gd_wave_sum_dpp(acc);
                    if (lane == 0) red[wave][t] = s;
                }
                if (norm) {
                    const float q = gd_wave_sum_dpp(ss);
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
        if (has_bias) v += bias_v;
        gd_buf<float>(a, a.c[10])[a.c[11] + tid * NE + row] = v;
    }
    if (rotate_here) {
        uint32_t *XH = gd_buf<uint32_t>(a, a.c[14]) + a.c[15];
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            if (4u * (uint32_t)p >= n_tok) break;  // uniform
            const uint32_t t = 4u * (uint32_t)p + (lane >> 4);  // the same for a 16-lane row
            const bool tv = t < n_tok;
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = tv ? rx[p][j] : 0.f;
            if (norm) {
                const uint32_t tq = tv ? t : 0u;
                const float q = (reds[0][tq] + reds[1][tq]) + (reds[2][tq] + reds[3][tq]);
                const float sc = 1.0f / sqrtf(q / (float)E + gd_bits_f32(a.c[19]));
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] *= sc;
            }
            if (has_signs || norm == 2u) {
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] *= rs[j];
            }
            if (has_signs) {
                // Widths 1, 2, 4 in registers, then 8, 16, 32, 64 with lanes l16 ^ 1, ^ 2, ^ 4,
                // ^ 8 of the 16-lane row (the stage order of src/gyro.zig:152-172).
#pragma unroll
                for (int w = 1; w < 8; w <<= 1)
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        if (!(j & w)) {
                            const float lo = v[j], hi = v[j + w];
                            v[j] = lo + hi;
                            v[j + w] = lo - hi;
                        }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float p1 = gd_dpp_f<0xB1>(v[j]);  // quad_perm [1,0,3,2]
                    v[j] = (l16 & 1u) ? p1 - v[j] : v[j] + p1;
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float p2 = gd_dpp_f<0x4E>(v[j]);  // quad_perm [2,3,0,1]
                    v[j] = (l16 & 2u) ? p2 - v[j] : v[j] + p2;
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float up4 = gd_dpp_f<0x104>(v[j]);  // row_shl:4, lane + 4
                    const float dn4 = gd_dpp_f<0x114>(v[j]);  // row_shr:4, lane - 4
                    v[j] = (l16 & 4u) ? dn4 - v[j] : v[j] + up4;
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float up8 = gd_dpp_f<0x108>(v[j]);  // row_shl:8, lane + 8
                    const float dn8 = gd_dpp_f<0x118>(v[j]);  // row_shr:8, lane - 8
                    v[j] = (l16 & 8u) ? dn8 - v[j] : v[j] + up8;
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] *= GD_INV_SQRT128;
            }
            if (tv) {
                gd_u32x4 o0, o1;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    o0[j] = gd_f32_bits(v[j]);
                    o1[j] = gd_f32_bits(v[4 + j]);
                }
                gd_u32x4 *dst = reinterpret_cast<gd_u32x4 *>(XH + t * E + blk * 128u + l16 * 8u);
                dst[0] = o0;
                dst[1] = o1;
            }
        }
    }
}
