// Decode path for layers whose experts and projections mix Gyro types, step 3: SwiGLU and the
// down-input rotation, the fused dequant-GEMV of the down rows, the route-weighted combine
// (src/engine.zig:603-641) and, when the layer has one, the shared expert's gated output
// (src/engine.zig:644-653), structured as moe_decode_down: a group owns 8 output rows of one
// token for all 8 selected experts. Each expert's down rows and type come from the layer's
// expert table (ExpertDesc); wave w streams the 8 rows of experts 2w and 2w+1 (32 bb contiguous
// bytes each for blocks of bb bytes) while it forms their down inputs. Each (expert, row,
// block) unit is decoded by one lane with the block decoder of the expert's type (the two
// half-waves of a wave hold two experts, so up to two types per wave).
// Grid: x = E / 8, y = n_tok; 256 threads.
// Constants: 0 gu_uav 1 gu_off 2 ids_uav 3 ids_off 4 weights_uav 5 weights_off 6 xtab_srv
// 7 (unused) 8 (unused) 9 (unused) 10 codebook_srv 11 signs_srv (0xffffffff: none) 12 signs_off
// 13 out_uav 14 out_off 15 E 16 F 17 n_used 18 n_tok 19 parts 20 n_expert 21 residual (0: none,
// 1: add) 22 res_uav 23 res_off 24 shared (0: none, 1: the layer's shared expert) 25 sh_h_uav
// (fp32 [n][2 SF]: W_sg x then W_su x, from moe_router) 26 (unused) 27 shg_uav (g . x [n])
// 28 shg_off 29 sh_down_srv (bf16 [E][SF]) 30 SF (<= 1024, a multiple of 256). The shared
// expert's SwiGLU a = silu(W_sg x) * W_su x is formed in LDS and its 8 down rows of the group
// are dotted with it (32 lanes per row); the combine adds sigmoid(g . x) times that, then the
// residual.
// Requires n_used == 8, F == 512 and at most 2 K-parts.
#include "gyro_fast.h"
#include "fwht.h"

#define DN_ROWS 8
#define DN_U 8
#define DN_F 512
#define DN_NB (DN_F / 128)
#define DN_MAX_BB 58
#define DN_EXPERT_WORDS (DN_ROWS * DN_NB * DN_MAX_BB / 4)  // 8 rows of the widest type
#define DN_SH_MAX_F 1024
#define DN_BLOCK_STRIDE 132  // floats per 128-block in LDS (bank spread for the 8 x streams)


template <int ID>
__device__ __forceinline__ float dx_unit(const uint32_t *rows_k, uint32_t r, uint32_t blk, const uint32_t *book,
                                         const float *x) {
    constexpr int BB = GyroT<ID>::BB, NW = gyro_nw<ID>();
    const uint32_t off = r * (DN_NB * BB) + blk * BB;  // even
    const uint32_t *w0 = rows_k + (off >> 2);
    uint32_t d[NW + 1];
#pragma unroll
    for (int j = 0; j <= NW; ++j) d[j] = w0[j];
    float sc;
    uint32_t w[NW];
    gyro_unpack<ID>(d, (off & 2u) != 0u, sc, w);
    return sc * gyro_block_dot<ID>(w, book, x);
}

GD_PIPELINE_NAMED(moe_decode_down_x, 256) {
    __shared__ uint4 book4[512];
    __shared__ uint32_t rows[DN_U * DN_EXPERT_WORDS];
    __shared__ float act[DN_U * DN_NB * DN_BLOCK_STRIDE];
    __shared__ float dk[DN_U][DN_ROWS];
    __shared__ float sh_a[DN_SH_MAX_F];
    __shared__ float shs[DN_ROWS];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t E = a.c[15], n_tok = a.c[18], parts = a.c[19], NE = a.c[20];
    const uint32_t t = blockIdx.y, row0 = blockIdx.x * DN_ROWS;
    const uint32_t n_slots = n_tok * DN_U;
    cuint *ids = as_const(gd_buf<const uint32_t>(a, a.c[2]) + a.c[3] + t * DN_U);
    const ExpertDesc *xt = gd_buf<const ExpertDesc>(a, a.c[6]);

    // Rows of experts 2w and 2w+1: 2 bb (at most 116) chunks of 16 bytes each, two loads per lane
    // and expert. Every lane's address is clamped into its own expert's rows (no per-lane choice
    // between the two experts' pointers), so each load is in bounds whatever lanes use it.
    const uint32_t e0 = min(ids[2 * wave], NE - 1u), e1 = min(ids[2 * wave + 1], NE - 1u);
    const uint32_t bb0 = block_bytes_of_type((xt[e0].types >> 16) & 0xffu);
    const uint32_t bb1 = block_bytes_of_type((xt[e1].types >> 16) & 0xffu);
    const uint8_t *src0 = reinterpret_cast<const uint8_t *>(xt[e0].down) + (size_t)row0 * DN_NB * bb0;
    const uint8_t *src1 = reinterpret_cast<const uint8_t *>(xt[e1].down) + (size_t)row0 * DN_NB * bb1;
    const uint32_t n0 = 2u * bb0, n1 = 2u * bb1;  // chunks per expert
    uint4 rv0[2], rv1[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t c = lane + 64u * j;
        rv0[j] = *reinterpret_cast<const uint4 *>(src0 + min(c, n0 - 1u) * 16u);
        rv1[j] = *reinterpret_cast<const uint4 *>(src1 + min(c, n1 - 1u) * 16u);
    }
    // Shared expert inputs, issued with the rows: thread (r = tid / 32, q = tid % 32) holds 8
    // bf16 of down row row0 + r at columns 8 q + 256 m; thread tid holds the gate and up values
    // of columns tid + 256 i.
    const bool shared = a.c[24] != 0u;
    const uint32_t SF = shared ? a.c[30] : 0u;
    uint4 sw[DN_SH_MAX_F / 256];
    float shgv[DN_SH_MAX_F / 256], shuv[DN_SH_MAX_F / 256];
    if (shared) {
        const uint16_t *Wsd = gd_buf<const uint16_t>(a, a.c[29]) + (size_t)(row0 + (tid >> 5)) * SF + 8u * (tid & 31u);
        const float *Hs = gd_buf<const float>(a, a.c[25]) + (size_t)t * 2u * SF;
#pragma unroll
        for (int m = 0; m < DN_SH_MAX_F / 256; ++m)
            if (256u * m < SF) {
                sw[m] = *reinterpret_cast<const uint4 *>(Wsd + 256u * m);
                shgv[m] = Hs[tid + 256u * m];
                shuv[m] = Hs[SF + tid + 256u * m];
            }
    }
    const uint4 *cb4 = gd_buf<const uint4>(a, a.c[10]);
    const uint4 cb0 = cb4[tid], cb1 = cb4[tid + 256u];

    // Down input of expert kk = 2 * wave + lane / 32, block b = (lane / 8) % 4, values
    // l8 * 16 .. l8 * 16 + 15 of the block.
    const uint32_t kk = wave * 2u + (lane >> 5), b = (lane >> 3) & 3u, l8 = lane & 7u;
    const uint32_t slot = t * DN_U + kk, i0 = b * 128u + l8 * 16u;
    const float *GU = gd_buf<const float>(a, a.c[0]) + a.c[1];
    float4 g4[2][4], u4[2][4];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const uint32_t pp = (uint32_t)p < parts ? p : 0u;
        const float *gp = GU + ((size_t)(pp * n_slots + slot) * 2u) * DN_F + i0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            g4[p][j] = *reinterpret_cast<const float4 *>(gp + 4 * j);
            u4[p][j] = *reinterpret_cast<const float4 *>(gp + DN_F + 4 * j);
        }
    }
    const bool has_signs = a.c[11] != 0xffffffffu;
    float4 s4[4];
    if (has_signs) {
        const float *S = gd_buf<const float>(a, a.c[11]) + a.c[12] + i0;
#pragma unroll
        for (int j = 0; j < 4; ++j) s4[j] = *reinterpret_cast<const float4 *>(S + 4 * j);
    }

    // Stage the rows and the codebook while the partials arrive.
    book4[tid] = cb0;
    book4[tid + 256u] = cb1;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t c = lane + 64u * j;
        if (c < n0) {
            uint32_t *dst = rows + (2u * wave) * DN_EXPERT_WORDS + c * 4u;
            dst[0] = rv0[j].x; dst[1] = rv0[j].y; dst[2] = rv0[j].z; dst[3] = rv0[j].w;
        }
        if (c < n1) {
            uint32_t *dst = rows + (2u * wave + 1u) * DN_EXPERT_WORDS + c * 4u;
            dst[0] = rv1[j].x; dst[1] = rv1[j].y; dst[2] = rv1[j].z; dst[3] = rv1[j].w;
        }
    }

    float v[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float4 g = parts > 1u ? make_float4(g4[0][j].x + g4[1][j].x, g4[0][j].y + g4[1][j].y,
                                                  g4[0][j].z + g4[1][j].z, g4[0][j].w + g4[1][j].w)
                                    : g4[0][j];
        const float4 u = parts > 1u ? make_float4(u4[0][j].x + u4[1][j].x, u4[0][j].y + u4[1][j].y,
                                                  u4[0][j].z + u4[1][j].z, u4[0][j].w + u4[1][j].w)
                                    : u4[0][j];
        v[4 * j + 0] = gd_silu(g.x) * u.x;
        v[4 * j + 1] = gd_silu(g.y) * u.y;
        v[4 * j + 2] = gd_silu(g.z) * u.z;
        v[4 * j + 3] = gd_silu(g.w) * u.w;
    }
    if (has_signs) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[4 * j + 0] *= s4[j].x;
            v[4 * j + 1] *= s4[j].y;
            v[4 * j + 2] *= s4[j].z;
            v[4 * j + 3] *= s4[j].w;
        }
        // Widths 1..8: element bits 0..3 are the register index bits.
#pragma unroll
        for (int w = 1; w < 16; w <<= 1)
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (!(j & w)) {
                    const float lo = v[j], hi = v[j + w];
                    v[j] = lo + hi;
                    v[j + w] = lo - hi;
                }
        // Widths 16, 32, 64: partners are lanes l8 ^ 1, ^ 2, ^ 4 of the 8-lane group.
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const float p1 = gd_dpp_f<0xB1>(v[j]);  // quad_perm [1,0,3,2]
            v[j] = (l8 & 1u) ? p1 - v[j] : v[j] + p1;
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const float p2 = gd_dpp_f<0x4E>(v[j]);  // quad_perm [2,3,0,1]
            v[j] = (l8 & 2u) ? p2 - v[j] : v[j] + p2;
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const float up4 = gd_dpp_f<0x104>(v[j]);  // row_shl:4, lane + 4
            const float dn4 = gd_dpp_f<0x114>(v[j]);  // row_shr:4, lane - 4
            v[j] = (l8 & 4u) ? dn4 - v[j] : v[j] + up4;
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] *= GD_INV_SQRT128;
    }
    if (shared) {
#pragma unroll
        for (int m = 0; m < DN_SH_MAX_F / 256; ++m)
            if (256u * m < SF) sh_a[tid + 256u * m] = gd_silu_accurate(shgv[m]) * shuv[m];
    }
    float4 *dst = reinterpret_cast<float4 *>(act + (kk * DN_NB + b) * DN_BLOCK_STRIDE + l8 * 16u);
#pragma unroll
    for (int j = 0; j < 4; ++j) dst[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
    __syncthreads();

    {   // Unit (expert k, row r, block blk), decoded with expert k's down type.
        const uint32_t k = tid >> 5, r = (tid >> 2) & 7u, blk = tid & 3u;
        const uint32_t ek = min(ids[k], NE - 1u);
        const uint32_t type_id = (xt[ek].types >> 16) & 0xffu;
        const uint32_t *rows_k = rows + k * DN_EXPERT_WORDS;
        const uint32_t *book = reinterpret_cast<const uint32_t *>(book4);
        const float *xa = act + (k * DN_NB + blk) * DN_BLOCK_STRIDE;
        float s = 0.f;
#define DX_CASE(ID) s = dx_unit<ID>(rows_k, r, blk, book, xa)
        GYRO_TYPE_SWITCH(type_id, DX_CASE)
#undef DX_CASE
        s = s + gd_dpp_f<0xB1>(s);  // b0 + b1, b2 + b3
        s = s + gd_dpp_f<0x4E>(s);  // (b0 + b1) + (b2 + b3)
        if (blk == 0) dk[k][r] = s;
    }
    if (shared) {  // shared down row row0 + tid / 32 over 32 lanes
        float p = 0.f;
        const uint32_t q = tid & 31u;
#pragma unroll
        for (int m = 0; m < DN_SH_MAX_F / 256; ++m) {
            if (256u * m >= SF) break;
            const uint32_t ww[4] = {sw[m].x, sw[m].y, sw[m].z, sw[m].w};
            const float *av = sh_a + 8u * q + 256u * m;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                p += gd_bits_f32(ww[e] << 16) * av[2 * e];
                p += gd_bits_f32(ww[e] & 0xffff0000u) * av[2 * e + 1];
            }
        }
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) p += __shfl_xor(p, o, 64);
        if (q == 0) shs[tid >> 5] = p;
    }
    __syncthreads();
    if (tid < DN_ROWS) {
        cfloat *wts = as_const(gd_buf<const float>(a, a.c[4]) + a.c[5] + t * DN_U);
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < DN_U; ++k) acc += wts[k] * dk[k][tid];
        if (shared) {
            const float g = gd_sigmoid_accurate(gd_buf<const float>(a, a.c[27])[a.c[28] + t]);
            acc += g * shs[tid];
        }
        if (a.c[21]) acc = gd_buf<const float>(a, a.c[22])[a.c[23] + t * E + row0 + tid] + acc;
        gd_buf<float>(a, a.c[13])[a.c[14] + t * E + row0 + tid] = acc;
    }
}
