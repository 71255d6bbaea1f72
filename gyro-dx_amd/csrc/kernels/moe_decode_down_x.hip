// Decode path for layers whose experts and projections mix Gyro types, step 3: SwiGLU and the
// down-input rotation, the fused dequant-GEMV of the down rows, the route-weighted combine
// (src/engine.zig:603-641) and, when the layer has one, the shared expert's gated output
// (src/engine.zig:644-653), structured as moe_decode_down: a group owns R output rows of one
// token for all 8 selected experts, the partials, signs and codebook are requested ahead of the
// routes, and wave w forms expert w's down input in 16-lane transform rows. Each expert's down
// rows and type come from the layer's expert table (ExpertDesc); wave w streams the R rows of
// expert w (4 R bb contiguous bytes for blocks of bb bytes, every lane's address clamped into
// them) and decodes them with the decoder of the expert's type, uniform per wave. The block or
// half-block sums of a row are added with DPP; the experts are combined in k order through LDS
// after a second barrier. Two builds:
//  - moe_decode_down_x, R = 8, for one token: lane 8 r + 2 b + hf takes half hf of block b of
//    row r, and E / 8 groups fill the GPU;
//  - moe_decode_down_xb, R = 16, for 2 to 8 tokens, whose E / 16 groups per token fill it
//    already: lane 4 r + b takes both halves of block b of row r, and each group's fixed loads
//    (partials, signs, codebook, routes) serve twice the rows.
// Both form each half block's scaled dot the same way and add the halves, then the blocks
// ((b0 + b1) + (b2 + b3)), in the same order, so a token's outputs do not depend on the build
// that ran it.
// Grid: x = E / R, y = n_tok; 512 threads.
// Constants: 0 gu_uav 1 gu_off 2 ids_uav 3 ids_off 4 weights_uav 5 weights_off 6 xtab_srv
// 7 (unused) 8 (unused) 9 (unused) 10 codebook_srv 11 signs_srv (0xffffffff: none) 12 signs_off
// 13 out_uav 14 out_off 15 E 16 F 17 n_used 18 n_tok 19 parts 20 n_expert 21 residual (0: none,
// 1: add) 22 res_uav 23 res_off 24 shared (0: none, 1: the layer's shared expert) 25 sh_h_uav
// (fp32 [n][2 SF]: W_sg x then W_su x, from moe_router) 26 (unused) 27 shg_uav (g . x [n])
// 28 shg_off 29 sh_down_srv (bf16 [E][SF]) 30 SF (<= 1024, a multiple of 256). The shared
// expert's SwiGLU a = silu(W_sg x) * W_su x is formed in LDS and its R down rows of the group
// are dotted with it (wave w takes rows w and, for R = 16, w + 8: 64 lanes per row, the same
// sums in either build); the combine adds sigmoid(g . x) times that, then the residual.
// Requires n_used == 8, F == 512 and at most 2 K-parts.
#include "gyro_fast.h"
#include "fwht.h"

#ifndef DX_PIPELINE
#define DX_PIPELINE moe_decode_down_x
#define DN_ROWS 8
#endif
#define DN_U 8
#define DN_F 512
#define DN_NB (DN_F / 128)
#define DN_MAX_BB 58
#define DN_EXPERT_WORDS (DN_ROWS * DN_NB * DN_MAX_BB / 4)  // R rows of the widest type
#define DN_ROW_LOADS (DN_ROWS / 4)                          // 16-byte loads per lane of a wave's rows
#define DN_SH_PASSES (DN_ROWS / 8)                          // shared down rows per wave
static_assert(DN_ROWS == 8 || DN_ROWS == 16, "the two builds");
#define DN_SH_MAX_F 1024
#define DN_BLOCK_STRIDE 132  // floats per 128-block in LDS (bank spread)


// Half hf of block blk of staged row r (R = 8), or the sum of its two halves (R = 16),
// against the block's activations x (128 fp32); each half's scaled dot rounded on its own.
template <int ID>
__device__ __forceinline__ float dx_unit(const uint32_t *rows_k, uint32_t r, uint32_t blk, uint32_t hf,
                                         const uint32_t *book, const float *x) {
    constexpr int BB = GyroT<ID>::BB, NW = gyro_nw<ID>();
    const uint32_t off = r * (DN_NB * BB) + blk * BB;  // even
    const uint32_t *w0 = rows_k + (off >> 2);
    uint32_t d[NW + 1];
#pragma unroll
    for (int j = 0; j <= NW; ++j) d[j] = w0[j];
    float sc;
    uint32_t w[NW];
    gyro_unpack<ID>(d, (off & 2u) != 0u, sc, w);
#if DN_ROWS == 8
    return gd_rounded(sc * gyro_half_dot<ID>(w, hf, book, x + 64u * hf));
#else
    const float h0 = gd_rounded(sc * gyro_half_dot<ID>(w, 0u, book, x));
    const float h1 = gd_rounded(sc * gyro_half_dot<ID>(w, 1u, book, x + 64u));
    return h0 + h1;
#endif
}

#define DX_DEFINE(NAME, WG) GD_PIPELINE_NAMED(NAME, WG)  // expands NAME before it is named
DX_DEFINE(DX_PIPELINE, 512) {
    __shared__ uint4 book4[512];
    __shared__ uint32_t rows[DN_U * DN_EXPERT_WORDS];
    __shared__ float act[DN_U * DN_NB * DN_BLOCK_STRIDE];
    __shared__ float dk[DN_U][DN_ROWS];
    __shared__ float sh_a[DN_SH_MAX_F];
    __shared__ float shs[DN_ROWS];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t E = a.c[15], n_tok = a.c[18], parts = a.c[19], NE = a.c[20];
    const uint32_t t = blockIdx.y, row0 = gd_xcd_group(blockIdx.x, gridDim.x) * DN_ROWS;
    const uint32_t n_slots = n_tok * DN_U;

    // Down input of expert `wave`, block b = lane / 16, values l16 * 8 .. l16 * 8 + 7 of the
    // block. The partials, signs and codebook go first: they do not depend on the routes.
    const uint32_t b = lane >> 4, l16 = lane & 15u;
    const uint32_t slot = t * DN_U + wave, i0 = b * 128u + l16 * 8u;
    const uint32_t *GU = gd_buf<const uint32_t>(a, a.c[0]) + a.c[1];
    gd_u32x4 g4[2][2], u4[2][2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const uint32_t pp = (uint32_t)p < parts ? p : 0u;
        gd_gu32x4 *gp = gd_global4(GU + ((size_t)(pp * n_slots + slot) * 2u) * DN_F + i0);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            g4[p][j] = gp[j];
            u4[p][j] = gp[DN_F / 4 + j];
        }
    }
    const bool has_signs = a.c[11] != 0xffffffffu;
    gd_u32x4 s4[2];
    if (has_signs) {
        gd_gu32x4 *S = gd_global4(gd_buf<const uint32_t>(a, a.c[11]) + a.c[12] + i0);
#pragma unroll
        for (int j = 0; j < 2; ++j) s4[j] = S[j];
    }
    const gd_u32x4 cbv = gd_global4(gd_buf<const uint32_t>(a, a.c[10]))[tid];
    // Shared expert inputs: lane q of wave w holds 8 bf16 of down row row0 + w + 8 ps (pass
    // ps) at columns 8 q + 512 m; thread tid holds the gate and up values of columns tid + 512 i.
    const bool shared = a.c[24] != 0u;
    const uint32_t SF = shared ? a.c[30] : 0u;
    constexpr int SHM = DN_SH_MAX_F / 512;
    gd_u32x4 sw[DN_SH_PASSES][SHM];
    float shgv[DN_SH_MAX_F / 512], shuv[DN_SH_MAX_F / 512];
    if (shared) {
        gd_guint *Hs = gd_global(gd_buf<const uint32_t>(a, a.c[25]) + (size_t)t * 2u * SF);
#pragma unroll
        for (int ps = 0; ps < DN_SH_PASSES; ++ps) {
            const uint32_t *Wsd =
                gd_buf<const uint32_t>(a, a.c[29]) + ((size_t)(row0 + wave + 8u * ps) * SF + 8u * lane) / 2u;
#pragma unroll
            for (int m = 0; m < SHM; ++m)
                if (8u * lane + 512u * m < SF) sw[ps][m] = *gd_global4(Wsd + 256u * m);
        }
#pragma unroll
        for (int m = 0; m < DN_SH_MAX_F / 512; ++m)
            if (tid + 512u * m < SF) {
                shgv[m] = gd_bits_f32(Hs[tid + 512u * m]);
                shuv[m] = gd_bits_f32(Hs[SF + tid + 512u * m]);
            }
    }

    // The R rows of expert `wave`: R bb / 4 (at most 232) chunks of 16 bytes, R / 4 loads per
    // lane, every address clamped into the expert's rows.
    cuint *ids = as_const(gd_buf<const uint32_t>(a, a.c[2]) + a.c[3] + t * DN_U);
    // The route weights too, so their latency overlaps the rows' (they are read at the end).
    cfloat *wtp = as_const(gd_buf<const float>(a, a.c[4]) + a.c[5] + t * DN_U);
    float wts[DN_U];
#pragma unroll
    for (int kx = 0; kx < DN_U; ++kx) wts[kx] = wtp[kx];
    // The shared expert's gate dot and the residual of the output rows, read at the end too.
    float sh_gate = 0.f, res_v = 0.f;
    if (tid < DN_ROWS) {
        if (shared) sh_gate = gd_bits_f32(*gd_global(gd_buf<const uint32_t>(a, a.c[27]) + a.c[28] + t));
        if (a.c[21]) res_v = gd_bits_f32(*gd_global(gd_buf<const uint32_t>(a, a.c[22]) + a.c[23] + t * E + row0 + tid));
    }
    // The expert table's down entries, lane l holding experts l + 64 j (row address and types,
    // j < 4), requested beside the routes: once the route names the wave's expert, its entry is
    // read from a register instead of a load that depends on the route.
    uint32_t tlo[4], thi[4], tty[4];
    {
        const uint32_t *XT = gd_buf<const uint32_t>(a, a.c[6]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t ex = min(lane + 64u * (uint32_t)j, NE - 1u);
            gd_guint *ent = gd_global(XT + (size_t)ex * (sizeof(ExpertDesc) / 4u));
            tlo[j] = ent[4];
            thi[j] = ent[5];
            tty[j] = ent[6];
        }
    }
    const uint32_t ew = min(ids[wave], NE - 1u);
    const uint32_t ej = ew >> 6, el = ew & 63u;  // uniform per wave
    uint32_t vlo = tlo[0], vhi = thi[0], vty = tty[0];
#pragma unroll
    for (int j = 1; j < 4; ++j)
        if (ej == (uint32_t)j) {
            vlo = tlo[j];
            vhi = thi[j];
            vty = tty[j];
        }
    const uint32_t type_id = ((uint32_t)__builtin_amdgcn_readlane((int)vty, (int)el) >> 16) & 0xffu;
    const uint64_t down_addr = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)vhi, (int)el) << 32) |
                               (uint32_t)__builtin_amdgcn_readlane((int)vlo, (int)el);
    const uint32_t bbw = block_bytes_of_type(type_id), nch = DN_ROWS / 4u * bbw;
    const uint8_t *src = reinterpret_cast<const uint8_t *>(down_addr) + (size_t)row0 * DN_NB * bbw;
    gd_u32x4 rv[DN_ROW_LOADS];
#pragma unroll
    for (int j = 0; j < DN_ROW_LOADS; ++j)
        rv[j] = *gd_global4(reinterpret_cast<const uint32_t *>(src + min(lane + 64u * j, nch - 1u) * 16u));

    float v[8];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float g = parts > 1u ? gd_bits_f32(g4[0][j][c]) + gd_bits_f32(g4[1][j][c]) : gd_bits_f32(g4[0][j][c]);
            const float u = parts > 1u ? gd_bits_f32(u4[0][j][c]) + gd_bits_f32(u4[1][j][c]) : gd_bits_f32(u4[0][j][c]);
            v[4 * j + c] = gd_silu_rcp(g) * u;
        }
    }
    if (has_signs) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int c = 0; c < 4; ++c) v[4 * j + c] *= gd_bits_f32(s4[j][c]);
        // Widths 1..4: element bits 0..2 are the register index bits.
#pragma unroll
        for (int w = 1; w < 8; w <<= 1)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (!(j & w)) {
                    const float lo = v[j], hi = v[j + w];
                    v[j] = lo + hi;
                    v[j + w] = lo - hi;
                }
        // Widths 8, 16, 32, 64: partners are lanes l16 ^ 1, ^ 2, ^ 4, ^ 8 of the 16-lane row.
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
    if (shared) {
#pragma unroll
        for (int m = 0; m < DN_SH_MAX_F / 512; ++m)
            if (tid + 512u * m < SF) sh_a[tid + 512u * m] = gd_silu_accurate(shgv[m]) * shuv[m];
    }
    float4 *dst = reinterpret_cast<float4 *>(act + (wave * DN_NB + b) * DN_BLOCK_STRIDE + l16 * 8u);
    dst[0] = make_float4(v[0], v[1], v[2], v[3]);
    dst[1] = make_float4(v[4], v[5], v[6], v[7]);
    reinterpret_cast<gd_u32x4 *>(book4)[tid] = cbv;
#pragma unroll
    for (int j = 0; j < DN_ROW_LOADS; ++j) {
        const uint32_t c = lane + 64u * j;
        if (c < nch) {
            uint32_t *rdst = rows + wave * DN_EXPERT_WORDS + c * 4u;
            rdst[0] = rv[j][0]; rdst[1] = rv[j][1]; rdst[2] = rv[j][2]; rdst[3] = rv[j][3];
        }
    }
    __syncthreads();

    {   // Unit (row r, block blk, half hf) of expert `wave` on lane 8 r + 2 blk + hf (R = 8), or
        // (row r, block blk, both halves) on lane 4 r + blk (R = 16), with the expert's down type.
#if DN_ROWS == 8
        const uint32_t r = lane >> 3, blk = (lane >> 1) & 3u, hf = lane & 1u;
#else
        const uint32_t r = lane >> 2, blk = lane & 3u, hf = 0u;
#endif
        const uint32_t *rows_k = rows + wave * DN_EXPERT_WORDS;
        const uint32_t *book = reinterpret_cast<const uint32_t *>(book4);
        const float *xa = act + (wave * DN_NB + blk) * DN_BLOCK_STRIDE;
        float s = 0.f;
#define DX_CASE(ID) s = dx_unit<ID>(rows_k, r, blk, hf, book, xa)
        GYRO_TYPE_SWITCH(type_id, DX_CASE)
#undef DX_CASE
#if DN_ROWS == 8
        s = s + gd_dpp_f<0xB1>(s);   // the two halves of a block
        s = s + gd_dpp_f<0x4E>(s);   // b0 + b1, b2 + b3
        s = s + gd_dpp_f<0x104>(s);  // row_shl:4: (b0 + b1) + (b2 + b3) in lane 8 r
        if ((lane & 7u) == 0u) dk[wave][r] = s;
#else
        s = s + gd_dpp_f<0xB1>(s);  // b0 + b1, b2 + b3
        s = s + gd_dpp_f<0x4E>(s);  // (b0 + b1) + (b2 + b3)
        if (blk == 0) dk[wave][r] = s;
#endif
    }
    if (shared) {  // shared down rows row0 + wave + 8 ps over the wave's 64 lanes
#pragma unroll
        for (int ps = 0; ps < DN_SH_PASSES; ++ps) {
            float p = 0.f;
#pragma unroll
            for (int m = 0; m < SHM; ++m) {
                if (8u * lane + 512u * m < SF) {
                    const float *av = sh_a + 8u * lane + 512u * m;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        p += gd_bits_f32(sw[ps][m][e] << 16) * av[2 * e];
                        p += gd_bits_f32(sw[ps][m][e] & 0xffff0000u) * av[2 * e + 1];
                    }
                }
            }
            p = gd_wave_sum_dpp(p);
            if (lane == 0u) shs[wave + 8u * ps] = p;
        }
    }
    __syncthreads();
    if (tid < DN_ROWS) {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < DN_U; ++k) acc += wts[k] * dk[k][tid];
        if (shared) {
            const float g = gd_sigmoid_accurate(sh_gate);
            acc += g * shs[tid];
        }
        if (a.c[21]) acc = res_v + acc;
        gd_buf<float>(a, a.c[13])[a.c[14] + t * E + row0 + tid] = acc;
    }
}
