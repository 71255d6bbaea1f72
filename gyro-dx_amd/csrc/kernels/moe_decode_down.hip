// Decode path, step 3: SwiGLU and the down-input rotation, the fused TQ2_T dequant-GEMV of the
// down rows, and the route-weighted combine (src/engine.zig:603-641), with no communication
// between groups.
//
// A group owns 8 output rows of one token for all 8 selected experts, so the combine is local
// and summed in k order. The routes, gate/up partials, signs and codebook are requested first
// (global and scalar loads); wave w streams the 8 down rows of expert w (1088 contiguous bytes)
// from HBM and, while they arrive, forms expert w's down input a = H_128(s_down * silu(g) * u)
// from the gate/up partials: a 16-lane row of the wave transforms one 128-block holding 8
// consecutive values per lane (widths 1..4 in registers, 8, 16, 32, 64 across lanes with DPP:
// the butterfly order of src/gyro.zig:152-172). After one barrier, lane 8 k + 2 bb + hf of wave
// w decodes half hf (16 trellis steps) of block bb of output row w of expert k against a in
// LDS; the 8 half-block sums of an expert are added with DPP, and lane 0 combines the experts
// in k order.
// Grid: x = E / 8, y = n_tok; 512 threads.
// Constants: 0 gu_uav 1 gu_off 2 ids_uav 3 ids_off 4 weights_uav 5 weights_off 6 base_lo
// 7 base_hi 8 slot_stride 9 down_off (bytes from an expert's bundle start) 10 codebook_srv
// 11 signs_srv (0xffffffff: none) 12 signs_off 13 out_uav 14 out_off 15 E 16 F 17 n_used
// 18 n_tok 19 parts 20 n_expert 21 residual (0: none, 1: add) 22 res_uav 23 res_off: with the
// residual each output adds res[t][row] after the combine (the residual step of a stack; res
// may alias out). Constants past the caller's count read zero, so a 21-constant dispatch has
// no residual.
// Requires TQ2_T experts, n_used == 8, F == 512 and at most 2 K-parts.
#include "gyro_fast.h"
#include "fwht.h"

#define DN_ROWS 8
#define DN_U 8
#define DN_F 512
#define DN_NB (DN_F / 128)
#define DN_ROW_BYTES (DN_NB * 34)
#define DN_BLOCK_STRIDE 132  // floats per 128-block in LDS (bank spread)


GD_PIPELINE_NAMED(moe_decode_down, 512) {
    __shared__ uint4 book4[512];
    __shared__ uint32_t rows[DN_U * DN_ROWS * DN_ROW_BYTES / 4];
    __shared__ float act[DN_U * DN_NB * DN_BLOCK_STRIDE];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
    const uint32_t E = a.c[15], n_tok = a.c[18], parts = a.c[19], NE = a.c[20];
    const uint32_t t = blockIdx.y, row0 = gd_xcd_group(blockIdx.x, gridDim.x) * DN_ROWS;
    const uint32_t n_slots = n_tok * DN_U;
    const bool has_signs = a.c[11] != 0xffffffffu;

    // Every table read up front (each is a dependent scalar load); the routes first, since the
    // rows' loads wait for them. Without signs the codebook entry stands in (never read).
    const uint32_t *ids_p = gd_buf<const uint32_t>(a, a.c[2]);
    const float *wts_p = gd_buf<const float>(a, a.c[4]);
    const uint32_t *GU = gd_buf<const uint32_t>(a, a.c[0]) + a.c[1];
    const uint32_t *cb_p = gd_buf<const uint32_t>(a, a.c[10]);
    const uint32_t *sg_p = gd_buf<const uint32_t>(a, has_signs ? a.c[11] : a.c[10]);
    cuint *ids = as_const(ids_p + a.c[3] + t * DN_U);
    cfloat *wtp = as_const(wts_p + a.c[5] + t * DN_U);
    const uint32_t ew = min(ids[wave], NE - 1u);
    float wts[DN_U];  // read at the end; loaded now so that their latency overlaps the rows'
#pragma unroll
    for (int kx = 0; kx < DN_U; ++kx) wts[kx] = wtp[kx];

    // Down input of expert `wave`, block b = lane / 16, values l16 * 8 .. l16 * 8 + 7 of the
    // block.
    const uint32_t b = lane >> 4, l16 = lane & 15u;
    const uint32_t slot = t * DN_U + wave, i0 = b * 128u + l16 * 8u;
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
    gd_u32x4 s4[2];
    if (has_signs) {
        gd_gu32x4 *S = gd_global4(sg_p + a.c[12] + i0);
#pragma unroll
        for (int j = 0; j < 2; ++j) s4[j] = S[j];
    }
    const gd_u32x4 cbv = gd_global4(cb_p)[tid];

    // The 8 rows of expert `wave`: 68 chunks of 16 bytes, two per lane (the second for lanes < 4).
    const uint64_t layer_base = (uint64_t)a.c[6] | ((uint64_t)a.c[7] << 32);
    const uint8_t *src = reinterpret_cast<const uint8_t *>(layer_base) + (uint64_t)ew * a.c[8] + a.c[9] +
                         (size_t)row0 * DN_ROW_BYTES;
    gd_u32x4 rv[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) rv[j] = *gd_global4(reinterpret_cast<const uint32_t *>(src + min(lane + 64u * j, 67u) * 16u));

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
    float4 *dst = reinterpret_cast<float4 *>(act + (wave * DN_NB + b) * DN_BLOCK_STRIDE + l16 * 8u);
    dst[0] = make_float4(v[0], v[1], v[2], v[3]);
    dst[1] = make_float4(v[4], v[5], v[6], v[7]);
    reinterpret_cast<gd_u32x4 *>(book4)[tid] = cbv;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t c = lane + 64u * j;
        if (c < 68u) {
            uint32_t *rdst = rows + wave * (DN_ROWS * DN_ROW_BYTES / 4) + c * 4u;
            rdst[0] = rv[j][0]; rdst[1] = rv[j][1]; rdst[2] = rv[j][2]; rdst[3] = rv[j][3];
        }
    }
    __syncthreads();

    // Unit (expert k, row w, block bb, half hf) on lane 8 k + 2 bb + hf.
    const uint32_t k = lane >> 3, bb = (lane >> 1) & 3u, hf = lane & 1u;
    const uint32_t off = k * (DN_ROWS * DN_ROW_BYTES) + wave * DN_ROW_BYTES + bb * 34u;
    const uint32_t *w = rows + (off >> 2);
    uint32_t d[9];
#pragma unroll
    for (int j = 0; j < 9; ++j) d[j] = w[j];
    float sc;
    uint32_t q[8];
    tq2_unpack(d, (off & 2u) != 0u, sc, q);
    float sum = gd_rounded(sc * tq2_half_dot(q, hf, reinterpret_cast<const uint32_t *>(book4),
                                             act + (k * DN_NB + bb) * DN_BLOCK_STRIDE + 64u * hf));
    sum = sum + gd_dpp_f<0xB1>(sum);   // the two halves of a block
    sum = sum + gd_dpp_f<0x4E>(sum);   // b0 + b1, b2 + b3
    sum = sum + gd_dpp_f<0x104>(sum);  // row_shl:4: (b0 + b1) + (b2 + b3) in lane 8 k
    // Lane 0 combines row w over the experts in k order from lanes 8 k.
    float acc = 0.f;
#pragma unroll
    for (int kx = 0; kx < DN_U; ++kx)
        acc += wts[kx] * gd_bits_f32((uint32_t)__builtin_amdgcn_readlane((int)gd_f32_bits(sum), 8 * kx));
    if (lane == 0u) {
        const uint32_t orow = row0 + wave;
        if (a.c[21]) acc = gd_buf<const float>(a, a.c[22])[a.c[23] + t * E + orow] + acc;
        gd_buf<float>(a, a.c[13])[a.c[14] + t * E + orow] = acc;
    }
}
