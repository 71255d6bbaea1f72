// Decode path, step 3: SwiGLU and the down-input rotation, the fused TQ2_T dequant-GEMV of the
// down rows, and the route-weighted combine (src/engine.zig:603-641), with no communication
// between groups.
//
// A group owns 8 output rows of one token for all 8 selected experts, so the combine is local
// and summed in k order. Wave w streams the 8 down rows of experts 2w and 2w+1 (2 x 1088
// contiguous bytes) from HBM and, while they arrive, forms those experts' down input
// a = H_128(s_down * silu(g) * u) from the gate/up partials: an 8-lane group transforms one
// 128-block holding 16 consecutive values per lane (widths 1..8 in registers, 16, 32, 64 across
// lanes with DPP: the butterfly order of src/gyro.zig:152-172). Each (expert, row, block) unit
// is then decoded by one lane against its block of a in LDS; the four block sums of a row are
// added in order and lanes 0..7 combine the experts.
// Grid: x = E / 8, y = n_tok; 256 threads.
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
#define DN_BLOCK_STRIDE 132  // floats per 128-block in LDS (bank spread for the 8 x streams)


GD_PIPELINE_NAMED(moe_decode_down, 256) {
    __shared__ uint4 book4[512];
    __shared__ uint32_t rows[DN_U * DN_ROWS * DN_ROW_BYTES / 4];
    __shared__ float act[DN_U * DN_NB * DN_BLOCK_STRIDE];
    __shared__ float dk[DN_U][DN_ROWS];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t E = a.c[15], n_tok = a.c[18], parts = a.c[19], NE = a.c[20];
    const uint32_t t = blockIdx.y, row0 = blockIdx.x * DN_ROWS;
    const uint32_t n_slots = n_tok * DN_U;
    cuint *ids = as_const(gd_buf<const uint32_t>(a, a.c[2]) + a.c[3] + t * DN_U);
    const uint64_t layer_base = (uint64_t)a.c[6] | ((uint64_t)a.c[7] << 32);

    // Rows of experts 2w and 2w+1: 136 chunks of 16 bytes, three per lane (the last partly).
    const uint32_t e0 = min(ids[2 * wave], NE - 1u), e1 = min(ids[2 * wave + 1], NE - 1u);
    uint4 rv[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const uint32_t c = min(lane + 64u * j, 135u), hi = c >= 68u, ch = c - 68u * hi;
        const uint8_t *src = reinterpret_cast<const uint8_t *>(layer_base) + (uint64_t)(hi ? e1 : e0) * a.c[8] +
                             a.c[9] + (size_t)row0 * DN_ROW_BYTES + ch * 16u;
        rv[j] = *reinterpret_cast<const uint4 *>(src);
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
    for (int j = 0; j < 3; ++j) {
        const uint32_t c = lane + 64u * j;
        if (c < 136u) {
            const uint32_t hi = c >= 68u, ch = c - 68u * hi;
            uint32_t *dst = rows + (2u * wave + hi) * (DN_ROWS * DN_ROW_BYTES / 4) + ch * 4u;
            dst[0] = rv[j].x; dst[1] = rv[j].y; dst[2] = rv[j].z; dst[3] = rv[j].w;
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
    float4 *dst = reinterpret_cast<float4 *>(act + (kk * DN_NB + b) * DN_BLOCK_STRIDE + l8 * 16u);
#pragma unroll
    for (int j = 0; j < 4; ++j) dst[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
    __syncthreads();

    {   // Unit (expert k, row r, block bb).
        const uint32_t k = tid >> 5, r = (tid >> 2) & 7u, bb = tid & 3u;
        const uint32_t off = k * (DN_ROWS * DN_ROW_BYTES) + r * DN_ROW_BYTES + bb * 34u;
        const uint32_t *w = rows + (off >> 2);
        uint32_t d[9];
#pragma unroll
        for (int j = 0; j < 9; ++j) d[j] = w[j];
        float sc;
        uint32_t q[8];
        tq2_unpack(d, (off & 2u) != 0u, sc, q);
        float s = sc * tq2_block_dot(q, reinterpret_cast<const uint32_t *>(book4),
                                     act + (k * DN_NB + bb) * DN_BLOCK_STRIDE);
        s = s + gd_dpp_f<0xB1>(s);  // b0 + b1, b2 + b3
        s = s + gd_dpp_f<0x4E>(s);  // (b0 + b1) + (b2 + b3)
        if (bb == 0) dk[k][r] = s;
    }
    __syncthreads();
    if (tid < DN_ROWS) {
        cfloat *wts = as_const(gd_buf<const float>(a, a.c[4]) + a.c[5] + t * DN_U);
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < DN_U; ++k) acc += wts[k] * dk[k][tid];
        if (a.c[21]) acc = gd_buf<const float>(a, a.c[22])[a.c[23] + t * E + row0 + tid] + acc;
        gd_buf<float>(a, a.c[13])[a.c[14] + t * E + row0 + tid] = acc;
    }
}
