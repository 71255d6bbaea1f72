// Decode path, step 3: SwiGLU and the down-input rotation, the fused TQ2_T dequant-GEMV of the
// down rows, and the route-weighted combine (src/engine.zig:603-641), with no communication
// between groups.
//
// A group owns 8 output rows of one token for all n_used experts, so the combine is local and
// summed in k order. It first streams the 8 down rows of every selected expert from HBM into
// LDS; meanwhile wave w forms the down input a = H_128(s_down * silu(g) * u) of experts 2w and
// 2w+1 from the gate/up partials (an 8-lane group transforms one 128-block, 16 values per lane:
// stages 1, 2, 4 across lanes with DPP, 8..64 in registers, the butterfly order of
// src/gyro.zig:152-172). Each (expert, row, block) unit is then decoded by one lane; the four
// block sums of a row are added in order; lane 0..7 combine the experts.
// Grid: x = E / 8, y = n_tok; 256 threads.
// Constants: 0 gu_uav 1 gu_off 2 ids_uav 3 ids_off 4 weights_uav 5 weights_off 6 base_lo
// 7 base_hi 8 slot_stride 9 down_off (bytes from an expert's bundle start) 10 codebook_srv
// 11 signs_srv (0xffffffff: none) 12 signs_off 13 out_uav 14 out_off 15 E 16 F 17 n_used
// 18 n_tok 19 parts 20 n_expert.
// Requires TQ2_T experts, n_used == 8 and F == 512.
#include "gyro_fast.h"

#define DN_ROWS 8
#define DN_U 8
#define DN_F 512
#define DN_NB (DN_F / 128)
#define DN_ROW_BYTES (DN_NB * 34)
#define DN_BLOCK_STRIDE 132  // floats per 128-block in LDS (bank spread for the 8 x streams)

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return gd_bits_f32((uint32_t)__builtin_amdgcn_update_dpp(0, (int)gd_f32_bits(v), CTRL, 0xf, 0xf, true));
}

GD_PIPELINE(256) {
    __shared__ uint32_t book[2048];
    __shared__ uint32_t rows[DN_U * DN_ROWS * DN_ROW_BYTES / 4];
    __shared__ float act[DN_U * DN_NB * DN_BLOCK_STRIDE];
    __shared__ float dk[DN_U][DN_ROWS];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t E = a.c[15], U = a.c[17], n_tok = a.c[18], parts = a.c[19], NE = a.c[20];
    const uint32_t t = blockIdx.y, row0 = blockIdx.x * DN_ROWS;
    const uint32_t n_slots = n_tok * U;
    const uint32_t *ids = gd_buf<const uint32_t>(a, a.c[2]) + a.c[3] + t * U;
    const float *wts = gd_buf<const float>(a, a.c[4]) + a.c[5] + t * U;
    const uint64_t layer_base = (uint64_t)a.c[6] | ((uint64_t)a.c[7] << 32);

    // Down rows row0..row0+7 of every selected expert: 8 x 1088 contiguous bytes.
    for (uint32_t c = tid; c < DN_U * 68u; c += 256u) {
        const uint32_t k = c / 68u, ch = c - k * 68u;
        uint32_t e = ids[k];
        e = e < NE ? e : NE - 1u;
        const uint8_t *src = reinterpret_cast<const uint8_t *>(layer_base) + (uint64_t)e * a.c[8] + a.c[9] +
                             (size_t)row0 * DN_ROW_BYTES + ch * 16u;
        const uint4 v = *reinterpret_cast<const uint4 *>(src);
        uint32_t *dst = rows + k * (DN_ROWS * DN_ROW_BYTES / 4) + ch * 4u;
        dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
    }
    const uint32_t *cb = gd_buf<const uint32_t>(a, a.c[10]);
    for (uint32_t i = tid; i < 2048u; i += 256u) book[i] = cb[i];

    {   // Down input of expert kk = 2 * wave + lane / 32, block b = (lane / 8) % 4.
        const uint32_t kk = wave * 2u + (lane >> 5), b = (lane >> 3) & 3u, l8 = lane & 7u;
        const uint32_t slot = t * U + kk;
        const float *GU = gd_buf<const float>(a, a.c[0]) + a.c[1];
        const float *S = a.c[11] != 0xffffffffu ? gd_buf<const float>(a, a.c[11]) + a.c[12] : nullptr;
        float v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t i = b * 128u + l8 + 8u * j;
            float g = 0.f, u = 0.f;
            for (uint32_t p = 0; p < parts; ++p) {
                const float *gp = GU + ((size_t)(p * n_slots + slot) * 2u) * DN_F;
                g += gp[i];
                u += gp[DN_F + i];
            }
            v[j] = gd_silu(g) * u;
            if (S) v[j] *= S[i];
        }
        if (S) {
            // Widths 1, 2, 4: partners are lanes l8 ^ 1, ^ 2, ^ 4 of the 8-lane group.
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float p1 = dpp_f<0xB1>(v[j]);  // quad_perm [1,0,3,2]
                v[j] = (l8 & 1u) ? p1 - v[j] : v[j] + p1;
            }
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float p2 = dpp_f<0x4E>(v[j]);  // quad_perm [2,3,0,1]
                v[j] = (l8 & 2u) ? p2 - v[j] : v[j] + p2;
            }
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float up4 = dpp_f<0x104>(v[j]);   // row_shl:4, lane + 4
                const float dn4 = dpp_f<0x114>(v[j]);   // row_shr:4, lane - 4
                v[j] = (l8 & 4u) ? dn4 - v[j] : v[j] + up4;
            }
            // Widths 8..64: element bits 3..6 are the register index bits 0..3.
#pragma unroll
            for (int w = 1; w < 16; w <<= 1)
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    if (!(j & w)) {
                        const float lo = v[j], hi = v[j + w];
                        v[j] = lo + hi;
                        v[j + w] = lo - hi;
                    }
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] *= GD_INV_SQRT128;
        }
        float *dst = act + (kk * DN_NB + b) * DN_BLOCK_STRIDE + l8;
#pragma unroll
        for (int j = 0; j < 16; ++j) dst[8 * j] = v[j];
    }
    __syncthreads();

    {   // Unit (expert k, row r, block b).
        const uint32_t k = tid >> 5, r = (tid >> 2) & 7u, b = tid & 3u;
        const uint32_t off = k * (DN_ROWS * DN_ROW_BYTES) + r * DN_ROW_BYTES + b * 34u;
        const uint32_t *w = rows + (off >> 2);
        uint32_t d[9];
#pragma unroll
        for (int j = 0; j < 9; ++j) d[j] = w[j];
        float sc;
        uint32_t q[8];
        tq2_unpack(d, (off & 2u) != 0u, sc, q);
        float s = sc * tq2_block_dot(q, book, act + (k * DN_NB + b) * DN_BLOCK_STRIDE);
        s = s + dpp_f<0xB1>(s);  // b0 + b1, b2 + b3
        s = s + dpp_f<0x4E>(s);  // (b0 + b1) + (b2 + b3)
        if (b == 0) dk[k][r] = s;
    }
    __syncthreads();
    if (tid < DN_ROWS) {
        float acc = 0.f;
        for (uint32_t k = 0; k < DN_U; ++k) acc += wts[k] * dk[k][tid];
        gd_buf<float>(a, a.c[13])[a.c[14] + t * E + row0 + tid] = acc;
    }
}
