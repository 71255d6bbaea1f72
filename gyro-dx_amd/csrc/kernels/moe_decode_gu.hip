// Decode path, step 2: routing and the fused TQ2_T dequant-GEMV of the gate and up rows.
//
// Every wave computes the token's top-8 from the router logits (route_fast.h), so no separate
// routing launch exists. A group of eight waves owns 64 rows of one projection (gate or up) of
// one selected expert over one K-part of 8 Gyro blocks (1024 columns). All independent loads
// are issued first: the logits, the codebook, the wave's 128 activations (binary16 pairs in
// scalar registers); once routing names the expert, its rows stream from HBM with 16-byte
// loads into LDS (69 words per row so that lane = row reads are bank-conflict free). Wave w
// decodes block w of its row (32 trellis steps per lane) with two v_dot2_f32_f16 per step;
// codebook pairs come from LDS; the eight partial sums are added in block order. Two groups
// fit a CU, so every SIMD runs two waves.
// Expert e's rows are at base + e * slot_stride (+ proj_bytes for up): no table lookup.
// Grid: x = F / 64, y = 2 * parts (projection-major), z = n_tok * 8; 512 threads.
// Output partials gu[part][slot][proj][F]; the down kernel adds the parts.
// Constants: 0 logits_uav 1 logits_off 2 n_expert 3 n_used (8) 4 scale (fp32 bits) 5 ids_uav
// 6 ids_off 7 weights_uav 8 weights_off 9 xh16_uav 10 xh16_off (words) 11 base_lo 12 base_hi
// 13 slot_stride 14 proj_bytes 15 codebook_srv 16 gu_uav 17 gu_off 18 E 19 F 20 n_tok.
// Requires TQ2_T experts, E a multiple of 1024, n_expert <= 256, top-8 and F a multiple of 64.
#include "gyro_fast.h"
#include "route_fast.h"

#define GU_ROWS 64
#define GU_ROW_WORDS 69  // 272 bytes of a part row + 4 bytes of padding
#define GU_U 8

GD_PIPELINE_NAMED(moe_decode_gu, 512) {
    __shared__ uint4 book4[512];
    __shared__ uint32_t rows[GU_ROWS * GU_ROW_WORDS];
    __shared__ float red[8][GU_ROWS];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t NE = a.c[2], E = a.c[18], F = a.c[19], n_tok = a.c[20];
    const uint32_t slot = blockIdx.z, t = slot / GU_U, k = slot - t * GU_U;
    const uint32_t parts = E / 1024u, proj = blockIdx.y / parts, part = blockIdx.y - proj * parts;
    const uint32_t row0 = blockIdx.x * GU_ROWS;

    // Independent loads first.
    float lv[4];
    rf_load<4>(gd_buf<const float>(a, a.c[0]) + a.c[1] + t * NE, NE, lv);
    const uint4 cbv = gd_buf<const uint4>(a, a.c[15])[tid];
    const uint32_t xblk = __builtin_amdgcn_readfirstlane(part * 8u + wave);
    cuint *x16 = as_const(gd_buf<const uint32_t>(a, a.c[9]) + a.c[10] + t * (E / 2u) + xblk * 64u);
    uint32_t xs[64];
#pragma unroll
    for (int j = 0; j < 64; ++j) xs[j] = x16[j];

    uint32_t ids[GU_U];
    float wts[GU_U];
    wave_route_fast<4, GU_U>(lv, NE, gd_bits_f32(a.c[4]), ids, wts);
    if (blockIdx.x == 0 && blockIdx.y == 0 && k == 0 && wave == 0 && lane < GU_U) {
        uint32_t id = ids[0];
        float w = wts[0];
#pragma unroll
        for (int j = 1; j < GU_U; ++j) {
            id = lane == (uint32_t)j ? ids[j] : id;
            w = lane == (uint32_t)j ? wts[j] : w;
        }
        gd_buf<uint32_t>(a, a.c[5])[a.c[6] + t * GU_U + lane] = id;
        gd_buf<float>(a, a.c[7])[a.c[8] + t * GU_U + lane] = w;
    }
    uint32_t e = ids[0];
#pragma unroll
    for (int j = 1; j < GU_U; ++j) e = k == (uint32_t)j ? ids[j] : e;
    e = e < NE ? e : NE - 1u;  // ids are always < NE for finite logits; never address past the layer

    const uint64_t layer_base = (uint64_t)a.c[11] | ((uint64_t)a.c[12] << 32);
    const uint32_t row_bytes = E / 128u * 34u;
    const uint8_t *base = reinterpret_cast<const uint8_t *>(layer_base) + (uint64_t)e * a.c[13] +
                          (proj ? a.c[14] : 0u) + (uint64_t)row0 * row_bytes + part * 272u;
    // 64 rows x 17 chunks of 16 bytes, three per thread (the last partly), all issued at once.
    uint4 rv[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const uint32_t c = min(tid + 512u * j, GU_ROWS * 17u - 1u);
        const uint32_t r = c / 17u, ch = c - r * 17u;
        rv[j] = *reinterpret_cast<const uint4 *>(base + (size_t)r * row_bytes + ch * 16u);
    }
    book4[tid] = cbv;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const uint32_t c = tid + 512u * j;
        if (c < GU_ROWS * 17u) {
            const uint32_t r = c / 17u, ch = c - r * 17u;
            uint32_t *dst = rows + r * GU_ROW_WORDS + ch * 4u;
            dst[0] = rv[j].x; dst[1] = rv[j].y; dst[2] = rv[j].z; dst[3] = rv[j].w;
        }
    }
    __syncthreads();

    // Block `wave` of the part row: byte offset 34 * wave (word aligned for even waves).
    const uint32_t *rw = rows + lane * GU_ROW_WORDS + (wave * 34u >> 2);
    uint32_t d[9];
#pragma unroll
    for (int j = 0; j < 9; ++j) d[j] = rw[j];
    float sc;
    uint32_t q[8];
    tq2_unpack(d, (wave & 1u) != 0u, sc, q);
    red[wave][lane] = sc * tq2_block_dot_h(q, reinterpret_cast<const uint32_t *>(book4), xs);
    __syncthreads();
    if (wave == 0) {
        float v = red[0][lane];
#pragma unroll
        for (int w = 1; w < 8; ++w) v += red[w][lane];
        const uint32_t n_slots = n_tok * GU_U;
        gd_buf<float>(a, a.c[16])[a.c[17] + ((size_t)(part * n_slots + slot) * 2u + proj) * F + row0 + lane] = v;
    }
}
