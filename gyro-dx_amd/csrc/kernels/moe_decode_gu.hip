// Decode path, step 2: routing and the fused TQ2_T dequant-GEMV of the gate and up rows.
//
// Every wave computes the token's top-k from the router logits (route_fast.h), so no separate
// routing launch exists. A group of eight waves owns 64 rows of one projection (gate or up) of
// one selected expert over one K-part of 8 Gyro blocks (1024 columns): the rows stream from
// HBM with 16-byte loads into LDS (69 words per row so that lane = row reads are bank-conflict
// free); wave w decodes block w of its row (32 trellis steps per lane) against activations that
// are uniform across the wave (scalar loads); codebook pairs come from LDS; the eight partial
// sums are added in block order. Two groups fit a CU, so every SIMD runs two waves.
// Expert e's rows are at base + e * slot_stride (+ proj_bytes for up): no table lookup.
// Grid: x = F / 64, y = 2 * parts (projection-major), z = n_tok * n_used; 512 threads.
// Output partials gu[part][slot][proj][F]; the down kernel adds the parts.
// Constants: 0 logits_uav 1 logits_off 2 n_expert 3 n_used 4 scale (fp32 bits) 5 ids_uav
// 6 ids_off 7 weights_uav 8 weights_off 9 xh_uav 10 xh_off 11 base_lo 12 base_hi
// 13 slot_stride 14 proj_bytes 15 codebook_srv 16 gu_uav 17 gu_off 18 E 19 F 20 n_tok.
// Requires TQ2_T experts, E a multiple of 1024, n_expert <= 256 and F a multiple of 64.
#include "gyro_fast.h"
#include "route_fast.h"

#define GU_ROWS 64
#define GU_ROW_WORDS 69  // 272 bytes of a part row + 4 bytes of padding

GD_PIPELINE(512) {
    __shared__ uint32_t book[2048];
    __shared__ uint32_t rows[GU_ROWS * GU_ROW_WORDS];
    __shared__ float red[8][GU_ROWS];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t NE = a.c[2], U = a.c[3], E = a.c[18], F = a.c[19], n_tok = a.c[20];
    const uint32_t slot = blockIdx.z, t = slot / U, k = slot - t * U;
    const uint32_t parts = E / 1024u, proj = blockIdx.y / parts, part = blockIdx.y - proj * parts;
    const uint32_t row0 = blockIdx.x * GU_ROWS;

    const uint32_t *cb = gd_buf<const uint32_t>(a, a.c[15]);
    for (uint32_t i = tid; i < 2048u; i += 512u) book[i] = cb[i];

    uint32_t ids[RF_MAX_USED];
    float wts[RF_MAX_USED];
    wave_route_fast<4>(gd_buf<const float>(a, a.c[0]) + a.c[1] + t * NE, NE, U, gd_bits_f32(a.c[4]), ids, wts);
    if (blockIdx.x == 0 && blockIdx.y == 0 && k == 0 && wave == 0 && lane < U) {
        uint32_t id = 0;
        float w = 0.f;
        for (uint32_t j = 0; j < RF_MAX_USED; ++j)
            if (j == lane) {
                id = ids[j];
                w = wts[j];
            }
        gd_buf<uint32_t>(a, a.c[5])[a.c[6] + t * U + lane] = id;
        gd_buf<float>(a, a.c[7])[a.c[8] + t * U + lane] = w;
    }
    uint32_t e = 0;
    for (uint32_t j = 0; j < RF_MAX_USED; ++j)
        if (j == k) e = ids[j];
    e = __builtin_amdgcn_readfirstlane(e);
    e = e < NE ? e : NE - 1u;  // ids are always < NE for finite logits; never address past the layer

    const uint64_t layer_base = (uint64_t)a.c[11] | ((uint64_t)a.c[12] << 32);
    const uint32_t row_bytes = E / 128u * 34u;
    const uint8_t *base = reinterpret_cast<const uint8_t *>(layer_base) + (uint64_t)e * a.c[13] +
                          (proj ? a.c[14] : 0u) + (uint64_t)row0 * row_bytes + part * 272u;
    for (uint32_t c = tid; c < GU_ROWS * 17u; c += 512u) {
        const uint32_t r = c / 17u, ch = c - r * 17u;
        const uint4 v = *reinterpret_cast<const uint4 *>(base + (size_t)r * row_bytes + ch * 16u);
        uint32_t *dst = rows + r * GU_ROW_WORDS + ch * 4u;
        dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
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
    const uint32_t xblk = __builtin_amdgcn_readfirstlane(part * 8u + wave);
    cfloat *xh = as_const(gd_buf<const float>(a, a.c[9]) + a.c[10] + t * E + xblk * 128u);
    red[wave][lane] = sc * tq2_block_dot(q, book, xh);
    __syncthreads();
    if (wave == 0) {
        float v = red[0][lane];
#pragma unroll
        for (int w = 1; w < 8; ++w) v += red[w][lane];
        const uint32_t n_slots = n_tok * U;
        gd_buf<float>(a, a.c[16])[a.c[17] + ((size_t)(part * n_slots + slot) * 2u + proj) * F + row0 + lane] = v;
    }
}
