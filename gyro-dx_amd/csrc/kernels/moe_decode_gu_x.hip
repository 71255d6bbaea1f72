// Decode path for layers whose experts and projections mix Gyro types, step 2: routing and the
// fused dequant-GEMV of the gate and up rows (src/engine.zig:567-602 with dotRow per matrix,
// src/kernels.zig:201-210), structured as moe_decode_gu: a group of eight waves owns 64 rows of
// one projection of one selected expert over one K-part of 8 Gyro blocks (1024 columns).
// The expert's rows and their type come from the layer's expert table (ExpertDesc); the type is
// uniform per group, so one instantiation of the block decoder runs (gyro_fast.h). The rows
// stream into LDS with 16-byte loads (2 bb + 1 words per row for blocks of bb bytes, so that
// lane = row reads are bank-conflict free); wave w decodes block w of its row.
// Grid: x = F / 64, y = 2 * parts (projection-major), z = n_tok * 8; 512 threads.
// Output partials gu[part][slot][proj][F]; the down kernel adds the parts.
// Constants: 0 logits_uav 1 logits_off 2 n_expert 3 n_used (8) 4 scale (fp32 bits) 5 ids_uav
// 6 ids_off 7 weights_uav 8 weights_off 9 xh16_uav 10 xh16_off (words) 11 xtab_srv
// 12 codebook_srv 13 gu_uav 14 gu_off 15 E 16 F 17 n_tok.
// Requires E a multiple of 1024, n_expert <= 256, top-8 and F a multiple of 64.
#include "gyro_fast.h"
#include "route_fast.h"

#define GX_ROWS 64
#define GX_MAX_ROW_WORDS 117  // 8 blocks of 58 bytes + 1 word of padding
#define GX_U 8

template <int ID>
__device__ __forceinline__ float gx_block(const uint32_t *row, uint32_t wave, const uint32_t *book,
                                          const uint32_t xs[64]) {
    constexpr int BB = GyroT<ID>::BB, NW = gyro_nw<ID>();
    const uint32_t off = wave * BB;  // even
    const uint32_t *rw = row + (off >> 2);
    uint32_t d[NW + 1];
#pragma unroll
    for (int j = 0; j <= NW; ++j) d[j] = rw[j];
    float sc;
    uint32_t w[NW];
    gyro_unpack<ID>(d, (off & 2u) != 0u, sc, w);
    return sc * gyro_block_dot_h<ID>(w, book, xs);
}

GD_PIPELINE_NAMED(moe_decode_gu_x, 512) {
    __shared__ uint4 book4[512];
    __shared__ uint32_t rows[GX_ROWS * GX_MAX_ROW_WORDS];
    __shared__ float red[8][GX_ROWS];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t NE = a.c[2], E = a.c[15], F = a.c[16], n_tok = a.c[17];
    const uint32_t slot = blockIdx.z, t = slot / GX_U, k = slot - t * GX_U;
    const uint32_t parts = E / 1024u, proj = blockIdx.y / parts, part = blockIdx.y - proj * parts;
    const uint32_t row0 = blockIdx.x * GX_ROWS;

    // Independent loads first.
    float lv[4];
    rf_load<4>(gd_buf<const float>(a, a.c[0]) + a.c[1] + t * NE, NE, lv);
    const uint4 cbv = gd_buf<const uint4>(a, a.c[12])[tid];
    const uint32_t xblk = __builtin_amdgcn_readfirstlane(part * 8u + wave);
    cuint *x16 = as_const(gd_buf<const uint32_t>(a, a.c[9]) + a.c[10] + t * (E / 2u) + xblk * 64u);
    uint32_t xs[64];
#pragma unroll
    for (int j = 0; j < 64; ++j) xs[j] = x16[j];

    uint32_t ids[GX_U];
    float wts[GX_U];
    wave_route_fast<4, GX_U>(lv, NE, gd_bits_f32(a.c[4]), ids, wts);
    if (blockIdx.x == 0 && blockIdx.y == 0 && k == 0 && wave == 0 && lane < GX_U) {
        uint32_t id = ids[0];
        float w = wts[0];
#pragma unroll
        for (int j = 1; j < GX_U; ++j) {
            id = lane == (uint32_t)j ? ids[j] : id;
            w = lane == (uint32_t)j ? wts[j] : w;
        }
        gd_buf<uint32_t>(a, a.c[5])[a.c[6] + t * GX_U + lane] = id;
        gd_buf<float>(a, a.c[7])[a.c[8] + t * GX_U + lane] = w;
    }
    uint32_t e = ids[0];
#pragma unroll
    for (int j = 1; j < GX_U; ++j) e = k == (uint32_t)j ? ids[j] : e;
    e = __builtin_amdgcn_readfirstlane(e < NE ? e : NE - 1u);

    const ExpertDesc *xt = gd_buf<const ExpertDesc>(a, a.c[11]);
    const uint32_t types = __builtin_amdgcn_readfirstlane(xt[e].types);
    const uint32_t type_id = (types >> (8u * proj)) & 0xffu;
    GyroType gt;
    if (!gd_type(type_id, gt)) return;  // uniform: the host admits only the eight types
    const uint64_t addr = proj ? xt[e].up : xt[e].gate;
    const uint32_t bb = gt.block_bytes, row_bytes = E / 128u * bb, chunks = bb / 2u, stride = 2u * bb + 1u;
    const uint8_t *base = reinterpret_cast<const uint8_t *>(addr) + (uint64_t)row0 * row_bytes + part * 8u * bb;
    // 64 rows x bb / 2 chunks of 16 bytes, up to four per thread, all issued at once.
    uint4 rv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t c = min(tid + 512u * j, GX_ROWS * chunks - 1u);
        const uint32_t r = c / chunks, ch = c - r * chunks;
        rv[j] = *reinterpret_cast<const uint4 *>(base + (size_t)r * row_bytes + ch * 16u);
    }
    book4[tid] = cbv;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t c = tid + 512u * j;
        if (c < GX_ROWS * chunks) {
            const uint32_t r = c / chunks, ch = c - r * chunks;
            uint32_t *dst = rows + r * stride + ch * 4u;
            dst[0] = rv[j].x; dst[1] = rv[j].y; dst[2] = rv[j].z; dst[3] = rv[j].w;
        }
    }
    __syncthreads();

    const uint32_t *row = rows + lane * stride;
    const uint32_t *book = reinterpret_cast<const uint32_t *>(book4);
    float v = 0.f;
#define GX_CASE(ID) v = gx_block<ID>(row, wave, book, xs)
    GYRO_TYPE_SWITCH(type_id, GX_CASE)
#undef GX_CASE
    red[wave][lane] = v;
    __syncthreads();
    if (wave == 0) {
        float s = red[0][lane];
#pragma unroll
        for (int w = 1; w < 8; ++w) s += red[w][lane];
        const uint32_t n_slots = n_tok * GX_U;
        gd_buf<float>(a, a.c[13])[a.c[14] + ((size_t)(part * n_slots + slot) * 2u + proj) * F + row0 + lane] = s;
    }
}
