// Decode path, step 2, for the shapes moe_decode_gu does not take (hidden not a multiple of
// 1024, top-U other than 8): routing and the fused TQ2_T dequant-GEMV of the gate and up rows,
// as moe_decode_gu, with a partial last K-part and a runtime expert count.
//
// Every wave computes the token's top-U from the router logits (route_fast.h), so no separate
// routing launch exists. A group of eight waves owns 64 rows of one projection (gate or up) of
// one selected expert over one K-part of up to 8 Gyro blocks (1024 columns); lane l of wave w decodes
// block l % 8 of row 8 w + l / 8 (32 trellis steps, two v_dot2_f32_f16 per step, codebook pairs
// from LDS) and the 8-lane groups add their blocks with DPP ((b0 + b1) + (b2 + b3)) +
// ((b4 + b5) + (b6 + b7)). The independent loads go first: the logits, the codebook and the
// part's 1024 binary16 activations (both into LDS, one barrier, then each lane keeps its block's
// 128 activations in registers). Once routing names the expert, every lane loads the 9 words of
// its own block straight from HBM, so no further barrier is needed.
// Expert e's rows are at base + e * slot_stride (+ proj_bytes for up): no table lookup.
// Grid: x = F / 64, y = 2 * parts (projection-major, parts = ceil(E / 1024); the last part
// holds the E / 128 - 8 (parts - 1) remaining blocks), z = n_tok * n_used; 512 threads.
// Output partials gu[part][slot][proj][F]; the down kernel adds the parts.
// Constants: 0 logits_uav 1 logits_off 2 n_expert 3 n_used (8) 4 scale (fp32 bits) 5 ids_uav
// 6 ids_off 7 weights_uav 8 weights_off 9 xh16_uav 10 xh16_off (words) 11 base_lo 12 base_hi
// 13 slot_stride 14 proj_bytes 15 codebook_srv 16 gu_uav 17 gu_off 18 E 19 F 20 n_tok.
// Requires TQ2_T experts, E a multiple of 256, n_expert <= 256, 1 <= n_used <= 16 and F a
// multiple of 64.
#include "gyro_fast.h"
#include "fwht.h"
#include "route_fast.h"

#define GU_ROWS 64
#define GU_MAX_U 16

GD_PIPELINE_NAMED(moe_decode_gu_g, 512) {
    __shared__ uint4 book4[512];
    __shared__ uint4 xpart[128];  // the part's 1024 activations as binary16 pairs
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t NE = a.c[2], U = a.c[3], E = a.c[18], F = a.c[19], n_tok = a.c[20];
    const uint32_t slot = blockIdx.z, t = slot / U, k = slot - t * U;
    const uint32_t parts = (E + 1023u) / 1024u, proj = blockIdx.y / parts, part = blockIdx.y - proj * parts;
    const uint32_t nbp = min(8u, E / 128u - part * 8u);  // blocks of this part
    const uint32_t row0 = blockIdx.x * GU_ROWS;
    const uint32_t b = lane & 7u, r = wave * 8u + (lane >> 3);  // this lane's block and row

    // Independent loads first, all in flight together (global loads, which no LDS store orders).
    float lv[4];
    rf_load<4>(gd_buf<const float>(a, a.c[0]) + a.c[1] + t * NE, NE, lv);
    const gd_u32x4 cbv = gd_global4(gd_buf<const uint32_t>(a, a.c[15]))[tid];
    const uint32_t xw = tid < nbp * 64u ? gd_global(gd_buf<const uint32_t>(a, a.c[9]) + a.c[10] + t * (E / 2u) + part * 512u)[tid] : 0u;
    reinterpret_cast<gd_u32x4 *>(book4)[tid] = cbv;
    // Chunk c (16 bytes) of block bx at position bx * 16 + (c + bx) % 16: the 8 blocks that a
    // wave reads at one chunk index sit in 8 different bank groups.
    const uint32_t bx = tid >> 6, cx = (tid >> 2) & 15u;
    reinterpret_cast<uint32_t *>(xpart)[(bx * 16u + ((cx + bx) & 15u)) * 4u + (tid & 3u)] = xw;
    __syncthreads();
    uint32_t xs[64];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const uint4 v = xpart[b * 16u + ((j + b) & 15u)];
        xs[4 * j] = v.x; xs[4 * j + 1] = v.y; xs[4 * j + 2] = v.z; xs[4 * j + 3] = v.w;
    }

    // Routing: this group needs the expert of rank k only, so it stops after round k; the one
    // group that records the token's ids and weights runs all rounds and forms the weights once
    // its own weight loads are in flight.
    const bool writer = blockIdx.x == 0 && blockIdx.y == 0 && k == 0;
    uint64_t key[4];
    rf_init<4>(lv, NE, key);
    uint32_t ids[GU_MAX_U], e = 0;
    float top[GU_MAX_U];
#pragma unroll
    for (int j = 0; j < GU_MAX_U; ++j) {
        if ((uint32_t)j < U && ((uint32_t)j <= k || writer)) {  // uniform
            ids[j] = rf_next<4>(key, top[j]);
            if ((uint32_t)j == k) e = ids[j];
        }
    }
    e = e < NE ? e : NE - 1u;  // ids are always < NE for finite logits; never address past the layer

    // Block b of row r of the part: 34 bytes at byte 34 b of the part (word aligned for even b),
    // read as the 9 words from its 4-byte-aligned start.
    const uint64_t layer_base = (uint64_t)a.c[11] | ((uint64_t)a.c[12] << 32);
    const uint32_t row_bytes = E / 128u * 34u;
    // Lanes past the last part's blocks contribute zero; their address stays on block 0.
    const bool live = b < nbp;
    gd_guint *w = gd_global(reinterpret_cast<const uint32_t *>(
        reinterpret_cast<const uint8_t *>(layer_base) + (uint64_t)e * a.c[13] + (proj ? a.c[14] : 0u) +
        (uint64_t)(row0 + r) * row_bytes + part * 272u + (((live ? b : 0u) * 34u) & ~3u)));
    uint32_t d[9];
#pragma unroll
    for (int j = 0; j < 9; ++j) d[j] = w[j];
    if (writer && wave == 0u) {
        // Softmax over the selected logits in rank order, times the scale unless it is 0 or 1.
        float wts[GU_MAX_U], total = 0.f;
#pragma unroll
        for (int j = 0; j < GU_MAX_U; ++j)
            if ((uint32_t)j < U) {
                wts[j] = expf(top[j] - top[0]);
                total += wts[j];
            }
        const float inv = 1.0f / total, scale = gd_bits_f32(a.c[4]);
        if (lane < U) {
            uint32_t id = ids[0];
            float wv = wts[0];
#pragma unroll
            for (int j = 1; j < GU_MAX_U; ++j) {
                if ((uint32_t)j >= U) break;
                id = lane == (uint32_t)j ? ids[j] : id;
                wv = lane == (uint32_t)j ? wts[j] : wv;
            }
            wv *= inv;
            if (scale != 0.f && scale != 1.f) wv *= scale;
            gd_buf<uint32_t>(a, a.c[5])[a.c[6] + t * U + lane] = id;
            gd_buf<float>(a, a.c[7])[a.c[8] + t * U + lane] = wv;
        }
    }
    float sc;
    uint32_t q[8];
    tq2_unpack(d, (b & 1u) != 0u, sc, q);
    float v = live ? sc * tq2_block_dot_h(q, reinterpret_cast<const uint32_t *>(book4), xs) : 0.f;
    v = v + gd_dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]: + lane ^ 1
    v = v + gd_dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]: + lane ^ 2
    v = v + gd_dpp_f<0x104>(v);  // row_shl:4: + lane + 4 (read by lanes b < 4)
    if (b == 0u) {
        const uint32_t n_slots = n_tok * U;
        gd_buf<float>(a, a.c[16])[a.c[17] + ((size_t)(part * n_slots + slot) * 2u + proj) * F + row0 + r] = v;
    }
}
