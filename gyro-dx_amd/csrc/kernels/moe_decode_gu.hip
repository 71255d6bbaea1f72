// Decode path, step 2: routing and the fused TQ2_T dequant-GEMV of the gate and up rows.
//
// Every wave computes the token's top-8 from the router logits (route_fast.h), so no separate
// routing launch exists. A group of eight waves owns 64 rows of one projection (gate or up) of
// one selected expert over one K-part of 8 Gyro blocks (1024 columns); lane l of wave w decodes
// block l % 8 of row 8 w + l / 8 (32 trellis steps, two codebook pairs per step gathered
// from LDS, four v_fma_mix_f32 per step: fp32(codebook) x fp32 activation, accumulated in fp32 as
// src/kernels.zig:161-183 does) and the 8-lane groups add their blocks with DPP ((b0 + b1) +
// (b2 + b3)) + ((b4 + b5) + (b6 + b7)). The independent loads go first: the logits, the codebook
// and the part's 1024 fp32 activations. Once routing names the expert, every lane loads the 9
// words of its own block straight from HBM; the routing runs as soon as the logits have landed.
// The codebook and the activations then go into LDS while the blocks are in flight (one barrier),
// so the expert blocks' HBM latency overlaps the staging.
// Two builds of this source: moe_decode_gu (batch 1) copies the block's 128 activations into
// registers at once, right after the barrier, so no read of them waits inside the dot (156
// VGPRs: one group per compute unit, which batch 1's 256 groups need anyway); moe_decode_gu_b
// (batches 2-8: 256 groups per token) reads them one half block at a time (64 VGPRs), so that
// up to four groups share a compute unit. Both compute the same products in the same order.
// Expert e's rows are at base + e * slot_stride (+ proj_bytes for up): no table lookup.
// Grid: x = F / 64, y = 2 * parts (projection-major), z = n_tok * 8; 512 threads.
// Output partials gu[part][slot][proj][F]; the down kernel adds the parts.
// Constants: 0 logits_uav 1 logits_off 2 n_expert 3 n_used (8) 4 scale (fp32 bits) 5 ids_uav
// 6 ids_off 7 weights_uav 8 weights_off 9 xh_uav (fp32 [n_tok][E]) 10 xh_off (words) 11 base_lo 12 base_hi
// 13 slot_stride 14 proj_bytes 15 codebook_srv 16 gu_uav 17 gu_off 18 E 19 F 20 n_tok.
// Requires TQ2_T experts, E a multiple of 1024, n_expert <= 256, top-8 and F a multiple of 64.
#include "gyro_fast.h"
#include "fwht.h"
#include "route_fast.h"

#ifndef GU_PIPELINE
#define GU_PIPELINE moe_decode_gu
#define GU_HALVES 0  // 1: the block's activations read into registers one half at a time
#endif
#define GU_DEFINE(NAME, WG) GD_PIPELINE_NAMED(NAME, WG)  // expands NAME before it is named
#define GU_ROWS 64
#define GU_U 8

GU_DEFINE(GU_PIPELINE, 512) {
    __shared__ uint4 book4[512];
    __shared__ uint4 xpart[8 * 33];  // the part's 1024 fp32 activations (x33_stage_index order)
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t NE = a.c[2], E = a.c[18], F = a.c[19], n_tok = a.c[20];
    const uint32_t slot = blockIdx.z, t = slot / GU_U, k = slot - t * GU_U;
    const uint32_t parts = E / 1024u, proj = blockIdx.y / parts, part = blockIdx.y - proj * parts;
    const uint32_t row0 = blockIdx.x * GU_ROWS;
    const uint32_t b = lane & 7u, r = wave * 8u + (lane >> 3);  // this lane's block and row

    // Independent loads first, all in flight together (global loads, which no LDS store orders).
    float lv[4];
    rf_load<4>(gd_buf<const float>(a, a.c[0]) + a.c[1] + t * NE, NE, lv);
    __builtin_amdgcn_sched_barrier(0);  // the logits issue first: the routing waits for them only
    const gd_u32x4 cbv = gd_global4(gd_buf<const uint32_t>(a, a.c[15]))[tid];
    // Thread tid stages words 2 tid, 2 tid + 1 of the part: half (tid & 1) of chunk (tid >> 1) % 32
    // of block tid / 64.
    gd_guint *xg = gd_global(gd_buf<const uint32_t>(a, a.c[9]) + a.c[10] + t * E + part * 1024u + 2u * tid);
    const uint32_t xw0 = xg[0], xw1 = xg[1];

    // Routing: this group needs the expert of rank k only, so it stops after round k; the one
    // group that records the token's ids and weights runs all rounds and forms the weights once
    // its own weight loads are in flight.
    const bool writer = blockIdx.x == 0 && blockIdx.y == 0 && k == 0;
    uint64_t key[4];
    rf_init<4>(lv, NE, key);
    uint32_t ids[GU_U], e = 0;
    float top[GU_U];
#pragma unroll
    for (int j = 0; j < GU_U; ++j) {
        if ((uint32_t)j <= k || writer) {  // uniform
            ids[j] = rf_next<4>(key, top[j]);
            if ((uint32_t)j == k) e = ids[j];
        }
    }
    e = e < NE ? e : NE - 1u;  // ids are always < NE for finite logits; never address past the layer

    // Block b of row r of the part: 34 bytes at byte 34 b of the part (word aligned for even b),
    // read as the 9 words from its 4-byte-aligned start.
    const uint64_t layer_base = (uint64_t)a.c[11] | ((uint64_t)a.c[12] << 32);
    const uint32_t row_bytes = E / 128u * 34u;
    gd_guint *w = gd_global(reinterpret_cast<const uint32_t *>(
        reinterpret_cast<const uint8_t *>(layer_base) + (uint64_t)e * a.c[13] + (proj ? a.c[14] : 0u) +
        (uint64_t)(row0 + r) * row_bytes + part * 272u + ((b * 34u) & ~3u)));
    uint32_t d[9];
#pragma unroll
    for (int j = 0; j < 9; ++j) d[j] = w[j];
    // Codebook and activations through LDS while the blocks are in flight.
    reinterpret_cast<gd_u32x4 *>(book4)[tid] = cbv;
    uint32_t *xst = reinterpret_cast<uint32_t *>(xpart) + x33_stage_index(tid >> 6, (tid >> 1) & 31u) * 4u + 2u * (tid & 1u);
    xst[0] = xw0;
    xst[1] = xw1;
    __syncthreads();
#if !GU_HALVES
    float xf[128];
    x33_from_lds(xpart + b * 33u, xf);
#endif
    if (writer && wave == 0u) {
        float wts[GU_U];
        rf_weights<GU_U>(top, gd_bits_f32(a.c[4]), wts);
        if (lane < GU_U) {
            uint32_t id = ids[0];
            float wv = wts[0];
#pragma unroll
            for (int j = 1; j < GU_U; ++j) {
                id = lane == (uint32_t)j ? ids[j] : id;
                wv = lane == (uint32_t)j ? wts[j] : wv;
            }
            gd_buf<uint32_t>(a, a.c[5])[a.c[6] + t * GU_U + lane] = id;
            gd_buf<float>(a, a.c[7])[a.c[8] + t * GU_U + lane] = wv;
        }
    }
    float sc;
    uint32_t q[8];
    tq2_unpack(d, (b & 1u) != 0u, sc, q);
    const uint32_t *book = reinterpret_cast<const uint32_t *>(book4);
#if GU_HALVES
    float v = gd_rounded(sc * tq2_block_dot_halves(q, book, xpart + b * 33u));
#else
    float v = gd_rounded(sc * tq2_block_dot(q, book, xf));
#endif
    v = v + gd_dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]: + lane ^ 1
    v = v + gd_dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]: + lane ^ 2
    v = v + gd_dpp_f<0x104>(v);  // row_shl:4: + lane + 4 (read by lanes b < 4)
    if (b == 0u) {
        const uint32_t n_slots = n_tok * GU_U;
        gd_buf<float>(a, a.c[16])[a.c[17] + ((size_t)(part * n_slots + slot) * 2u + proj) * F + row0 + r] = v;
    }
}
