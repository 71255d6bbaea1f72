// Decode path, step 2, for the shapes moe_decode_gu does not take (hidden not a multiple of
// 1024, F other than 512, top-U other than 8): routing and the fused TQ2_T dequant-GEMV of the
// gate and up rows with the SwiGLU (src/engine.zig:567-606 without the down rotation).
//
// The n_tok x n_used x F output rows (token, slot, row) are cut into runs of RPG consecutive
// rows, one run per group, so one launch round covers a token on the whole GPU whatever the
// shape (RPG <= F: a run touches at most two slots and two tokens).
//  - Independent loads first: each token's logits, the codebook and each token's rotated input
//    (fp32, staged in LDS with block b's 16-byte chunk c at b * 32 + (c + b) % 32).
//  - Routing (route_fast.h, unrolled rounds): wave 0 selects the first token's experts up to the
//    last rank the run needs, wave 1 the second token's; a group whose run holds a token's first
//    row runs all rounds for that token and stores its ids and weights.
//  - Item (row, block), up to GG_ITEMS per thread: the row's gate and up blocks, each loaded
//    straight from HBM (9 words each) and decoded against the block's 128 fp32 activations, read
//    once from LDS for both (tq2_block_dot: fp32(codebook) x activation accumulated in fp32, as
//    src/kernels.zig:161-199); each row's gate and up sums in block order through LDS.
//  - act[(t n_used + k) F + f] = silu(g) * u.
// Expert e's rows are at base + e * slot_stride (+ proj_bytes for up): no table lookup.
// Grid: ceil(n_tok n_used F / RPG) groups; 512 threads.
// Constants: 0 logits_uav 1 logits_off 2 n_expert 3 n_used 4 scale (fp32 bits) 5 ids_uav
// 6 ids_off 7 weights_uav 8 weights_off 9 xh_uav (fp32 [n_tok][E]) 10 xh_off (words) 11 base_lo 12 base_hi
// 13 slot_stride 14 proj_bytes 15 codebook_srv 16 act_uav 17 act_off 18 E 19 F 20 n_tok 21 RPG
// (22 xtab_srv: the generic form).
// Requires TQ2_T experts (any types in the generic form), E a multiple of 256 up to 4096,
// n_expert <= 256, 1 <= n_used <= 16,
// F a multiple of 128, RPG <= F and RPG E / 128 <= 512 GG_ITEMS (the host checks).
#include "gyro_fast.h"
#include "fwht.h"
#include "route_fast.h"

#define GG_ITEMS 2       // (row, block) items per thread
#define GG_MAX_U 16
#define GG_MAX_RPG 512   // RPG E / 128 <= 1024 items
#ifndef GG_PIPELINE
#define GG_PIPELINE moe_decode_gu_g
#define GG_GENERIC 0     // 1: any Gyro type per expert and projection, rows from the expert table
#endif
// Words loaded per block: TQ2_T's 34 bytes, or the widest type's 58 (whole words from the
// block's first byte rounded down to a word; the arena's slack covers reads past the last row).
#define GG_WORDS (GG_GENERIC ? 15 : 9)
#define GG_DEFINE(NAME, WG) GD_PIPELINE_NAMED(NAME, WG)  // expands NAME before it is named

// Selection rounds 0 .. need of one token (uniform per wave): the ids of ranks ka and kb; when
// `writer`, every round and the token's ids and renormalised weights (rf_weights) stored by
// lanes 0 .. U - 1.
__device__ __forceinline__ void gg_route(const float lv[4], uint32_t NE, uint32_t U, uint32_t need, uint32_t ka,
                                         uint32_t kb, bool writer, float scale, uint32_t *ids_out, float *w_out,
                                         uint32_t &ida, uint32_t &idb) {
    const uint32_t lane = threadIdx.x & 63u;
    uint64_t key[4];
    rf_init<4>(lv, NE, key);
    uint32_t ids[GG_MAX_U];
    float top[GG_MAX_U];
    ida = idb = 0u;
#pragma unroll
    for (int k = 0; k < GG_MAX_U; ++k) {
        ids[k] = 0u;
        top[k] = 0.f;
        if ((uint32_t)k < U && ((uint32_t)k <= need || writer)) {  // uniform
            ids[k] = rf_next<4>(key, top[k]);
            if ((uint32_t)k == ka) ida = ids[k];
            if ((uint32_t)k == kb) idb = ids[k];
        }
    }
    if (!writer) return;
    float wts[GG_MAX_U], total = 0.f;
#pragma unroll
    for (int k = 0; k < GG_MAX_U; ++k) {
        wts[k] = 0.f;
        if ((uint32_t)k < U) {
            wts[k] = expf(top[k] - top[0]);
            total += wts[k];
        }
    }
    const float inv = 1.0f / total;
    uint32_t id = ids[0];
    float w = wts[0];
#pragma unroll
    for (int k = 1; k < GG_MAX_U; ++k) {
        id = lane == (uint32_t)k ? ids[k] : id;
        w = lane == (uint32_t)k ? wts[k] : w;
    }
    w *= inv;
    if (scale != 0.f && scale != 1.f) w *= scale;
    if (lane < U) {
        ids_out[lane] = id;
        w_out[lane] = w;
    }
}

GG_DEFINE(GG_PIPELINE, 512) {
    __shared__ gd_u32x4 book4[512];
#if GG_GENERIC
    __shared__ gd_u32x4 xdesc[2 * 256];  // the expert table: {gate, up}, {down, types, pad} per expert
#endif
    __shared__ uint4 xh4[2][4096 / 4];  // the run's (up to) two tokens' rotated fp32 inputs
    __shared__ float gred[2 * GG_ITEMS * 512];  // (row, projection) block dots
    __shared__ float gsum[2 * GG_MAX_RPG];
    __shared__ uint32_t sid[2];  // experts of the run's first and second slot
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t NE = a.c[2], U = a.c[3], E = a.c[18], F = a.c[19], n_tok = a.c[20], RPG = a.c[21];
    const uint32_t nb = E / 128u, UF = U * F;
    const uint32_t row0 = blockIdx.x * RPG, rows = min(RPG, n_tok * UF - row0);
    const uint32_t s0 = row0 / F, s1 = (row0 + rows - 1u) / F;  // s1 <= s0 + 1
    const uint32_t t0 = s0 / U, t1 = s1 / U, k0 = s0 - t0 * U, k1 = s1 - t1 * U;

    // Independent loads: logits (wave 0: t0, wave 1: t1), codebook, rotated inputs.
    const uint32_t tw = wave == 0u ? t0 : t1;
    float lv[4];
    if (wave < 2u) rf_load<4>(gd_buf<const float>(a, a.c[0]) + a.c[1] + tw * NE, NE, lv);
#if GG_GENERIC
    const gd_u32x4 xdv = gd_global4(gd_buf<const uint32_t>(a, a.c[22]))[min(tid, 2u * NE - 1u)];
#endif
    book4[tid] = gd_global4(gd_buf<const uint32_t>(a, a.c[15]))[tid];
#if GG_GENERIC
    if (tid < 2u * NE) xdesc[tid] = xdv;
#endif
    const uint32_t *XH = gd_buf<const uint32_t>(a, a.c[9]) + a.c[10];
    for (uint32_t q = tid; q < (t1 != t0 ? 2u : 1u) * (E / 4u); q += 512u) {  // uint4 chunks
        const uint32_t ti = q / (E / 4u), c16 = q - ti * (E / 4u);
        const gd_u32x4 v = gd_global4(XH + (size_t)(ti ? t1 : t0) * E)[c16];
        xh4[ti][x32_stage_index(c16 >> 5, c16 & 31u)] = make_uint4(v[0], v[1], v[2], v[3]);
    }

    // Routing.
    const float scale = gd_bits_f32(a.c[4]);
    uint32_t *ids_out = gd_buf<uint32_t>(a, a.c[5]) + a.c[6];
    float *w_out = gd_buf<float>(a, a.c[7]) + a.c[8];
    if (wave == 0u) {
        const bool writer = row0 % UF == 0u;  // the run holds t0's first row
        const uint32_t need = t1 == t0 ? k1 : k0;
        uint32_t ida, idb;
        gg_route(lv, NE, U, need, k0, k1, writer, scale, ids_out + t0 * U, w_out + t0 * U, ida, idb);
        if (lane == 0) {
            sid[0] = min(ida, NE - 1u);
            if (t1 == t0) sid[1] = min(idb, NE - 1u);
        }
    } else if (wave == 1u && t1 != t0) {  // the run holds t1's first row (k1 == 0)
        uint32_t ida, idb;
        gg_route(lv, NE, U, 0u, k1, k1, true, scale, ids_out + t1 * U, w_out + t1 * U, ida, idb);
        if (lane == 0) sid[1] = min(ida, NE - 1u);
    }
    __syncthreads();

    // Items: row rr of the run and block b (b fastest), the gate and the up block of that row
    // against the same 128 activations: 2 x 9 words from HBM each.
    const uint32_t n_items = rows * nb;
#if !GG_GENERIC
    const uint64_t layer_base = (uint64_t)a.c[11] | ((uint64_t)a.c[12] << 32);
    const uint8_t *LB = reinterpret_cast<const uint8_t *>(layer_base);
    const uint32_t stride = a.c[13], proj_bytes = a.c[14], row_bytes = nb * 34u;
#endif
    uint32_t dw[GG_ITEMS][2][GG_WORDS];
    bool odd[GG_ITEMS][2];
    uint32_t ty[GG_ITEMS][2];
#pragma unroll
    for (int s = 0; s < GG_ITEMS; ++s) {
        const uint32_t j = tid + 512u * (uint32_t)s;
        odd[s][0] = odd[s][1] = false;
        ty[s][0] = ty[s][1] = 144u;
        if (j < n_items) {
            const uint32_t rr = j / nb, b = j - rr * nb;
            const uint32_t R = row0 + rr, f = R % F, e = sid[R / F != s0 ? 1 : 0];
#if GG_GENERIC
            const gd_u32x4 ptr = xdesc[2u * e], tys = xdesc[2u * e + 1u];
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                ty[s][p] = (tys[2] >> (8 * p)) & 0xffu;
                GyroType gt;
                gd_type(ty[s][p], gt);  // the host admits only the eight types
                const uint64_t addr = (((uint64_t)ptr[2 * p + 1] << 32) | ptr[2 * p]) +
                                      ((uint64_t)f * nb + b) * gt.block_bytes;
                gd_guint *w = gd_global(reinterpret_cast<const uint32_t *>(addr & ~uint64_t(3)));
#pragma unroll
                for (int q = 0; q < GG_WORDS; ++q) dw[s][p][q] = w[q];
                odd[s][p] = (addr & 2u) != 0u;
            }
#else
            const uint64_t off = (uint64_t)e * stride + (uint64_t)f * row_bytes + b * 34u;
#pragma unroll
            for (int p = 0; p < 2; ++p) tq2_load_block(LB, off + (p ? proj_bytes : 0u), dw[s][p]);
            odd[s][0] = odd[s][1] = (off & 2u) != 0u;  // proj_bytes is a multiple of 4
#endif
        }
    }
    const uint32_t *book = reinterpret_cast<const uint32_t *>(book4);
#pragma unroll
    for (int s = 0; s < GG_ITEMS; ++s) {
        const uint32_t j = tid + 512u * (uint32_t)s;
        if (j < n_items) {
            const uint32_t rr = j / nb, b = j - rr * nb;
            const uint32_t ti = (row0 + rr) / UF != t0 ? 1u : 0u;
            float xf[128];
            x32_from_lds(xh4[ti], b, xf);
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                float v = 0.f;
#if GG_GENERIC
#define GG_CASE(ID)                                                       \
    {                                                                     \
        float sc;                                                         \
        uint32_t q[gyro_nw<ID>()];                                        \
        gyro_unpack<ID>(dw[s][p], odd[s][p], sc, q);                      \
        v = sc * gyro_block_dot<ID>(q, book, xf);                         \
    }
                GYRO_TYPE_SWITCH(ty[s][p], GG_CASE)
#undef GG_CASE
#else
                float sc;
                uint32_t q[8];
                tq2_unpack(dw[s][p], odd[s][p], sc, q);
                v = sc * tq2_block_dot(q, book, xf);
#endif
                gred[(2u * rr + (uint32_t)p) * nb + b] = v;
            }
        }
    }
    __syncthreads();
    // Row sums in block order (nb <= 32 loads at once), then the SwiGLU.
    for (uint32_t p = tid; p < rows * 2u; p += 512u) {
        const float *src = gred + p * nb;
        float acc = 0.f;
#pragma unroll
        for (uint32_t b = 0; b < 32u; ++b) {
            const float v = src[b < nb ? b : nb - 1u];
            acc += b < nb ? v : 0.f;
        }
        gsum[p] = acc;
    }
    __syncthreads();
    float *act = gd_buf<float>(a, a.c[16]) + a.c[17];
    for (uint32_t rr = tid; rr < rows; rr += 512u) act[row0 + rr] = gd_silu_rcp(gsum[2u * rr]) * gsum[2u * rr + 1u];
}
