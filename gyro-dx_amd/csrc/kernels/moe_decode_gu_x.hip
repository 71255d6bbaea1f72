// Decode path for layers whose experts and projections mix Gyro types, step 2: routing and the
// fused dequant-GEMV of the gate and up rows (src/engine.zig:567-602 with dotRow per matrix,
// src/kernels.zig:201-210), structured as moe_decode_gu: a group of eight waves owns 64 rows of
// one projection of one selected expert over one K-part of 8 Gyro blocks (1024 columns); lane l
// of wave w decodes block l % 8 of row 8 w + l / 8 and the 8-lane groups add their blocks with
// DPP. The expert's rows and their type come from the layer's expert table (ExpertDesc); the
// type is uniform per group, so one instantiation of the block decoder runs (gyro_fast.h), and
// every lane loads its own block straight from HBM as the widest type's 15 words from the block's
// 4-byte-aligned start (the arena's 256 bytes of slack cover the words past a row's last block).
// As in moe_decode_gu, the routing runs as soon as the logits have landed and the blocks are
// loaded before the codebook and activations go through LDS. Two builds of this source, as for
// moe_decode_gu: moe_decode_gu_x (batch 1) copies the block's 128 activations into registers at
// once; moe_decode_gu_xb (batches 2-8) reads them from LDS step by step, with fewer VGPRs, so
// that several groups share a compute unit. Both compute the same products in the same order.
// Grid: x = F / 64, y = 2 * parts (projection-major), z = n_tok * 8; 512 threads.
// Output partials gu[part][slot][proj][F]; the down kernel adds the parts.
// Constants: 0 logits_uav 1 logits_off 2 n_expert 3 n_used (8) 4 scale (fp32 bits) 5 ids_uav
// 6 ids_off 7 w_uav 8 w_off 9 xh_uav (fp32 [n_tok][E]) 10 xh_off (words) 11 xtab_srv 12 codebook_srv 13 gu_uav
// 14 gu_off 15 E 16 F 17 n_tok.
// Requires E a multiple of 1024, n_expert <= 256, top-8 and F a multiple of 64.
#include "gyro_fast.h"
#include "fwht.h"
#include "route_fast.h"

#ifndef GX_PIPELINE
#define GX_PIPELINE moe_decode_gu_x
#define GX_STEPWISE 0  // 1: the block dot reads the activations from LDS step by step
#endif
#define GX_DEFINE(NAME, WG) GD_PIPELINE_NAMED(NAME, WG)  // expands NAME before it is named
#define GX_ROWS 64
#define GX_U 8

// A block of type ID from the words d (its 4-byte-aligned start; odd: the block starts 2 bytes
// into d[0]) against the lane's 128 fp32 activations (fp32(codebook) x activation in fp32, as
// src/kernels.zig:185-199 multiplies the decoded fp32 weights; the block scale after the sum).
template <int ID, typename XP>
__device__ __forceinline__ float gx_block(const uint32_t *d, bool odd, const uint32_t *book, XP x) {
    float sc;
    uint32_t w[gyro_nw<ID>()];
    gyro_unpack<ID>(d, odd, sc, w);
    return gd_rounded(sc * gyro_block_dot<ID>(w, book, x));
}

GX_DEFINE(GX_PIPELINE, 512) {
    __shared__ uint4 book4[512];
    __shared__ uint4 xpart[8 * 33];  // the part's 1024 fp32 activations (x33_stage_index order)
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t NE = a.c[2], E = a.c[15], F = a.c[16], n_tok = a.c[17];
    const uint32_t slot = blockIdx.z, t = slot / GX_U, k = slot - t * GX_U;
    const uint32_t parts = E / 1024u, proj = blockIdx.y / parts, part = blockIdx.y - proj * parts;
    const uint32_t row0 = blockIdx.x * GX_ROWS;
    const uint32_t b = lane & 7u, r = wave * 8u + (lane >> 3);  // this lane's block and row

    // Independent loads first, all in flight together (global loads, which no LDS store orders).
    float lv[4];
    rf_load<4>(gd_buf<const float>(a, a.c[0]) + a.c[1] + t * NE, NE, lv);
    __builtin_amdgcn_sched_barrier(0);  // the logits issue first: the routing waits for them only
    const gd_u32x4 cbv = gd_global4(gd_buf<const uint32_t>(a, a.c[12]))[tid];
    // Thread tid stages words 2 tid, 2 tid + 1 of the part (moe_decode_gu's layout).
    gd_guint *xg = gd_global(gd_buf<const uint32_t>(a, a.c[9]) + a.c[10] + t * E + part * 1024u + 2u * tid);
    const uint32_t xw0 = xg[0], xw1 = xg[1];
#if !GX_STEPWISE
    // The expert table's entries of this group's projection, lane l holding experts l + 64 j
    // (row address and types, j < 4): requested with the other inputs, so that routing names the
    // expert and its entry is read from a register instead of a dependent load (the batch build
    // keeps its registers for occupancy and reads the table after routing).
    uint32_t tlo[4], thi[4], tty[4];
    {
        const uint32_t *XT = gd_buf<const uint32_t>(a, a.c[11]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t ex = min(lane + 64u * (uint32_t)j, NE - 1u);
            gd_guint *ent = gd_global(XT + (size_t)ex * (sizeof(ExpertDesc) / 4u));
            tlo[j] = ent[2u * proj];
            thi[j] = ent[2u * proj + 1u];
            tty[j] = ent[6];
        }
    }
#endif

    // Routing to this group's rank k only; the recording group runs every round (moe_decode_gu).
    const bool writer = blockIdx.x == 0 && blockIdx.y == 0 && k == 0;
    uint64_t key[4];
    rf_init<4>(lv, NE, key);
    uint32_t ids[GX_U], e = 0;
    float top[GX_U];
#pragma unroll
    for (int j = 0; j < GX_U; ++j) {
        if ((uint32_t)j <= k || writer) {  // uniform
            ids[j] = rf_next<4>(key, top[j]);
            if ((uint32_t)j == k) e = ids[j];
        }
    }
    e = __builtin_amdgcn_readfirstlane(e < NE ? e : NE - 1u);
    if (writer && wave == 0u) {
        float wts[GX_U];
        rf_weights<GX_U>(top, gd_bits_f32(a.c[4]), wts);
        if (lane < GX_U) {
            uint32_t id = ids[0];
            float wv = wts[0];
#pragma unroll
            for (int j = 1; j < GX_U; ++j) {
                id = lane == (uint32_t)j ? ids[j] : id;
                wv = lane == (uint32_t)j ? wts[j] : wv;
            }
            gd_buf<uint32_t>(a, a.c[5])[a.c[6] + t * GX_U + lane] = id;
            gd_buf<float>(a, a.c[7])[a.c[8] + t * GX_U + lane] = wv;
        }
    }

#if GX_STEPWISE
    const ExpertDesc *xt = gd_buf<const ExpertDesc>(a, a.c[11]);
    const uint32_t types = __builtin_amdgcn_readfirstlane(xt[e].types);
    const uint64_t addr = proj ? xt[e].up : xt[e].gate;
#else
    const uint32_t ej = e >> 6, el = e & 63u;  // uniform
    uint32_t vlo = tlo[0], vhi = thi[0], vty = tty[0];
#pragma unroll
    for (int j = 1; j < 4; ++j)
        if (ej == (uint32_t)j) {
            vlo = tlo[j];
            vhi = thi[j];
            vty = tty[j];
        }
    const uint32_t types = (uint32_t)__builtin_amdgcn_readlane((int)vty, (int)el);
    const uint64_t addr = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)vhi, (int)el) << 32) |
                          (uint32_t)__builtin_amdgcn_readlane((int)vlo, (int)el);
#endif
    const uint32_t type_id = (types >> (8u * proj)) & 0xffu;
    GyroType gt;
    if (!gd_type(type_id, gt)) return;  // uniform: the host admits only the eight types
    const uint32_t bb = gt.block_bytes, row_bytes = E / 128u * bb;
    const uint8_t *row = reinterpret_cast<const uint8_t *>(addr) + (uint64_t)(row0 + r) * row_bytes + part * 8u * bb;
    const uint32_t off = b * bb;  // even
    gd_guint *rw = gd_global(reinterpret_cast<const uint32_t *>(row + (off & ~3u)));
    uint32_t d[15];
#pragma unroll
    for (int j = 0; j < 15; ++j) d[j] = rw[j];
    // Codebook and activations through LDS while the blocks are in flight.
    reinterpret_cast<gd_u32x4 *>(book4)[tid] = cbv;
    uint32_t *xst = reinterpret_cast<uint32_t *>(xpart) + x33_stage_index(tid >> 6, (tid >> 1) & 31u) * 4u + 2u * (tid & 1u);
    xst[0] = xw0;
    xst[1] = xw1;
    __syncthreads();
#if GX_STEPWISE
    const float *xf = reinterpret_cast<const float *>(xpart + b * 33u);
#else
    float xf[128];
    x33_from_lds(xpart + b * 33u, xf);
#endif
    const uint32_t *book = reinterpret_cast<const uint32_t *>(book4);
    float v = 0.f;
#define GX_CASE(ID) v = gx_block<ID>(d, (off & 2u) != 0u, book, xf)
    GYRO_TYPE_SWITCH(type_id, GX_CASE)
#undef GX_CASE
    v = v + gd_dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]: + lane ^ 1
    v = v + gd_dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]: + lane ^ 2
    v = v + gd_dpp_f<0x104>(v);  // row_shl:4: + lane + 4 (read by lanes b < 4)
    if (b == 0u) {
        const uint32_t n_slots = n_tok * GX_U;
        gd_buf<float>(a, a.c[13])[a.c[14] + ((size_t)(part * n_slots + slot) * 2u + proj) * F + row0 + r] = v;
    }
}
