// Decode path, type-generic gate/up for the shapes moe_decode_gu_x does not take (hidden not a
// multiple of 1024, top-U other than 8): as moe_decode_gu_x, with a partial last K-part (lanes
// past its blocks contribute zero) and a runtime expert count.
// Grid: x = F / 64, y = 2 * parts (parts = ceil(E / 1024)), z = n_tok * n_used; 512 threads.
// Constants: as moe_decode_gu_x (3 n_used).
// Requires E a multiple of 256, n_expert <= 256, 1 <= n_used <= 16 and F a multiple of 64.
#include "gyro_fast.h"
#include "fwht.h"
#include "route_fast.h"

#define GX_ROWS 64
#define GX_MAX_U 16

// Block b of the part row at `row` (bytes): its NW + 1 words from byte (b BB) & ~3, decoded
// against the lane's 128 activations.
template <int ID>
__device__ __forceinline__ float gx_block(const uint8_t *row, uint32_t b, const uint32_t *book, const uint32_t xs[64]) {
    constexpr int BB = GyroT<ID>::BB, NW = gyro_nw<ID>();
    const uint32_t off = b * BB;  // even
    gd_guint *rw = gd_global(reinterpret_cast<const uint32_t *>(row + (off & ~3u)));
    uint32_t d[NW + 1];
#pragma unroll
    for (int j = 0; j <= NW; ++j) d[j] = rw[j];
    float sc;
    uint32_t w[NW];
    gyro_unpack<ID>(d, (off & 2u) != 0u, sc, w);
    return sc * gyro_block_dot_h<ID>(w, book, xs);
}

GD_PIPELINE_NAMED(moe_decode_gu_xg, 512) {
    __shared__ uint4 book4[512];
    __shared__ uint4 xpart[128];  // the part's 1024 activations as binary16 pairs, bank-rotated
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t NE = a.c[2], U = a.c[3], E = a.c[15], F = a.c[16], n_tok = a.c[17];
    const uint32_t slot = blockIdx.z, t = slot / U, k = slot - t * U;
    const uint32_t parts = (E + 1023u) / 1024u, proj = blockIdx.y / parts, part = blockIdx.y - proj * parts;
    const uint32_t nbp = min(8u, E / 128u - part * 8u);  // blocks of this part
    const uint32_t row0 = blockIdx.x * GX_ROWS;
    const uint32_t b = lane & 7u, r = wave * 8u + (lane >> 3);  // this lane's block and row

    // Independent loads first, all in flight together (global loads, which no LDS store orders).
    float lv[4];
    rf_load<4>(gd_buf<const float>(a, a.c[0]) + a.c[1] + t * NE, NE, lv);
    const gd_u32x4 cbv = gd_global4(gd_buf<const uint32_t>(a, a.c[12]))[tid];
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

    // Routing to this group's rank k only; the recording group runs every round (moe_decode_gu).
    const bool writer = blockIdx.x == 0 && blockIdx.y == 0 && k == 0;
    uint64_t key[4];
    rf_init<4>(lv, NE, key);
    uint32_t ids[GX_MAX_U], e = 0;
    float top[GX_MAX_U];
#pragma unroll
    for (int j = 0; j < GX_MAX_U; ++j) {
        if ((uint32_t)j < U && ((uint32_t)j <= k || writer)) {  // uniform
            ids[j] = rf_next<4>(key, top[j]);
            if ((uint32_t)j == k) e = ids[j];
        }
    }
    e = __builtin_amdgcn_readfirstlane(e < NE ? e : NE - 1u);
    if (writer && wave == 0u) {
        // Softmax over the selected logits in rank order, times the scale unless it is 0 or 1.
        float wts[GX_MAX_U], total = 0.f;
#pragma unroll
        for (int j = 0; j < GX_MAX_U; ++j)
            if ((uint32_t)j < U) {
                wts[j] = expf(top[j] - top[0]);
                total += wts[j];
            }
        const float inv = 1.0f / total, scale = gd_bits_f32(a.c[4]);
        if (lane < U) {
            uint32_t id = ids[0];
            float wv = wts[0];
#pragma unroll
            for (int j = 1; j < GX_MAX_U; ++j) {
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

    const ExpertDesc *xt = gd_buf<const ExpertDesc>(a, a.c[11]);
    const uint32_t types = __builtin_amdgcn_readfirstlane(xt[e].types);
    const uint32_t type_id = (types >> (8u * proj)) & 0xffu;
    GyroType gt;
    if (!gd_type(type_id, gt)) return;  // uniform: the host admits only the eight types
    const uint64_t addr = proj ? xt[e].up : xt[e].gate;
    const uint32_t bb = gt.block_bytes, row_bytes = E / 128u * bb;
    const uint8_t *row = reinterpret_cast<const uint8_t *>(addr) + (uint64_t)(row0 + r) * row_bytes + part * 8u * bb;
    const uint32_t *book = reinterpret_cast<const uint32_t *>(book4);
    // Lanes past the last part's blocks contribute zero; their address stays on block 0.
    const bool live = b < nbp;
    float v = 0.f;
#define GX_CASE(ID) v = gx_block<ID>(row, live ? b : 0u, book, xs)
    GYRO_TYPE_SWITCH(type_id, GX_CASE)
#undef GX_CASE
    v = live ? v : 0.f;
    v = v + gd_dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]: + lane ^ 1
    v = v + gd_dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]: + lane ^ 2
    v = v + gd_dpp_f<0x104>(v);  // row_shl:4: + lane + 4 (read by lanes b < 4)
    if (b == 0u) {
        const uint32_t n_slots = n_tok * U;
        gd_buf<float>(a, a.c[13])[a.c[14] + ((size_t)(part * n_slots + slot) * 2u + proj) * F + row0 + r] = v;
    }
}
