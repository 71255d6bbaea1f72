// Decode path, type-generic down for the shapes moe_decode_down_x does not take (F other than
// 512, top-U other than 8, more than two K-parts; no shared expert): SwiGLU and the down-input
// rotation, the fused dequant-GEMV of the down rows and the route-weighted combine
// (src/engine.zig:603-641), structured as moe_decode_down_g with each expert's down rows in
// its own Gyro type (from the layer's expert table) and full-block units.
// (1) Down inputs as moe_decode_down_g.
// (2) Down rows: expert k's 8 rows are one contiguous run of 8 F / 128 blocks of its type
//     (a multiple of 16 bytes), copied to LDS at the prefix of the runs before it.
// (3) Wave w computes output row w: unit (k, bb) decodes block bb of row w of expert k against
//     block bb of a_k; the unit sums go through LDS, lane k < U adds expert k's F / 128 units in
//     block order, and the experts are combined in k order before the residual is added.
// Grid: x = E / 8, y = n_tok; 512 threads.
// Constants (as moe_decode_down_x): 0 gu_uav 1 gu_off 2 ids_uav 3 ids_off 4 weights_uav
// 5 weights_off 6 xtab_srv 7-9 unused 10 codebook_srv 11 signs_srv (0xffffffff: none)
// 12 signs_off 13 out_uav 14 out_off 15 E 16 F 17 n_used 18 n_tok 19 parts 20 n_expert
// 21 residual 22 res_uav 23 res_off.
// Requires F a multiple of 128 up to 1024, 1 <= n_used <= 16, parts <= 8.
#include "gyro_fast.h"
#include "fwht.h"

#define DG_ROWS 8
#define DG_MAX_U 16
#define DG_MAX_NB 8                          // F <= 1024
#define DG_BLOCK_STRIDE 132                  // floats per 128-block in LDS (bank spread)
#define DG_MAX_UNITS (DG_MAX_U * DG_MAX_NB)
#define DG_MAX_BB 58

// Unit (k, bb) of output row w: the block at byte `off` of the staged rows, of type ID, against
// the 128 fp32 inputs x.
template <int ID>
__device__ __forceinline__ float xg_unit(const uint32_t *rw, uint32_t off, const uint32_t *book, const float *x) {
    constexpr int NW = gyro_nw<ID>();
    uint32_t d[NW + 1];
#pragma unroll
    for (int j = 0; j <= NW; ++j) d[j] = rw[(off >> 2) + j];
    float sc;
    uint32_t w[NW];
    gyro_unpack<ID>(d, (off & 2u) != 0u, sc, w);
    return sc * gyro_block_dot<ID>(w, book, x);
}

GD_PIPELINE_NAMED(moe_decode_down_xg, 512) {
    __shared__ uint4 book4[512];
    __shared__ float act[DG_MAX_U * DG_MAX_NB * DG_BLOCK_STRIDE];
    __shared__ gd_u32x4 rows[DG_MAX_U * DG_ROWS * DG_MAX_NB * DG_MAX_BB / 16 + 1];  // + 1: the last block's tail word
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t E = a.c[15], F = a.c[16], U = a.c[17], n_tok = a.c[18], parts = a.c[19], NE = a.c[20];
    const uint32_t NB = F / 128u, t = blockIdx.y, row0 = gd_xcd_group(blockIdx.x, gridDim.x) * DG_ROWS;
    const uint32_t n_slots = n_tok * U;
    const bool has_signs = a.c[11] != 0xffffffffu;
    const uint32_t *GU = gd_buf<const uint32_t>(a, a.c[0]) + a.c[1];
    cuint *ids = as_const(gd_buf<const uint32_t>(a, a.c[2]) + a.c[3] + t * U);
    cfloat *wtp = as_const(gd_buf<const float>(a, a.c[4]) + a.c[5] + t * U);
    reinterpret_cast<gd_u32x4 *>(book4)[tid] = gd_global4(gd_buf<const uint32_t>(a, a.c[10]))[tid];

    // (2) Down rows: expert k's run (8 NB BB_k bytes) starts at row0 NB BB_k bytes of its down
    // matrix and goes to LDS at the prefix of the earlier runs (every offset a multiple of 16).
    const ExpertDesc *xt = gd_buf<const ExpertDesc>(a, a.c[6]);
    uint32_t run_off[DG_MAX_U + 1], dtype[DG_MAX_U];
    run_off[0] = 0;
#pragma unroll
    for (int k = 0; k < DG_MAX_U; ++k) {
        dtype[k] = 0u;
        run_off[k + 1] = run_off[k];
        if ((uint32_t)k < U) {
            const uint32_t e = min(ids[k], NE - 1u);
            dtype[k] = (xt[e].types >> 16) & 0xffu;
            GyroType gt;
            const uint32_t bbk = gd_type(dtype[k], gt) ? gt.block_bytes : 0u;
            run_off[k + 1] = run_off[k] + DG_ROWS * NB * bbk;
        }
    }
    for (uint32_t k = 0; k < U; ++k) {  // uniform
        const uint32_t e = min(ids[k], NE - 1u), nch = (run_off[k + 1] - run_off[k]) / 16u;
        const uint8_t *src = reinterpret_cast<const uint8_t *>(xt[e].down) + (size_t)row0 * ((run_off[k + 1] - run_off[k]) / DG_ROWS);
        for (uint32_t j = tid; j < nch; j += 512u)
            rows[run_off[k] / 16u + j] = *gd_global4(reinterpret_cast<const uint32_t *>(src + j * 16u));
    }

    // (1) Down inputs, unit (k, bb) per 16 lanes.
    const uint32_t l16 = lane & 15u;
    for (uint32_t u = tid >> 4; u < U * NB; u += 32u) {  // uniform per 16-lane row
        const uint32_t k = u / NB, bb = u - k * NB, i0 = bb * 128u + l16 * 8u;
        const uint32_t slot = t * U + k;
        float g[8] = {}, up[8] = {};
        for (uint32_t p = 0; p < parts; ++p) {
            gd_gu32x4 *gp = gd_global4(GU + ((size_t)(p * n_slots + slot) * 2u) * F + i0);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const gd_u32x4 gv = gp[j], uv = gp[F / 4u + j];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    g[4 * j + c] += gd_bits_f32(gv[c]);
                    up[4 * j + c] += gd_bits_f32(uv[c]);
                }
            }
        }
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = gd_silu_rcp(g[j]) * up[j];
        if (has_signs) {
            gd_gu32x4 *S = gd_global4(gd_buf<const uint32_t>(a, a.c[11]) + a.c[12] + i0);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const gd_u32x4 sv = S[j];
#pragma unroll
                for (int c = 0; c < 4; ++c) v[4 * j + c] *= gd_bits_f32(sv[c]);
            }
#pragma unroll
            for (int w = 1; w < 8; w <<= 1)
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (!(j & w)) {
                        const float lo = v[j], hi = v[j + w];
                        v[j] = lo + hi;
                        v[j + w] = lo - hi;
                    }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float p1 = gd_dpp_f<0xB1>(v[j]);
                v[j] = (l16 & 1u) ? p1 - v[j] : v[j] + p1;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float p2 = gd_dpp_f<0x4E>(v[j]);
                v[j] = (l16 & 2u) ? p2 - v[j] : v[j] + p2;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float up4 = gd_dpp_f<0x104>(v[j]);
                const float dn4 = gd_dpp_f<0x114>(v[j]);
                v[j] = (l16 & 4u) ? dn4 - v[j] : v[j] + up4;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float up8 = gd_dpp_f<0x108>(v[j]);
                const float dn8 = gd_dpp_f<0x118>(v[j]);
                v[j] = (l16 & 8u) ? dn8 - v[j] : v[j] + up8;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] *= GD_INV_SQRT128;
        }
        float4 *dst = reinterpret_cast<float4 *>(act + u * DG_BLOCK_STRIDE + l16 * 8u);
        dst[0] = make_float4(v[0], v[1], v[2], v[3]);
        dst[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
    __syncthreads();

    // (3) Output row `wave`: unit k NB + bb on lanes l, l + 64.
    const uint32_t n_units = U * NB;
    const uint32_t *rw = reinterpret_cast<const uint32_t *>(rows);
    const uint32_t *book = reinterpret_cast<const uint32_t *>(book4);
    float part[DG_MAX_UNITS / 64];
    uint32_t pk[DG_MAX_UNITS / 64];
#pragma unroll
    for (int i = 0; i < DG_MAX_UNITS / 64; ++i) {
        const uint32_t u = lane + 64u * (uint32_t)i;
        part[i] = 0.f;
        pk[i] = DG_MAX_U;
        if (u < n_units) {
            const uint32_t k = u / NB, bb = u - k * NB;
            uint32_t ty = dtype[0], ro = run_off[0];
#pragma unroll
            for (int kk = 1; kk < DG_MAX_U; ++kk)
                if ((uint32_t)kk == k) { ty = dtype[kk]; ro = run_off[kk]; }
            GyroType gt;
            const uint32_t bbk = gd_type(ty, gt) ? gt.block_bytes : 0u;
            const uint32_t off = ro + (wave * NB + bb) * bbk;  // byte of the block in rows
            const float *x = act + u * DG_BLOCK_STRIDE;
            float v = 0.f;
#define XG_CASE(ID) v = xg_unit<ID>(rw, off, book, x)
            GYRO_TYPE_SWITCH(ty, XG_CASE)
#undef XG_CASE
            part[i] = v;
            pk[i] = k;
        }
    }
    // Per-expert sums of the units in unit order: lanes write their partials to LDS, then
    // lane k < U adds expert k's NB units in order.
    __shared__ float upart[DG_ROWS][DG_MAX_UNITS];
#pragma unroll
    for (int i = 0; i < DG_MAX_UNITS / 64; ++i)
        if (pk[i] < DG_MAX_U) upart[wave][lane + 64u * (uint32_t)i] = part[i];
    __syncthreads();
    float s = 0.f;
    if (lane < U)
        for (uint32_t j = 0; j < NB; ++j) s += upart[wave][lane * NB + j];
    // Lane 0 combines the experts in k order.
    float acc = 0.f;
    for (uint32_t k = 0; k < U; ++k)
        acc += wtp[k] * gd_bits_f32((uint32_t)__builtin_amdgcn_readlane((int)gd_f32_bits(s), (int)k));
    if (lane == 0u) {
        const uint32_t orow = row0 + wave;
        if (a.c[21]) acc = gd_buf<const float>(a, a.c[22])[a.c[23] + t * E + orow] + acc;
        gd_buf<float>(a, a.c[13])[a.c[14] + t * E + orow] = acc;
    }
}
