// Decode path, step 3, for the shapes moe_decode_down does not take (F other than 512, top-U
// other than 8, hidden not a multiple of 1024): the down-input rotation, the fused TQ2_T
// dequant-GEMV of the down rows and the route-weighted combine (src/engine.zig:607-641).
//
// A group owns R consecutive output rows of one token for all U selected experts, so the
// combine stays local and runs in slot order; the host picks R so that a token spans about one
// group per CU.
//  - Item (slot k, block bb, half hf, row pair): each thread loads the expert id of its item,
//    its inputs' values (below), then block bb of both rows straight from HBM (9 words each),
//    so the weight loads are in flight while the inputs are rotated.
//  - Input unit (k, bb) of 16 lanes: block bb of a_k = H_128(s_down * act_k) / sqrt(128) (the
//    16-lane butterfly of moe_decode_down), 8 consecutive values per lane, into LDS.
//  - Item dots: the thread reads its 64 fp32 activations (half hf of block bb of a_k) from LDS
//    once and decodes that half of both rows' blocks against them (tq2_half_dot); per (row, k)
//    the half sums in (block, half) order times w_k, then per row the slots in slot order, then
//    the residual (every LDS sum reads its operands at once).
// Load order: the ids, the residual, the slot weights, the codebook and the inputs, then the
// blocks, every one issued by every lane (a lane past the last item or unit repeats it), so
// that each wait leaves the loads issued after it in flight.
// Grid: x = E / R, y = n_tok; 512 threads.
// Constants: 0 act_uav 1 act_off (act[(t U + k) F + f], from moe_decode_gu_g) 2 ids_uav 3 ids_off
// 4 weights_uav 5 weights_off 6 base_lo 7 base_hi 8 slot_stride 9 down_off 10 codebook_srv
// 11 signs_srv (0xffffffff: none) 12 signs_off 13 out_uav 14 out_off 15 E 16 F 17 n_used
// 18 n_tok 19 R 20 n_expert 21 residual 22 res_uav 23 res_off (24 xtab_srv: the generic form).
// Requires TQ2_T experts (any types in the generic form), F a multiple of 128 up to 1024,
// 1 <= n_used <= 16, n_used F / 128 <= DG_MAX_ABLK, n_used F / 64 ceil(R / 2) <= 512 DG_ITEMS
// and R n_used <= 512 (the host checks).
#include "gyro_fast.h"
#include "fwht.h"

#ifndef DG_MAX_ABLK
#define DG_MAX_ABLK 64  // rotated input blocks (slots x F / 128) in LDS
#define DG_PIPELINE moe_decode_down_g
#endif
#ifndef DG_GENERIC
#define DG_GENERIC 0  // 1: any Gyro type per expert, rows from the expert table
#endif
// Words loaded per block: TQ2_T's 34 bytes, or the widest type's 58 (whole words from the
// block's first byte rounded down to a word; the arena's slack covers reads past the last row).
#define DG_WORDS (DG_GENERIC ? 15 : 9)
#define DG_ITEMS 2  // (slot, block, half, row pair) items per thread
#define DG_MAX_U 16
#define DG_MAX_EXPERTS 256
#define DG_DEFINE(NAME, WG) GD_PIPELINE_NAMED(NAME, WG)  // expands NAME before it is named
// A rotated 128-block in LDS: half 0 at 0, half 1 at DG_HALF_OFF, blocks DG_BLOCK_STRIDE floats
// apart. Modulo the 64 banks, blocks are 8 banks apart and halves 4: the dozen (block, half)
// rows that a wave's items read at one 16-byte step fall in different banks.
#define DG_BLOCK_STRIDE 136
#define DG_HALF_OFF 68

DG_DEFINE(DG_PIPELINE, 512) {
    __shared__ gd_u32x4 book4[512];
    __shared__ float actr[DG_MAX_ABLK * DG_BLOCK_STRIDE];
    __shared__ float dred[2 * DG_ITEMS * 512];  // half dots by (slot, row, block, half)
    __shared__ float sw[DG_MAX_U];
#if DG_GENERIC
    __shared__ gd_u32x4 xdesc[DG_MAX_EXPERTS];  // per expert {down lo, down hi, types, pad}
#endif
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t E = a.c[15], F = a.c[16], U = a.c[17], R = a.c[19], NE = a.c[20];
    const uint32_t NB = F / 128u, t = blockIdx.y, r0 = gd_xcd_group(blockIdx.x, gridDim.x) * R;
    const uint32_t NP = (R + 1u) / 2u, PK = NB * 2u * NP;  // row pairs; items per slot
    const uint32_t n_items = U * PK;
    const uint32_t *IDS = gd_buf<const uint32_t>(a, a.c[2]) + a.c[3] + t * U;
#if DG_GENERIC
    // The expert table's down pointers and types first: they go to LDS while the ids load.
    const gd_u32x4 xdv = gd_global4(gd_buf<const uint32_t>(a, a.c[24]))[2u * min(tid, NE - 1u) + 1u];
#endif

    // Expert ids of this thread's items (item j = ((k NB + bb) 2 + hf) NP + pair), then their
    // blocks. A thread past the last item loads that item's block again, so that the first item's
    // block loads are issued by every thread: with loads skipped on some path, the compiler could
    // only wait for all loads (the blocks included) before the inputs are rotated.
    uint32_t e[DG_ITEMS];
#pragma unroll
    for (int s = 0; s < DG_ITEMS; ++s) {
        const uint32_t j = min(tid + 512u * (uint32_t)s, n_items - 1u);
        e[s] = gd_global(IDS)[j / PK];
    }
    // The output row's address and its residual now, not after the sums: there they would add
    // two table reads and a load to the end of the group. Without a residual the output row is
    // read instead, and not used.
    float *OUT = gd_buf<float>(a, a.c[13]) + a.c[14];
    const bool residual = a.c[21] != 0u;
    const float *RES = residual ? gd_buf<const float>(a, a.c[22]) + a.c[23] : OUT;
    // Lane k of 16-lane row q stores output row q (see the row sums below).
    const uint32_t resv = gd_global(reinterpret_cast<const uint32_t *>(RES))[t * E + r0 + min(tid >> 4, R - 1u)];
    // The codebook and weights are stored to LDS only after the block loads are issued (an LDS
    // store of a loaded value waits for every load issued before it; so does the rotation).
    const uint32_t swv = tid < U ? gd_global(gd_buf<const uint32_t>(a, a.c[4]) + a.c[5] + t * U)[tid] : 0u;
    const gd_u32x4 bkv = gd_global4(gd_buf<const uint32_t>(a, a.c[10]))[tid];
#if !DG_GENERIC
    const uint64_t layer_base = (uint64_t)a.c[6] | ((uint64_t)a.c[7] << 32);
    const uint8_t *LB = reinterpret_cast<const uint8_t *>(layer_base);
    const uint32_t stride = a.c[8], down_off = a.c[9], drow_bytes = NB * 34u;
#endif
    // Inputs: unit (k, bb) per 16 lanes, up to DG_MAX_ABLK / 32 passes, every pass's loads
    // issued before the first is rotated. Every lane loads (a row past the last unit repeats
    // it; without signs the inputs stand in for them), so that the waits for the ids and the
    // inputs leave the loads issued after them in flight.
    const bool has_signs = a.c[11] != 0xffffffffu;
    const float *ACT = gd_buf<const float>(a, a.c[0]) + a.c[1] + (size_t)t * U * F;
    const uint32_t *SG = has_signs ? gd_buf<const uint32_t>(a, a.c[11]) + a.c[12] : reinterpret_cast<const uint32_t *>(ACT);
    const uint32_t l16 = lane & 15u;
    constexpr int PASSES = DG_MAX_ABLK / 32;
    gd_u32x4 av[PASSES][2], svv[PASSES][2];
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
        if (ps >= 2 && 32u * (uint32_t)ps >= U * NB) break;  // uniform: passes past 64 blocks only when used
        const uint32_t u = min((tid >> 4) + 32u * (uint32_t)ps, U * NB - 1u);
        const uint32_t k = u / NB, bb = u - k * NB, i0 = bb * 128u + l16 * 8u;
        gd_gu32x4 *ap = gd_global4(reinterpret_cast<const uint32_t *>(ACT + (size_t)k * F + i0));
        av[ps][0] = ap[0];
        av[ps][1] = ap[1];
        gd_gu32x4 *S = gd_global4(SG + i0);
        svv[ps][0] = S[0];
        svv[ps][1] = S[1];
    }
#if DG_GENERIC
    if (tid < NE) xdesc[tid] = xdv;
    __syncthreads();
#endif
    // The blocks after the inputs' loads, so the inputs can be rotated while they are in flight.
    uint32_t dw[DG_ITEMS][2][DG_WORDS];
    bool odd[DG_ITEMS][2];
    uint32_t ty[DG_ITEMS];
#pragma unroll
    for (int s = 0; s < DG_ITEMS; ++s) {
        const uint32_t j = min(tid + 512u * (uint32_t)s, n_items - 1u);
        odd[s][0] = odd[s][1] = false;
        ty[s] = 144u;
        if (s == 0 || n_items > 512u * (uint32_t)s) {  // uniform
            const uint32_t rem = j % PK, bb = rem / (2u * NP), pair = rem % NP;
#if DG_GENERIC
            const gd_u32x4 xd = xdesc[min(e[s], NE - 1u)];
            ty[s] = (xd[2] >> 16) & 0xffu;
            GyroType gt;
            gd_type(ty[s], gt);  // the host admits only the eight types
            const uint8_t *LB = reinterpret_cast<const uint8_t *>(((uint64_t)xd[1] << 32) | xd[0]);
#endif
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint32_t row = min(2u * pair + (uint32_t)i, R - 1u);  // an odd R repeats its last row
#if DG_GENERIC
                const uint64_t off = ((uint64_t)(r0 + row) * NB + bb) * gt.block_bytes;
                gd_guint *w = gd_global(reinterpret_cast<const uint32_t *>(LB + (off & ~uint64_t(3))));
#pragma unroll
                for (int q = 0; q < DG_WORDS; ++q) dw[s][i][q] = w[q];
                odd[s][i] = ((reinterpret_cast<uintptr_t>(LB) + off) & 2u) != 0u;
#else
                const uint64_t off = (uint64_t)min(e[s], NE - 1u) * stride + down_off +
                                     (uint64_t)(r0 + row) * drow_bytes + bb * 34u;
                tq2_load_block(LB, off, dw[s][i]);
                odd[s][i] = (off & 2u) != 0u;
#endif
            }
        }
    }

    book4[tid] = bkv;
    if (tid < U) sw[tid] = gd_bits_f32(swv);
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
        const uint32_t u = (tid >> 4) + 32u * (uint32_t)ps;
        if (u >= U * NB) break;  // uniform per 16-lane row
        float v[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) { v[j] = gd_bits_f32(av[ps][0][j]); v[4 + j] = gd_bits_f32(av[ps][1][j]); }
        if (has_signs) {
#pragma unroll
            for (int j = 0; j < 4; ++j) { v[j] *= gd_bits_f32(svv[ps][0][j]); v[4 + j] *= gd_bits_f32(svv[ps][1][j]); }
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
                const float p1 = gd_dpp_f<0xB1>(v[j]);  // quad_perm [1,0,3,2]
                v[j] = (l16 & 1u) ? p1 - v[j] : v[j] + p1;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float p2 = gd_dpp_f<0x4E>(v[j]);  // quad_perm [2,3,0,1]
                v[j] = (l16 & 2u) ? p2 - v[j] : v[j] + p2;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float up4 = gd_dpp_f<0x104>(v[j]), dn4 = gd_dpp_f<0x114>(v[j]);  // row_shl:4, row_shr:4
                v[j] = (l16 & 4u) ? dn4 - v[j] : v[j] + up4;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float up8 = gd_dpp_f<0x108>(v[j]), dn8 = gd_dpp_f<0x118>(v[j]);  // row_shl:8, row_shr:8
                v[j] = (l16 & 8u) ? dn8 - v[j] : v[j] + up8;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] *= GD_INV_SQRT128;
        }
        float4 *dst = reinterpret_cast<float4 *>(actr + u * DG_BLOCK_STRIDE + l16 * 8u + (l16 >= 8u ? DG_HALF_OFF - 64u : 0u));
        dst[0] = make_float4(v[0], v[1], v[2], v[3]);
        dst[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
    __syncthreads();

    // Item dots: the half's 64 activations from LDS once, then that half of both rows' blocks;
    // dred[((k R + row) NB + bb) 2 + hf].
    const uint32_t *book = reinterpret_cast<const uint32_t *>(book4);
#pragma unroll
    for (int s = 0; s < DG_ITEMS; ++s) {
        const uint32_t j = tid + 512u * (uint32_t)s;
        if (j < n_items) {
            const uint32_t k = j / PK, rem = j - k * PK, bh = rem / NP, pair = rem - bh * NP;
            const uint32_t bb = bh >> 1, hf = bh & 1u;
            const float4 *ar = reinterpret_cast<const float4 *>(actr + (k * NB + bb) * DG_BLOCK_STRIDE + DG_HALF_OFF * hf);
            float x[64];
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                const float4 v = ar[c];
                x[4 * c] = v.x; x[4 * c + 1] = v.y; x[4 * c + 2] = v.z; x[4 * c + 3] = v.w;
            }
            float h[2] = {0.f, 0.f};
#if DG_GENERIC
#define DG_CASE(ID)                                                       \
    _Pragma("unroll") for (int i = 0; i < 2; ++i) {                       \
        float sc;                                                         \
        uint32_t q[gyro_nw<ID>()];                                        \
        gyro_unpack<ID>(dw[s][i], odd[s][i], sc, q);                      \
        h[i] = sc * gyro_half_dot<ID>(q, hf, book, x);                    \
    }
            GYRO_TYPE_SWITCH(ty[s], DG_CASE)
#undef DG_CASE
#else
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                float sc;
                uint32_t q[8];
                tq2_unpack(dw[s][i], odd[s][i], sc, q);
                h[i] = sc * tq2_half_dot(q, hf, book, x);
            }
#endif
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint32_t row = 2u * pair + (uint32_t)i;
                if (row < R) dred[((k * R + row) * NB + bb) * 2u + hf] = h[i];
            }
        }
    }
    __syncthreads();
    // Output rows, 32 at a time: lane k of 16-lane row q holds slot k of output row q, w_k times
    // the row's half sums in (block, half) order (2 NB <= 16 loads at once); the 16 lanes then
    // add the slot terms in slot order (one DPP step per slot), and lane U - 1 adds the residual
    // and stores. No second pass through LDS.
    const uint32_t nbh = 2u * NB, k16 = tid & 15u;
    for (uint32_t row = tid >> 4; row < R; row += 32u) {  // uniform per 16-lane row
        float term = 0.f;
        if (k16 < U) {
            const float *d = dred + (k16 * R + row) * nbh;
            float dk = 0.f;
#pragma unroll
            for (uint32_t bh = 0; bh < 16u; ++bh) {
                const float v = d[bh < nbh ? bh : nbh - 1u];
                dk += bh < nbh ? v : 0.f;
            }
            term = sw[k16] * dk;
        }
        float acc = 0.f + term;
#pragma unroll
        for (uint32_t k = 1; k < DG_MAX_U; ++k) {
            const float prev = gd_dpp_f<0x111>(acc);  // row_shr:1, lane k - 1
            acc = k16 == k ? prev + term : acc;
        }
        if (k16 == U - 1u) {
            const uint32_t o = t * E + r0 + row;
            if (residual) acc = (row < 32u ? gd_bits_f32(resv) : RES[o]) + acc;
            OUT[o] = acc;
        }
    }
}
