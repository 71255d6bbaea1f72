// Decode path, steps 1 and 2 in one launch: router logits, the input rotation, routing and the
// fused TQ2_T dequant-GEMV of the gate and up rows, for up to 8 tokens.
//   logits[t][r] = W_r[r] . x[t] (+ bias[r])          src/engine.zig:526 (kernels.matmul)
//   xh[t] = H_128 (gate_signs * x[t]) per 128-block    src/engine.zig:547-551
//   top-8, renormalised weights                        src/engine.zig:527-540, :670-687
//   gate/up rows of the selected experts               src/engine.zig:567-602
// (optionally after the stack's RMSNorm, src/kernels.zig:281-291, as moe_router.)
//
// moe_router followed by moe_decode_gu costs a dependent launch between them; here the logits
// pass from group to group inside one grid instead:
//  (1) group L < P = min(G, n_expert) (G groups in all, L the linear group id) computes router
//      rows L and L + P of every token with waves 0-3, in moe_router's arithmetic (thread t of
//      the four waves takes columns 4 t + 1024 j; DPP wave sums; the four wave sums added
//      (w0 + w1) + (w2 + w3)), so the logits are bit-identical to moe_router's. Each logit goes
//      out as one 64-bit word (epoch << 32 | bits) with a device-scope store, one word per
//      128-byte line (every group polls all of its token's words: packed into 16 lines, the
//      polls of 256 groups queued on a few memory channels and the launch ran 5% slower); the
//      epoch is a per-call constant, never 0, that the host increases from call to call;
//  (2) meanwhile waves 4 and 5 rotate this group's K-part of its token (eight 128-blocks, in
//      16-lane DPP rows as moe_router) into the binary16 activation layout of moe_decode_gu, and
//      every thread stages its 16 bytes of the codebook;
//  (3) wave 0 polls its token's n_expert logit words (device-scope loads) until all carry the
//      epoch, and puts the logits in LDS;
//  (4) from there on, moe_decode_gu: every wave routes to rank k, loads its block of the
//      expert's row, and decodes it; the group of (row block 0, projection 0, part 0, rank 0) of
//      each token stores its ids and weights.
// Groups that produce logits are the first P of the grid, which the dispatcher places first on
// every XCD; a group waits only on those, so every wait ends once the first P groups run. Each
// wait is still bounded (constant 15 polls); a group that gives up stores 1 to the sticky error
// word (its outputs are then invalid and the host recomputes or refuses the call).
// Grid: x = F / 64, y = 2 * parts, z = n_tok * 8; 512 threads. Output partials gu[part][slot][proj][F].
// Constants: 0 x_uav 1 x_off 2 x_stride 3 n_tok 4 router_srv 5 bias_srv (0xffffffff: none)
// 6 n_expert 7 E 8 F 9 signs_srv (gate signs [E]; 0xffffffff: none) 10 norm (0: none, 1: RMSNorm
// without weight, 2: with weight) 11 norm_w_srv 12 eps (fp32 bits) 13 lgx_uav (n_tok x n_expert
// 64-bit logit words, 128 bytes apart) 14 epoch 15 spin limit 16 err_uav 17 err_off (the sticky error word)
// 18 scale (fp32 bits) 19 ids_uav 20 ids_off 21 weights_uav 22 weights_off 23 base_lo 24 base_hi
// 25 slot_stride 26 proj_bytes 27 codebook_srv 28 gu_uav 29 gu_off 30 range flag (table index;
// 0: none).
// Requires TQ2_T experts, E 1024 or 2048, F a multiple of 64, top-8, n_expert <= 256 with at
// most two router rows per producing group, n_tok <= 8 (the host checks).
#include "gyro_fast.h"
#include "fwht.h"
#include "route_fast.h"

#define RGU_ROWS 64
#define RGU_U 8
#define RGU_MAX_TOK 8
#define RGU_MAX_R 2
#define RGU_WORD_STRIDE 16  // 64-bit words: one logit word per 128-byte line

typedef unsigned long long rgu_u64;

__device__ __forceinline__ float4 rgu_f4(gd_u32x4 v) {
    return make_float4(gd_bits_f32(v[0]), gd_bits_f32(v[1]), gd_bits_f32(v[2]), gd_bits_f32(v[3]));
}

GD_PIPELINE_NAMED(moe_decode_rgu, 512) {
    __shared__ uint4 book4[512];
    __shared__ uint4 xpart[128];  // the part's 1024 activations as binary16 pairs
    __shared__ float lg[256];     // the token's logits
    __shared__ float red[RGU_MAX_R][4][RGU_MAX_TOK], reds[4][RGU_MAX_TOK];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t NE = a.c[6], E = a.c[7], F = a.c[8], n_tok = a.c[3] < RGU_MAX_TOK ? a.c[3] : RGU_MAX_TOK;
    const uint32_t slot = blockIdx.z, t = slot / RGU_U, k = slot - t * RGU_U;
    const uint32_t parts = E / 1024u, proj = blockIdx.y / parts, part = blockIdx.y - proj * parts;
    const uint32_t row0 = blockIdx.x * RGU_ROWS;
    const uint32_t b = lane & 7u, r = wave * 8u + (lane >> 3);  // this lane's block and row
    const uint32_t G = gridDim.x * gridDim.y * gridDim.z;
    const uint32_t L = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    const uint32_t P = G < NE ? G : NE;
    const bool producer = L < P;  // uniform
    const uint32_t norm = a.c[10], x_off = a.c[1], x_stride = a.c[2];
    const float *X = gd_buf<const float>(a, a.c[0]);
    const float *NW = norm == 2u ? gd_buf<const float>(a, a.c[11]) : nullptr;

    // Codebook: every thread's 16 bytes, a global load in flight with the others.
    const gd_u32x4 cbv = gd_global4(gd_buf<const uint32_t>(a, a.c[27]))[tid];

    // Rotation inputs of waves 4 and 5: lane l holds values 8 (l % 16) .. + 7 of the part's block
    // 4 (wave - 4) + l / 16 of token t.
    const bool rot_wave = wave == 4u || wave == 5u;  // uniform per wave
    const uint32_t l16 = lane & 15u, bx = (wave & 1u) * 4u + (lane >> 4);
    const uint32_t ri = (part * 8u + bx) * 128u + l16 * 8u;
    const bool has_signs = a.c[9] != 0xffffffffu;
    float rx[8], rs[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) rs[j] = 1.f;
    if (rot_wave) {
        if (has_signs) {
            gd_gu32x4 *sv = gd_global4(gd_buf<const uint32_t>(a, a.c[9]) + ri);
            const float4 s0 = rgu_f4(sv[0]), s1 = rgu_f4(sv[1]);
            rs[0] = s0.x; rs[1] = s0.y; rs[2] = s0.z; rs[3] = s0.w;
            rs[4] = s1.x; rs[5] = s1.y; rs[6] = s1.z; rs[7] = s1.w;
        }
        if (norm == 2u) {
            gd_gu32x4 *nv = gd_global4(reinterpret_cast<const uint32_t *>(NW) + ri);
            const float4 n0 = rgu_f4(nv[0]), n1 = rgu_f4(nv[1]);
            rs[0] *= n0.x; rs[1] *= n0.y; rs[2] *= n0.z; rs[3] *= n0.w;
            rs[4] *= n1.x; rs[5] *= n1.y; rs[6] *= n1.z; rs[7] *= n1.w;
        }
        gd_gu32x4 *xv = gd_global4(reinterpret_cast<const uint32_t *>(X) + x_off + t * x_stride + ri);
        const float4 x0 = rgu_f4(xv[0]), x1 = rgu_f4(xv[1]);
        rx[0] = x0.x; rx[1] = x0.y; rx[2] = x0.z; rx[3] = x0.w;
        rx[4] = x1.x; rx[5] = x1.y; rx[6] = x1.z; rx[7] = x1.w;
    }

    // (1) Router rows (waves 0-3), moe_router's arithmetic; with the norm, the sums of squares of
    // every token (producers) or of token t (the others) from the same loads.
    if (wave < 4u) {
        constexpr int PER = 2;  // E <= 2048: columns 4 tid + 1024 j, j < E / 1024
        const uint32_t *XU = reinterpret_cast<const uint32_t *>(X) + x_off + tid * 4u;
        float4 w[RGU_MAX_R][PER];
#pragma unroll
        for (int rr = 0; rr < RGU_MAX_R; ++rr) {
            const uint32_t row = L + (uint32_t)rr * P;
            const bool dot = producer && row < NE;  // uniform
            const uint32_t *W = gd_buf<const uint32_t>(a, a.c[4]) + (size_t)(dot ? row : 0u) * E;
#pragma unroll
            for (int j = 0; j < PER; ++j)
                if (dot && tid * 4u + 1024u * j < E) {
                    w[rr][j] = rgu_f4(*gd_global4(W + tid * 4u + 1024u * j));
                    if (norm == 2u) {
                        const float4 g = rgu_f4(*gd_global4(reinterpret_cast<const uint32_t *>(NW) + tid * 4u + 1024u * j));
                        w[rr][j] = make_float4(w[rr][j].x * g.x, w[rr][j].y * g.y, w[rr][j].z * g.z, w[rr][j].w * g.w);
                    }
                }
        }
#pragma unroll
        for (int tt = 0; tt < RGU_MAX_TOK; ++tt) {
            if ((uint32_t)tt < n_tok && (producer || (uint32_t)tt == t)) {  // uniform
                float acc[RGU_MAX_R] = {0.f, 0.f}, ss = 0.f;
#pragma unroll
                for (int j = 0; j < PER; ++j)
                    if (tid * 4u + 1024u * j < E) {
                        const float4 v = rgu_f4(*gd_global4(XU + tt * x_stride + 1024u * j));
#pragma unroll
                        for (int rr = 0; rr < RGU_MAX_R; ++rr)
                            if (producer && L + (uint32_t)rr * P < NE)
                                acc[rr] += (w[rr][j].x * v.x + w[rr][j].y * v.y) + (w[rr][j].z * v.z + w[rr][j].w * v.w);
                        if (norm) ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
                    }
#pragma unroll
                for (int rr = 0; rr < RGU_MAX_R; ++rr) {
                    if (producer && L + (uint32_t)rr * P < NE) {
                        const float s = gd_wave_sum_dpp(acc[rr]);
                        if (lane == 0) red[rr][wave][tt] = s;
                    }
                }
                if (norm) {
                    const float q = gd_wave_sum_dpp(ss);
                    if (lane == 0) reds[wave][tt] = q;
                }
            }
        }
    }
    reinterpret_cast<gd_u32x4 *>(book4)[tid] = cbv;
    __syncthreads();

    uint32_t *err = gd_buf<uint32_t>(a, a.c[16]) + a.c[17];
    rgu_u64 *lgx = gd_buf<rgu_u64>(a, a.c[13]);
    const uint32_t epoch = a.c[14];
    if (wave == 0u) {
        // Logit words: thread (rr, tt) = (tid / 8, tid % 8).
        const uint32_t rr = tid >> 3, tt = tid & 7u, row = L + rr * P;
        if (producer && rr < RGU_MAX_R && tt < n_tok && row < NE) {
            float v = (red[rr][0][tt] + red[rr][1][tt]) + (red[rr][2][tt] + red[rr][3][tt]);
            if (norm) {
                const float q = (reds[0][tt] + reds[1][tt]) + (reds[2][tt] + reds[3][tt]);
                v *= 1.0f / sqrtf(q / (float)E + gd_bits_f32(a.c[12]));
            }
            if (a.c[5] != 0xffffffffu) v += gd_buf<const float>(a, a.c[5])[row];
            __hip_atomic_store(lgx + (tt * NE + row) * RGU_WORD_STRIDE, ((rgu_u64)epoch << 32) | gd_f32_bits(v), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
        // (3) The token's logits, once every word carries the epoch.
        const rgu_u64 *src = lgx + t * NE * RGU_WORD_STRIDE;
        float lv[4];
        uint32_t n = 0;
        bool done = false;
        while (!done) {
            bool ok = true;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t i = lane + 64u * j;
                lv[j] = 0.f;
                if (i < NE) {
                    const rgu_u64 wv = __hip_atomic_load(src + i * RGU_WORD_STRIDE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ok = ok && (uint32_t)(wv >> 32) == epoch;
                    lv[j] = gd_bits_f32((uint32_t)wv);
                }
            }
            done = __ballot(!ok) == 0ull;
            if (!done && ++n >= a.c[15]) {
                if (lane == 0) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                done = true;
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (lane + 64u * j < 256u) lg[lane + 64u * j] = lv[j];
    }
    if (rot_wave) {
        // (2) This group's eight blocks of token t, rotated (moe_router's arithmetic).
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = rx[j];
        if (norm) {
            const float q = (reds[0][t] + reds[1][t]) + (reds[2][t] + reds[3][t]);
            const float sc = 1.0f / sqrtf(q / (float)E + gd_bits_f32(a.c[12]));
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] *= sc;
        }
        if (has_signs || norm == 2u) {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] *= rs[j];
        }
        if (has_signs) {
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
                const float up4 = gd_dpp_f<0x104>(v[j]);  // row_shl:4, lane + 4
                const float dn4 = gd_dpp_f<0x114>(v[j]);  // row_shr:4, lane - 4
                v[j] = (l16 & 4u) ? dn4 - v[j] : v[j] + up4;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float up8 = gd_dpp_f<0x108>(v[j]);  // row_shl:8, lane + 8
                const float dn8 = gd_dpp_f<0x118>(v[j]);  // row_shr:8, lane - 8
                v[j] = (l16 & 8u) ? dn8 - v[j] : v[j] + up8;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] *= GD_INV_SQRT128;
        }
        gd_u32x4 o;
        bool bad = false;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            bad |= !gd_half_ok(v[2 * j]) || !gd_half_ok(v[2 * j + 1]);
            const uint32_t h0 = __builtin_bit_cast(uint16_t, (_Float16)v[2 * j]);
            const uint32_t h1 = __builtin_bit_cast(uint16_t, (_Float16)v[2 * j + 1]);
            o[j] = h0 | (h1 << 16);
        }
        // Chunk l16 of block bx at position bx * 16 + (l16 + bx) % 16 (moe_decode_gu's layout).
        reinterpret_cast<gd_u32x4 *>(xpart)[bx * 16u + ((l16 + bx) & 15u)] = o;
        gd_range_flag(a.table, a.c[30], bad);
    }
    __syncthreads();

    // (4) moe_decode_gu from here: activations in registers, routing to rank k.
    uint32_t xs[64];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const uint4 v = xpart[b * 16u + ((j + b) & 15u)];
        xs[4 * j] = v.x; xs[4 * j + 1] = v.y; xs[4 * j + 2] = v.z; xs[4 * j + 3] = v.w;
    }
    float lv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t i = lane + 64u * j;
        lv[j] = lg[i < NE ? i : NE - 1u];
    }
    const bool writer = blockIdx.x == 0 && blockIdx.y == 0 && k == 0;
    uint64_t key[4];
    rf_init<4>(lv, NE, key);
    uint32_t ids[RGU_U], e = 0;
    float top[RGU_U];
#pragma unroll
    for (int j = 0; j < RGU_U; ++j) {
        if ((uint32_t)j <= k || writer) {  // uniform
            ids[j] = rf_next<4>(key, top[j]);
            if ((uint32_t)j == k) e = ids[j];
        }
    }
    e = e < NE ? e : NE - 1u;  // ids are always < NE for finite logits; never address past the layer

    const uint64_t layer_base = (uint64_t)a.c[23] | ((uint64_t)a.c[24] << 32);
    const uint32_t row_bytes = E / 128u * 34u;
    gd_guint *w = gd_global(reinterpret_cast<const uint32_t *>(
        reinterpret_cast<const uint8_t *>(layer_base) + (uint64_t)e * a.c[25] + (proj ? a.c[26] : 0u) +
        (uint64_t)(row0 + r) * row_bytes + part * 272u + ((b * 34u) & ~3u)));
    uint32_t d[9];
#pragma unroll
    for (int j = 0; j < 9; ++j) d[j] = w[j];
    if (writer && wave == 0u) {
        float wts[RGU_U];
        rf_weights<RGU_U>(top, gd_bits_f32(a.c[18]), wts);
        if (lane < RGU_U) {
            uint32_t id = ids[0];
            float wv = wts[0];
#pragma unroll
            for (int j = 1; j < RGU_U; ++j) {
                id = lane == (uint32_t)j ? ids[j] : id;
                wv = lane == (uint32_t)j ? wts[j] : wv;
            }
            gd_buf<uint32_t>(a, a.c[19])[a.c[20] + t * RGU_U + lane] = id;
            gd_buf<float>(a, a.c[21])[a.c[22] + t * RGU_U + lane] = wv;
        }
    }
    float sc;
    uint32_t q[8];
    tq2_unpack(d, (b & 1u) != 0u, sc, q);
    float v = sc * tq2_block_dot_h(q, reinterpret_cast<const uint32_t *>(book4), xs);
    v = v + gd_dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]: + lane ^ 1
    v = v + gd_dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]: + lane ^ 2
    v = v + gd_dpp_f<0x104>(v);  // row_shl:4: + lane + 4 (read by lanes b < 4)
    if (b == 0u) {
        const uint32_t n_slots = n_tok * RGU_U;
        gd_buf<float>(a, a.c[28])[a.c[29] + ((size_t)(part * n_slots + slot) * 2u + proj) * F + row0 + r] = v;
    }
}
