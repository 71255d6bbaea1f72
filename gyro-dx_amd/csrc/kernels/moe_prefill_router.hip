// Prefill path, step 1: router logits of many tokens on binary16 MFMA with split operands, and
// the rotated expert input in binary16.
//   logits[t][r] = W_r[r] . x[t] (+ bias[r])          src/engine.zig:526 (kernels.matmul)
//   xh16[t]      = H_128 (gate_signs * x[t]) per 128-block, as binary16 pairs
//                                                      src/engine.zig:547-551
// Split operands. Each fp32 value v is carried as two binary16 values, v = hi + lo 2^-11 with
// hi = f16(v) and lo = f16((v - hi) 2^11) (both round to nearest even; v - hi is exact in fp32):
// 22 significant bits instead of fp32's 24, over the binary16 range of hi. The products that
// matter, x.w = hi_x hi_w + 2^-11 (hi_x lo_w + lo_x hi_w) (dropping lo_x lo_w, 2^-22 relative),
// run as three v_mfma_f32_32x32x16_f16 with fp32 accumulation, about a fifth of the issue time of
// fp32 MFMA. The router rows come split at load time (the layout below), each row scaled by a
// power of two 2^k_r so that its largest |weight| lies in [2^14, 2^15); the logit is multiplied
// by 2^-k_r at the end. The tokens are split here as they are staged; a value beyond 65504 sets
// the range flag (the caller then recomputes the call on fp32 weights and activations).
// Group (bx, by, bz) computes the 32 x 32 logit tile of tokens 32 bx.. and experts 32 by.. over
// K range bz of S (the K split, chosen by the host so that small batches still fill the GPU);
// its waves 0..3 split the range into quarters and their partial tiles are added in wave order
// through LDS. Range bz writes logit plane bz; the top-k kernel adds the S planes in plane
// order. Each of these waves stages its own 32-wide K chunks of the 32 token rows (fp32) and the
// 32 router rows (split) into LDS first: direct global-to-LDS loads (8 lanes per 128-byte row,
// so that every load instruction fetches whole cache lines; 64-byte rows took the K loop about
// 2 µs longer at 1024 tokens), the 16-byte piece q of row r stored at position q ^ (r % 8), two
// chunks ahead in three buffers per wave; only the wave's own load count is waited for, so the K
// loop has no barrier. A group takes 96 KB of LDS, one group per CU. Lane half h of a wave takes
// k = 8h .. 8h + 7 of every 16-K step for both operands (the MFMA's operand layout), so every
// product x[t][k] W[r][k] enters the sum once. Waves 4..7 meanwhile rotate: all n * E/128
// blocks are spread over the rotation waves of the grid, eight blocks per wave at a time, so the
// rotation's memory traffic and VALU work overlap the MFMA chains on the same SIMDs.
// Grid: (ceil(n / 32), ceil(n_expert / 32), S); 512 threads, 96 KB of LDS. Requires
// E % (128 S) == 0.
// Router layout (router_srv, from router_off): row r, chunk c (k = 16 c .. 16 c + 15) at word
// 16 (r E / 16 + c): the 16 hi values, then the 16 lo values, as binary16; after the n_expert x E
// words, the n_expert factors 2^-k_r (fp32).
// Constants: 0 x_uav 1 x_off (words; rows of E floats) 2 n_tok 3 E 4 router_srv 5 router_off
// 6 n_expert 7 bias_srv (0xffffffff: none) 8 bias_off 9 logits_uav 10 logits_off
// 11 signs_srv (0xffffffff: no rotation, plain conversion) 12 signs_off 13 xh16_uav
// 14 xh16_off (words) 15 x16 (1: also write the unrotated input as binary16, for the shared
// expert; zero when the caller passes 15 constants) 16 x16_uav 17 x16_off (words) 18 S (0 or
// 1: no split; plane z at logits_off + z n n_expert; the bias enters plane 0) 19 range flag
// (table index of a word set to 1 when a value written or split as binary16 is outside its
// range; 0: none) 20 hist_uav (0: none) 21 hist_off (words) 22 hist_words: the rotation waves
// zero these words of moe_prefill_topk's chunk histogram.
#include "ggemm.h"
#include "fwht.h"

#define RT_WAVES 4
#define RT_KC 32    // K per staged chunk: one 128-byte line of every token row
#define RT_NBUF 3   // chunks c .. c + 2 of a wave in LDS: two chunks in flight
#ifndef RT_PIPELINE
// This build: each MFMA wave takes one 32-expert column tile over a quarter of the group's K
// range (the group's tile is 32 x 32, the four partial tiles added through LDS).
#define RT_PIPELINE moe_prefill_router
#define RT_TW 1
#endif
// Loads per chunk and wave: four of token rows, four per 32-expert column tile.
#define RT_LOADS (4 * (1 + RT_TW))

// The staging buffers of the four MFMA waves; in the one-tile build a wave's partial tile (4 KB,
// fp32) goes over its own first activation buffer after its K loop.
struct __attribute__((aligned(16))) RtLds {
    gd_u32x4 x[RT_WAVES][RT_NBUF][32 * RT_KC / 4];          // 32 rows x 128 bytes
    gd_u32x4 w[RT_WAVES][RT_NBUF][32 * RT_TW * RT_KC / 4];  // 32 RT_TW rows x 128 bytes
};
static_assert(sizeof(RtLds) <= 163840, "the CU's 160 KB");
static_assert(sizeof(RtLds::x[0]) >= 32 * 32 * 4, "a wave's partial tile fits its activation buffers");

// Swizzled position of 16-byte piece q of staged row r: the piece that the 8 lanes of rows
// m .. m + 7 read at one index sits in 8 different 16-byte bank groups.
__device__ __forceinline__ uint32_t rt_pos(uint32_t q, uint32_t r) { return q ^ (r & 7u); }

// Waits until chunk c's loads have landed, with `ahead` (0 or 1) later chunks of RT_LOADS loads in
// flight.
__device__ __forceinline__ void rt_wait(uint32_t ahead) {
    if (ahead) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(RT_LOADS) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Stages a chunk of this wave's 32 token rows and 32 RT_TW router rows (xk, wk: the bases advanced
// to the chunk's K offset): 4 + 4 RT_TW loads, lane l of load i carrying row 8 i + l / 8,
// position l % 8.
__device__ __forceinline__ void rt_stage(RtLds &sm, uint32_t wave, uint32_t buf, const char *xk, const char *wk,
                                         const uint32_t xoff[4], const uint32_t woff[4 * RT_TW]) {
    const uint32_t lx = gg_lds_addr(&sm.x[wave][buf][0]), lw = gg_lds_addr(&sm.w[wave][buf][0]);
#pragma unroll
    for (int i = 0; i < 4; ++i) gg_dma16(lx + (uint32_t)i * 1024u, xk, xoff[i]);
#pragma unroll
    for (int i = 0; i < 4 * RT_TW; ++i) gg_dma16(lw + (uint32_t)i * 1024u, wk, woff[i]);
}

// Operands of one K-step (16 K) for this lane (row m, lane half h; k = 8 h .. 8 h + 7 of the
// step): the token row's values split into hi and lo, and the hi and lo of the router row of
// each column tile.
struct RtOps {
    f16x8 xh, xl, wh[RT_TW], wl[RT_TW];
};
// The step's raw reads from LDS (step s of the chunk in buffer buf): two 16-byte pieces of the
// token row (fp32), and per column tile one of the router row's hi values and one of its lo
// values. A staged router row holds, per 16 K, the 16 hi values then the 16 lo values.
struct RtRaw {
    gd_u32x4 x[2], wh[RT_TW], wl[RT_TW];
};
__device__ __forceinline__ void rt_read(const RtLds &sm, uint32_t wave, uint32_t buf, uint32_t s, uint32_t m,
                                        uint32_t h, RtRaw &o) {
    o.x[0] = sm.x[wave][buf][m * 8u + rt_pos(4u * s + 2u * h, m)];
    o.x[1] = sm.x[wave][buf][m * 8u + rt_pos(4u * s + 2u * h + 1u, m)];
#pragma unroll
    for (int j = 0; j < RT_TW; ++j) {
        const uint32_t r = m + 32u * (uint32_t)j;
        o.wh[j] = sm.w[wave][buf][r * 8u + rt_pos(4u * s + h, r)];
        o.wl[j] = sm.w[wave][buf][r * 8u + rt_pos(4u * s + 2u + h, r)];
    }
}
// hi = f16(v), lo = f16((v - hi) 2^11) of the eight token values; xmax tracks max |v|. The lo
// value is one mixed-precision fused multiply-add, 2^11 v - 2^11 hi (exact before its rounding
// to binary16), that reads hi from its half of the packed conversion.
__device__ __forceinline__ void rt_split(const RtRaw &r, RtOps &o, float &xmax) {
    typedef _Float16 h2v __attribute__((ext_vector_type(2)));
    gd_u32x4 xh, xl;
    const float m2048 = -2048.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float v0 = gd_bits_f32(r.x[j >> 1][2 * (j & 1)]), v1 = gd_bits_f32(r.x[j >> 1][2 * (j & 1) + 1]);
        const h2v hi = {(_Float16)v0, (_Float16)v1};
        const uint32_t hp = __builtin_bit_cast(uint32_t, hi);
        uint32_t lo;
        asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(lo) : "v"(hp), "s"(m2048), "v"(v0 * 2048.0f));
        asm("v_fma_mixhi_f16 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
            : "+v"(lo)
            : "v"(hp), "s"(m2048), "v"(v1 * 2048.0f));
        xh[j] = hp;
        xl[j] = lo;
        xmax = fmaxf(xmax, __builtin_fabsf(v0));
        xmax = fmaxf(xmax, __builtin_fabsf(v1));
    }
    o.xh = __builtin_bit_cast(f16x8, xh);
    o.xl = __builtin_bit_cast(f16x8, xl);
#pragma unroll
    for (int j = 0; j < RT_TW; ++j) {
        o.wh[j] = __builtin_bit_cast(f16x8, r.wh[j]);
        o.wl[j] = __builtin_bit_cast(f16x8, r.wl[j]);
    }
}
// One K-step's MFMAs (operands `cur`; three per column tile) with the step's other work between
// them, so that the matrix pipe has the next MFMA waiting. A chunk takes two steps:
//  - the first (SECOND false) issues the loads staging chunk c + RT_NBUF - 1 (into buffer
//    bstage, that of chunk c - 1, whose reads are done) around its first MFMAs, then reads the
//    chunk's second step from the same buffer (bcur);
//  - the second waits for chunk c + 1 and reads its first step (buffer bnext).
// The reads are split into `next` after the last MFMAs. The cross products go to acc_x, hi x hi
// to acc.
template <bool SECOND>
__device__ __forceinline__ void rt_step(RtLds &sm, uint32_t wave, uint32_t c, uint32_t nc, uint32_t m, uint32_t h,
                                        const char *xk, const char *wk, const uint32_t xoff[4],
                                        const uint32_t woff[4 * RT_TW], uint32_t bstage, uint32_t bcur, uint32_t bnext,
                                        const RtOps &cur, RtOps &next, f32x16 (&acc)[RT_TW], f32x16 (&acc_x)[RT_TW],
                                        float &xmax) {
    const bool stage = !SECOND && c + RT_NBUF - 1u < nc;
    const uint32_t lx = gg_lds_addr(&sm.x[wave][bstage][0]), lw = gg_lds_addr(&sm.w[wave][bstage][0]);
#pragma unroll
    for (int j = 0; j < RT_TW; ++j) {
        acc_x[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur.xh, cur.wl[j], acc_x[j], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (stage) {
            if (j == 0) {
#pragma unroll
                for (int i = 0; i < 4; ++i) gg_dma16(lx + (uint32_t)i * 1024u, xk, xoff[i]);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) gg_dma16(lw + (uint32_t)(4 + i) * 1024u, wk, woff[4 + i]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur.xh, cur.wh[j], acc[j], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (stage && j == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) gg_dma16(lw + (uint32_t)i * 1024u, wk, woff[i]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    const bool more = !SECOND || c + 1u < nc;
    if (SECOND && more) rt_wait(c + RT_NBUF <= nc ? 1u : 0u);  // chunk c + 2 may stay in flight
    __builtin_amdgcn_sched_barrier(0);
    RtRaw raw;
    if (more) rt_read(sm, wave, SECOND ? bnext : bcur, SECOND ? 0u : 1u, m, h, raw);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < RT_TW; ++j) {
        acc_x[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur.xl, cur.wh[j], acc_x[j], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (more) rt_split(raw, next, xmax);
    // The operands stay allocated to the end of the step: a VGPR written while an MFMA that
    // reads it is in flight holds the write (and the wave) until the MFMA has read it.
    const gd_u32x4 k0 = __builtin_bit_cast(gd_u32x4, cur.xh), k1 = __builtin_bit_cast(gd_u32x4, cur.xl);
    asm volatile("" ::"v"(k0[0]), "v"(k0[1]), "v"(k0[2]), "v"(k0[3]), "v"(k1[0]), "v"(k1[1]), "v"(k1[2]), "v"(k1[3]));
#pragma unroll
    for (int j = 0; j < RT_TW; ++j) {
        const gd_u32x4 k2 = __builtin_bit_cast(gd_u32x4, cur.wh[j]), k3 = __builtin_bit_cast(gd_u32x4, cur.wl[j]);
        asm volatile("" ::"v"(k2[0]), "v"(k2[1]), "v"(k2[2]), "v"(k2[3]), "v"(k3[0]), "v"(k3[1]), "v"(k3[2]), "v"(k3[3]));
    }
}

// Sixteen values as binary16 pairs (32 bytes) at dst; `bad` records a value outside the range.
__device__ __forceinline__ void rt_store_h16(uint32_t *dst, const float (&v)[16], bool &bad) {
    gd_u32x4 o[2];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        bad |= !gd_half_ok(v[2 * j]) || !gd_half_ok(v[2 * j + 1]);
        const uint32_t h0 = __builtin_bit_cast(uint16_t, (_Float16)v[2 * j]);
        const uint32_t h1 = __builtin_bit_cast(uint16_t, (_Float16)v[2 * j + 1]);
        o[j >> 2][j & 3] = h0 | (h1 << 16);
    }
    gd_u32x4 *d = reinterpret_cast<gd_u32x4 *>(dst);
    d[0] = o[0];
    d[1] = o[1];
}

// One group: waves 0..3 the router tile, waves 4..7 the rotation share. The name expands before
// the pipeline macro stringises it.
#define RT_DEFINE(NAME, OCC) GD_PIPELINE_NAMED_OCC(NAME, 512, OCC)
RT_DEFINE(RT_PIPELINE, RT_TW == 1 ? 4 : 2) {
    __shared__ RtLds sm;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t n = a.c[2], E = a.c[3], NE = a.c[6];
    const float *X = gd_buf<const float>(a, a.c[0]) + a.c[1];
    const uint32_t t0 = blockIdx.x * 32u, z = blockIdx.z;
    // The group's first expert; in the wide build wave w takes experts r0 + 32 RT_TW w ...
    const uint32_t r0 = blockIdx.y * (RT_TW == 1 ? 32u : 32u * RT_TW * RT_WAVES);
    const uint32_t rw = RT_TW == 1 ? r0 : r0 + 32u * RT_TW * wave;
    const uint32_t S = a.c[18] > 1u ? a.c[18] : 1u, ES = E / S;
    const uint32_t m = lane & 31u, h = lane >> 5;
    const float *unscale = gd_buf<const float>(a, a.c[4]) + a.c[5] + (size_t)NE * E;
    const bool has_bias = a.c[7] != 0xffffffffu && z == 0u;
    float *L = gd_buf<float>(a, a.c[9]) + a.c[10] + (size_t)z * n * NE;
    f32x16 acc[RT_TW];
#pragma unroll
    for (int j = 0; j < RT_TW; ++j) acc[j] = (f32x16){};

    if (wave < RT_WAVES && rw < NE) {  // uniform per wave; the wide build's waves past n_expert idle
        // Router tile: K quarter `wave` of range z (one-tile build) or all of range z.
        const float *W = gd_buf<const float>(a, a.c[4]) + a.c[5];
        const uint32_t kq = RT_TW == 1 ? z * ES + wave * (ES / 4u) : z * ES;
        const uint32_t nc = (RT_TW == 1 ? ES / 4u : ES) / RT_KC;
        uint32_t xoff[4], woff[4 * RT_TW];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t r = 8u * (uint32_t)i + (lane >> 3), q = rt_pos(lane & 7u, r);
            xoff[i] = (min(t0 + r, n - 1u) * E + kq + 4u * q) * 4u;
        }
#pragma unroll
        for (int i = 0; i < 4 * RT_TW; ++i) {
            const uint32_t r = 8u * (uint32_t)i + (lane >> 3), q = rt_pos(lane & 7u, r);
            woff[i] = (min(rw + r, NE - 1u) * E + kq + 4u * q) * 4u;
        }
        const char *xb = reinterpret_cast<const char *>(X), *wb = reinterpret_cast<const char *>(W);
        for (uint32_t c = 0; c < nc && c < RT_NBUF - 1u; ++c)
            rt_stage(sm, wave, c, xb + c * RT_KC * 4u, wb + c * RT_KC * 4u, xoff, woff);
        // Rows beyond n or n_expert were staged as copies of the last row (finite values); they
        // reach only tile rows and columns that are never stored.
        RtOps ops[2];
        f32x16 acc_x[RT_TW];
#pragma unroll
        for (int j = 0; j < RT_TW; ++j) acc_x[j] = (f32x16){};
        float xmax = 0.f;
        rt_wait(min(nc - 1u, RT_NBUF - 2u));  // chunk 1 may be in flight
        {
            RtRaw raw;
            rt_read(sm, wave, 0, 0, m, h, raw);
            rt_split(raw, ops[0], xmax);
        }
        // Chunk c sits in buffer c % RT_NBUF (b); its first step stages chunk c + RT_NBUF - 1
        // into chunk c - 1's buffer.
        uint32_t b = 0;
        for (uint32_t c = 0; c < nc; ++c) {
            const uint32_t bn = b + 1u == RT_NBUF ? 0u : b + 1u, bs = b == 0u ? RT_NBUF - 1u : b - 1u;
            const uint32_t kb = (c + RT_NBUF - 1u) * RT_KC * 4u;
            rt_step<false>(sm, wave, c, nc, m, h, xb + kb, wb + kb, xoff, woff, bs, b, bn, ops[0], ops[1], acc, acc_x,
                           xmax);
            rt_step<true>(sm, wave, c, nc, m, h, xb + kb, wb + kb, xoff, woff, bs, b, bn, ops[1], ops[0], acc, acc_x,
                          xmax);
            b = bn;
        }
        gd_range_flag(a.table, a.c[19], !(xmax <= 65504.0f));
        // Accumulator register r holds tile row 8 (r / 4) + 4 h + r % 4, column m.
#pragma unroll
        for (int j = 0; j < RT_TW; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[j][r] += acc_x[j][r] * (1.0f / 2048.0f);
        if (RT_TW > 1) {
            // Wide build: the wave's tiles are whole logits of plane z.
#pragma unroll
            for (int j = 0; j < RT_TW; ++j) {
                const uint32_t col = rw + 32u * (uint32_t)j + m;
                if (col < NE) {
                    const float us = unscale[col];
                    const float bias = has_bias ? gd_buf<const float>(a, a.c[7])[a.c[8] + col] : 0.f;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const uint32_t t = t0 + (uint32_t)((r / 4) * 8 + (r % 4)) + 4u * h;
                        if (t < n) L[(size_t)t * NE + col] = acc[j][r] * us + bias;
                    }
                }
            }
        }
    } else if (wave >= RT_WAVES) {
        // Rotation share of this group's waves 4..7: each wave transforms eight 128-blocks at a
        // time, an 8-lane group per block holding 16 consecutive values per lane
        // (gd_fwht128_x16); the blocks b = 8 (first + waves j) + lane / 8. Two such steps run
        // together, every load of both issued before the first transform.
        const uint32_t nblk = E / 128u, total = n * nblk;
        const uint32_t waves = gridDim.x * gridDim.y * gridDim.z * RT_WAVES;
        const uint32_t first = ((z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * RT_WAVES + (wave - RT_WAVES);
        const bool has_signs = a.c[11] != 0xffffffffu;
        const uint32_t *S = has_signs ? gd_buf<const uint32_t>(a, a.c[11]) + a.c[12] : nullptr;
        const uint32_t *XU = reinterpret_cast<const uint32_t *>(X);
        uint32_t *XH = gd_buf<uint32_t>(a, a.c[13]) + a.c[14];
        const uint32_t l8 = lane & 7u;
        bool bad = false;
        for (uint32_t g = first; g * 8u < total; g += 2u * waves) {
            gd_u32x4 xv[2][4], sv[2][4];
            uint32_t tk[2], bk[2];
            bool ok[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const uint32_t b = (g + (uint32_t)u * waves) * 8u + (lane >> 3);
                ok[u] = b < total;  // the same for the 8 lanes of a block
                const uint32_t bb = ok[u] ? b : 0u;  // a block that exists: loaded, not used
                tk[u] = bb / nblk;
                bk[u] = bb - tk[u] * nblk;
                const uint32_t i = bk[u] * 128u + 16u * l8;
                gd_gu32x4 *src = gd_global4(XU + (size_t)tk[u] * E + i);
#pragma unroll
                for (int q = 0; q < 4; ++q) xv[u][q] = src[q];
                if (has_signs) {
                    gd_gu32x4 *sg = gd_global4(S + i);
#pragma unroll
                    for (int q = 0; q < 4; ++q) sv[u][q] = sg[q];
                }
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                if (!ok[u]) continue;
                const uint32_t t = tk[u], blk = bk[u];
                float v[16];
#pragma unroll
                for (int j = 0; j < 16; ++j) v[j] = gd_bits_f32(xv[u][j >> 2][j & 3]);
                if (a.c[15]) rt_store_h16(gd_buf<uint32_t>(a, a.c[16]) + a.c[17] + (size_t)t * (E / 2u) + blk * 64u + 8u * l8, v, bad);
                // The DPP stages read lanes of the same 8-lane group only, and whole groups share
                // b < total, so every source lane is active.
                if (has_signs) {
#pragma unroll
                    for (int j = 0; j < 16; ++j) v[j] *= gd_bits_f32(sv[u][j >> 2][j & 3]);
                    gd_fwht128_x16(v, l8);
#pragma unroll
                    for (int j = 0; j < 16; ++j) v[j] *= GD_INV_SQRT128;
                }
                rt_store_h16(XH + (size_t)t * (E / 2u) + blk * 64u + 8u * l8, v, bad);
            }
        }
        gd_range_flag(a.table, a.c[19], bad);
        // The chunk histogram that moe_prefill_topk counts into, zeroed for this call: word
        // range of this rotation wave.
        if (a.c[20]) {
            uint32_t *H = gd_buf<uint32_t>(a, a.c[20]) + a.c[21];
            for (uint32_t i = first * 64u + lane; i < a.c[22]; i += waves * 64u) H[i] = 0u;
        }
    }
    if (RT_TW == 1) {
        // One-tile build: the four K quarters added in wave order. The waves' buffers are free:
        // their last LDS reads were waited for before their last MFMAs.
        float *red = reinterpret_cast<float *>(&sm.x[0][0][0]);  // red(w) at sm.x[w][0]
        constexpr uint32_t kRedStride = sizeof(sm.x[0]) / 4u;   // floats from one wave's buffers to the next
        if (wave < RT_WAVES) {
#pragma unroll
            for (int r = 0; r < 16; ++r) red[wave * kRedStride + ((r / 4) * 8 + h * 4 + (r % 4)) * 32 + m] = acc[0][r];
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const uint32_t idx = tid + 512u * q, i = idx >> 5, j = idx & 31u;
            const uint32_t t = t0 + i, r = r0 + j;
            if (t < n && r < NE) {
                float v = red[idx];
#pragma unroll
                for (int w = 1; w < RT_WAVES; ++w) v += red[w * kRedStride + idx];
                v *= unscale[r];
                if (has_bias) v += gd_buf<const float>(a, a.c[7])[a.c[8] + r];
                L[(size_t)t * NE + r] = v;
            }
        }
    }
}
