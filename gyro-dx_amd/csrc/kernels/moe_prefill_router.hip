// Prefill path, step 1: router logits of many tokens on fp32 MFMA, and the rotated expert
// input in binary16.
//   logits[t][r] = W_r[r] . x[t] (+ bias[r])          src/engine.zig:526 (kernels.matmul)
//   xh16[t]      = H_128 (gate_signs * x[t]) per 128-block, as binary16 pairs
//                                                      src/engine.zig:547-551
// Group (bx, by, bz) computes the 32 x 32 logit tile of tokens 32 bx.. and experts 32 by.. over
// K range bz of S (the K split, chosen by the host so that small batches still fill the GPU)
// with v_mfma_f32_32x32x2_f32; its waves 0..3 split the range into quarters and their partial
// tiles are added in wave order through LDS. Range bz writes logit plane bz; the top-k kernel
// adds the S planes in plane order. The MFMA operands take one row per lane, so each of these
// waves stages its own 16-wide K chunks of the 32 token rows and the 32 router rows into LDS
// first: direct global-to-LDS loads (4 lanes per 64-byte row, whole rows per load), the
// 16-byte chunk q of row r stored at position q ^ ((r / 2) % 4), four chunks ahead in five
// buffers per wave; only the wave's own load count is waited for, so the K loop has no barrier.
// A group takes 80 KB of LDS and at most 128 VGPRs, so that grids of more than one group per
// CU (4096 tokens: 1024 groups) run two groups per CU. A wave's MFMA holds back that wave's
// following instructions until it has nearly finished (other waves issue meanwhile), so each
// chunk's eight MFMAs carry the chunk's other work one piece at a time: a staging load after
// each of the first four, the reads of chunk c + 1 (into the other of two operand sets, no
// copies) after the next two. Lane half h takes k + 4h .. k + 4h + 3 of every 8 for both operands, so
// every product x[t][k] W[r][k] enters the sum once. Waves 4..7 meanwhile rotate: all
// n * E/128 blocks are spread over the rotation waves of the grid, eight blocks per wave at a
// time, so the rotation's memory traffic and VALU work overlap the MFMA chains on the same
// SIMDs.
// Grid: (ceil(n / 32), ceil(n_expert / 32), S); 512 threads, 80 KB of LDS (two groups per CU).
// Requires E % (128 S) == 0.
// Constants: 0 x_uav 1 x_off (words; rows of E floats) 2 n_tok 3 E 4 router_srv 5 router_off
// 6 n_expert 7 bias_srv (0xffffffff: none) 8 bias_off 9 logits_uav 10 logits_off
// 11 signs_srv (0xffffffff: no rotation, plain conversion) 12 signs_off 13 xh16_uav
// 14 xh16_off (words) 15 x16 (1: also write the unrotated input as binary16, for the shared
// expert; zero when the caller passes 15 constants) 16 x16_uav 17 x16_off (words) 18 S (0 or
// 1: no split; plane z at logits_off + z n n_expert; the bias enters plane 0) 19 range flag
// (table index of a word set to 1 when a value written as binary16 is outside its range; 0:
// none) 20 hist_uav (0: none) 21 hist_off (words) 22 hist_words: the rotation waves zero these
// words of moe_prefill_topk's chunk histogram.
#include "ggemm.h"
#include "fwht.h"

#define RT_WAVES 4
#define RT_KC 16    // K per staged chunk
#define RT_NBUF 5    // chunks c .. c + 4 of a wave in LDS: four chunks (16 KB) in flight
#define RT_LOADS 4   // global-to-LDS loads per chunk: two of token rows, two of router rows

// 80 KB, so that two groups share a CU: the staging buffers of the four K waves; after its K
// loop a wave's partial tile (4 KB, fp32) goes over its own first two activation buffers.
struct __attribute__((aligned(16))) RtLds {
    gd_u32x4 x[RT_WAVES][RT_NBUF][32 * RT_KC / 4];  // 32 rows x 64 bytes
    gd_u32x4 w[RT_WAVES][RT_NBUF][32 * RT_KC / 4];
};
static_assert(sizeof(RtLds) == 81920, "two groups fill the CU's 160 KB");
static_assert(sizeof(RtLds::x[0]) >= 32 * 32 * 4, "a wave's partial tile fits its activation buffers");

// Swizzled position of 16-byte chunk q of staged row r: the chunk that the 8 lanes of rows
// m .. m + 7 read at one index sits in 8 different 16-byte bank groups.
__device__ __forceinline__ uint32_t rt_pos(uint32_t q, uint32_t r) { return q ^ ((r >> 1) & 3u); }

// Waits until chunk c's loads have landed, with `ahead` later chunks (RT_LOADS loads each) in
// flight.
__device__ __forceinline__ void rt_wait(uint32_t ahead) {
    switch (ahead) {
        case 3: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
        case 2: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
        case 1: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
        default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    }
}

// Stages chunk c (K = kq + 16 c ..) of this wave's 32 token rows and 32 router rows: 2 + 2
// loads, lane l of load i carrying row 16 i + l / 4, position l % 4.
__device__ __forceinline__ void rt_stage(RtLds &sm, uint32_t wave, uint32_t buf, const void *xbase,
                                         const void *wbase, const uint32_t xoff[2], const uint32_t woff[2],
                                         uint32_t kbytes) {
    const uint32_t lx = gg_lds_addr(&sm.x[wave][buf][0]), lw = gg_lds_addr(&sm.w[wave][buf][0]);
#pragma unroll
    for (int i = 0; i < 2; ++i) gg_dma16(lx + (uint32_t)i * 1024u, xbase, xoff[i] + kbytes);
#pragma unroll
    for (int i = 0; i < 2; ++i) gg_dma16(lw + (uint32_t)i * 1024u, wbase, woff[i] + kbytes);
}

// Operands of one staged chunk for this lane (row m, lane half h): two float4 of the token row
// and two of the router row, k = 8 j + 4 h .. + 3 of the chunk for j = 0, 1.
struct RtOps {
    float4 x[2], w[2];
};
__device__ __forceinline__ void rt_read(const RtLds &sm, uint32_t wave, uint32_t buf, uint32_t m, uint32_t h, RtOps &o) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t p = rt_pos(2u * (uint32_t)j + h, m);
        o.x[j] = __builtin_bit_cast(float4, sm.x[wave][buf][m * 4u + p]);
        o.w[j] = __builtin_bit_cast(float4, sm.w[wave][buf][m * 4u + p]);
    }
}
// Chunk c's eight MFMAs (operands `cur`) with the chunk's other work between them, so that the
// matrix pipe always has the next MFMA waiting: the four loads staging chunk c + 4 (into the
// buffer of chunk c - 1, read into registers two chunks ago) one after each of the first four
// MFMAs, then the wait for chunk c + 1 and its reads into `next`, two after each of the next
// two. The following chunk's MFMAs use `next` once the two MFMAs after the reads have issued.
// STEADY: chunks c + 1 .. c + 4 are all in flight (c + 4 < nc), so the wait is one immediate
// count; otherwise `ahead` (the chunks issued after chunk c + 1) picks it.
template <bool STEADY>
__device__ __forceinline__ void rt_chunk(RtLds &sm, uint32_t wave, uint32_t c, uint32_t nc, uint32_t m, uint32_t h,
                                         const void *xbase, const void *wbase, const uint32_t xoff[2],
                                         const uint32_t woff[2], const RtOps &cur, RtOps &next, f32x16 &acc) {
    const bool stage = STEADY || c + 4u < nc;
    const uint32_t buf = (c + 4u) % RT_NBUF, kbytes = (c + 4u) * RT_KC * 4u;
    const uint32_t lx = gg_lds_addr(&sm.x[wave][buf][0]), lw = gg_lds_addr(&sm.w[wave][buf][0]);
    {
        const float *x0 = reinterpret_cast<const float *>(&cur.x[0]), *w0 = reinterpret_cast<const float *>(&cur.w[0]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(x0[q], w0[q], acc, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (stage) {
                if (q < 2) gg_dma16(lx + (uint32_t)q * 1024u, xbase, xoff[q] + kbytes);
                else gg_dma16(lw + (uint32_t)(q - 2) * 1024u, wbase, woff[q - 2] + kbytes);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    const bool more = STEADY || c + 1u < nc;
    if (STEADY) {
        asm volatile("s_waitcnt vmcnt(12)" ::: "memory");  // chunks c + 2 .. c + 4 in flight
    } else if (more) {
        rt_wait(min(nc - 2u - c, RT_NBUF - 2u));
    }
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t rb = (c + 1u) % RT_NBUF;
    const float *x1 = reinterpret_cast<const float *>(&cur.x[1]), *w1 = reinterpret_cast<const float *>(&cur.w[1]);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(x1[q], w1[q], acc, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (more) {
            const uint32_t p = rt_pos(2u * (uint32_t)q + h, m);
            next.x[q] = __builtin_bit_cast(float4, sm.x[wave][rb][m * 4u + p]);
            next.w[q] = __builtin_bit_cast(float4, sm.w[wave][rb][m * 4u + p]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(x1[2], w1[2], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(x1[3], w1[3], acc, 0, 0, 0);
    // The operands stay allocated to the end of the chunk: a VGPR written while an MFMA that
    // reads it is in flight holds the write (and the wave) until the MFMA has read it, about 27
    // of its 64 cycles; left free, the compiler reuses them for address arithmetic right after
    // the MFMA that reads them.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        asm volatile("" ::"v"(cur.x[j].x), "v"(cur.x[j].y), "v"(cur.x[j].z), "v"(cur.x[j].w));
        asm volatile("" ::"v"(cur.w[j].x), "v"(cur.w[j].y), "v"(cur.w[j].z), "v"(cur.w[j].w));
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

GD_PIPELINE_NAMED_OCC(moe_prefill_router, 512, 4) {
    __shared__ RtLds sm;
    float *red = reinterpret_cast<float *>(&sm.x[0][0][0]);  // red(w) at sm.x[w][0]
    constexpr uint32_t kRedStride = sizeof(sm.x[0]) / 4u;   // floats from one wave's buffers to the next
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t n = a.c[2], E = a.c[3], NE = a.c[6];
    const float *X = gd_buf<const float>(a, a.c[0]) + a.c[1];
    const uint32_t t0 = blockIdx.x * 32u, r0 = blockIdx.y * 32u, z = blockIdx.z;
    const uint32_t S = a.c[18] > 1u ? a.c[18] : 1u, ES = E / S;
    const uint32_t m = lane & 31u, h = lane >> 5;
    f32x16 acc = {};

    if (wave < RT_WAVES) {
        // Router tile, K quarter `wave`.
        const float *W = gd_buf<const float>(a, a.c[4]) + a.c[5];
        const uint32_t kq = z * ES + wave * (ES / 4u), nc = ES / 4u / RT_KC;
        uint32_t xoff[2], woff[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t r = 16u * (uint32_t)i + (lane >> 2), q = rt_pos(lane & 3u, r);
            xoff[i] = (min(t0 + r, n - 1u) * E + kq + 4u * q) * 4u;
            woff[i] = (min(r0 + r, NE - 1u) * E + kq + 4u * q) * 4u;
        }
        for (uint32_t c = 0; c < nc && c < RT_NBUF - 1u; ++c) rt_stage(sm, wave, c, X, W, xoff, woff, c * RT_KC * 4u);
        // Rows beyond n or n_expert were staged as copies of the last row (finite values); they
        // reach only tile rows and columns that are never stored.
        RtOps ops[2];
        rt_wait(min(nc - 1u, RT_NBUF - 2u));  // chunks 1 .. 3 may be in flight
        rt_read(sm, wave, 0, m, h, ops[0]);
        uint32_t c = 0;
        for (; c + 5u < nc; c += 2u) {  // chunks c + 4 and c + 5 exist: steady state
            rt_chunk<true>(sm, wave, c, nc, m, h, X, W, xoff, woff, ops[0], ops[1], acc);
            rt_chunk<true>(sm, wave, c + 1u, nc, m, h, X, W, xoff, woff, ops[1], ops[0], acc);
        }
        for (; c < nc; c += 2u) {
            rt_chunk<false>(sm, wave, c, nc, m, h, X, W, xoff, woff, ops[0], ops[1], acc);
            if (c + 1u < nc) rt_chunk<false>(sm, wave, c + 1u, nc, m, h, X, W, xoff, woff, ops[1], ops[0], acc);
        }
        // Accumulator register r holds tile row 8 (r / 4) + 4 h + r % 4, column m. The wave's
        // buffers are free: its last LDS reads were waited for before its last MFMAs.
#pragma unroll
        for (int r = 0; r < 16; ++r) red[wave * kRedStride + ((r / 4) * 8 + h * 4 + (r % 4)) * 32 + m] = acc[r];
    } else {
        // Rotation share of this group's waves 4..7: each wave transforms eight 128-blocks at a
        // time, an 8-lane group per block holding 16 consecutive values per lane
        // (gd_fwht128_x16); the blocks b = 8 (first + waves j) + lane / 8.
        const uint32_t nblk = E / 128u, total = n * nblk;
        const uint32_t waves = gridDim.x * gridDim.y * gridDim.z * RT_WAVES;
        const uint32_t first = ((z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * RT_WAVES + (wave - RT_WAVES);
        const bool has_signs = a.c[11] != 0xffffffffu;
        const float *S = has_signs ? gd_buf<const float>(a, a.c[11]) + a.c[12] : nullptr;
        uint32_t *XH = gd_buf<uint32_t>(a, a.c[13]) + a.c[14];
        const uint32_t l8 = lane & 7u;
        bool bad = false;
        for (uint32_t g = first; g * 8u < total; g += waves) {
            const uint32_t b = g * 8u + (lane >> 3);
            if (b < total) {
                const uint32_t t = b / nblk, blk = b - t * nblk, i = blk * 128u + 16u * l8;
                float v[16];
                const float4 *src = reinterpret_cast<const float4 *>(X + (size_t)t * E + i);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 f = src[q];
                    v[4 * q] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
                }
                if (a.c[15]) rt_store_h16(gd_buf<uint32_t>(a, a.c[16]) + a.c[17] + (size_t)t * (E / 2u) + blk * 64u + 8u * l8, v, bad);
                if (has_signs) {
                    const float4 *sg = reinterpret_cast<const float4 *>(S + i);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float4 f = sg[q];
                        v[4 * q] *= f.x; v[4 * q + 1] *= f.y; v[4 * q + 2] *= f.z; v[4 * q + 3] *= f.w;
                    }
                }
                // The DPP stages read lanes of the same 8-lane group only, and whole groups share
                // b < total, so every source lane is active.
                if (has_signs) {
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
    __syncthreads();
    const bool has_bias = a.c[7] != 0xffffffffu && z == 0u;
    float *L = gd_buf<float>(a, a.c[9]) + a.c[10] + (size_t)z * n * NE;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint32_t idx = tid + 512u * q, i = idx >> 5, j = idx & 31u;
        const uint32_t t = t0 + i, r = r0 + j;
        if (t < n && r < NE) {
            float v = red[idx];
#pragma unroll
            for (int w = 1; w < RT_WAVES; ++w) v += red[w * kRedStride + idx];
            if (has_bias) v += gd_buf<const float>(a, a.c[7])[a.c[8] + r];
            L[(size_t)t * NE + r] = v;
        }
    }
}
