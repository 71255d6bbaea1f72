// Prefill path: the shared expert of src/engine.zig:644-653 over many tokens, as two dense fp16
// MFMA GEMMs with the bf16 weights held as binary16 copies scaled by powers of two (exact for
// every bf16 weight whose scaled magnitude is a normal binary16; the host picks each matrix's
// scale so that its largest |weight| lands in [2^14, 2^15)).
//   mode 0 (gate/up):  a[t][j] = silu(g) * u, g = W_g[j] . x[t], u = W_u[j] . x[t]
//                      (binary16 a, the A operand of mode 1)
//   mode 1 (down):     o[t][r] = W_d[r] . a[t]  (fp32)
// The activations are binary16 rows (x unrotated, from moe_prefill_router).
//
// Group: 32 tokens x 128 weight rows, four waves, K blocks of 64 in a five-buffer pipeline of
// direct global-to-LDS loads (ggemm.h) four blocks ahead. Mode 0 stages gate rows j0 .. j0 + 63
// and up rows j0 .. j0 + 63 (a columns j0 .. + 63); mode 1 stages down rows c0 .. c0 + 127.
// Wave w computes the 32 tokens against staged rows 32 w .. + 31 with one
// v_mfma_f32_32x32x16_f16 per K-step, so in mode 0 waves 0, 1 hold gate and waves 2, 3 the
// matching up products. 32-token groups give 512-token calls 256 groups, one per CU. LDS rows
// are 128 bytes (8 chunks of 16); chunk c of row r sits at position c ^ ((r / 2) % 8), so the 16
// lanes of one ds_read_b128 pass (rows r .. r + 15 at one chunk) cover all 64 banks.
// Grid: mode 0 (SF / 64, ceil(n / 32)), mode 1 (E / 128, ceil(n / 32)); 256 threads; 100 KB LDS.
// Requires K % 64 == 0 and the A rows' and weight rows' lengths multiples of 8 values.
// Constants: 0 mode 1 a_uav 2 a_off (words) 3 lda (values per A row) 4 w_srv 5 w_off (words)
// 6 K 7 out_uav 8 out_off (words) 9 n_tok 10 up_row0 (mode 0: first up row, = SF) 11 scale0
// (fp32 bits: 2^-k of the gate or the down matrix) 12 scale1 (the up matrix) 13 ldo (values per
// output row) 14 range flag (mode 0: table index of a word set to 1 when a SwiGLU value of a token
// row leaves the binary16 range; 0: none).
#include "ggemm.h"

#define SH_TM 32
#define SH_TN 128
#define SH_NBUF 5  // K blocks kb .. kb + 4 in LDS: four blocks ahead

struct __attribute__((aligned(16))) ShLds {
    gd_u32x4 a[SH_NBUF][SH_TM * 8];
    gd_u32x4 b[SH_NBUF][SH_TN * 8];
};

// Start of K block kb: at most the 5 loads per block (1 activation, 4 weight) of blocks
// kb + 1 .. kb + 3 are this wave's outstanding ones.
__device__ __forceinline__ void sh_sync(uint32_t kb, uint32_t nk) {
    switch (min(nk - 1u - kb, SH_NBUF - 2u)) {
        case 3: gg_sync<15>(); break;
        case 2: gg_sync<10>(); break;
        case 1: gg_sync<5>(); break;
        default: gg_sync<0>(); break;
    }
}

// Block kb into buffer buf: wave w issues activation load w and weight loads 4 w .. 4 w + 3;
// load L carries staged rows 8 L .. 8 L + 7 (lane l: row 8 L + l / 8, position l % 8).
__device__ __forceinline__ void sh_stage(ShLds &sm, uint32_t buf, uint32_t wave, const void *abase, uint32_t aoff,
                                         const void *wbase, const uint32_t woff[4], uint32_t kb) {
    const uint32_t la = gg_lds_addr(&sm.a[buf][0]) + wave * 1024u, lw = gg_lds_addr(&sm.b[buf][0]) + wave * 4096u;
    gg_dma16(la, abase, aoff + kb * 128u);
#pragma unroll
    for (int i = 0; i < 4; ++i) gg_dma16(lw + (uint32_t)i * 1024u, wbase, woff[i] + kb * 128u);
}

__device__ __forceinline__ f16x8 sh_read(const gd_u32x4 *rows, uint32_t r, uint32_t c) {
    return __builtin_bit_cast(f16x8, rows[r * 8u + (c ^ ((r >> 1) & 7u))]);
}

template <int BUF>
__device__ __forceinline__ void sh_step(ShLds &sm, uint32_t kb, uint32_t nk, uint32_t wave, uint32_t m, uint32_t h,
                                        const void *abase, uint32_t aoff, const void *wbase, const uint32_t woff[4],
                                        f32x16 &acc) {
    sh_sync(kb, nk);
    if (kb + SH_NBUF - 1u < nk) sh_stage(sm, (BUF + SH_NBUF - 1) % SH_NBUF, wave, abase, aoff, wbase, woff, kb + SH_NBUF - 1u);
    const uint32_t rb = wave * 32u + m;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const uint32_t c = 2u * (uint32_t)s + h;
        const f16x8 av = sh_read(sm.a[BUF], m, c);
        const f16x8 bv = sh_read(sm.b[BUF], rb, c);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc, 0, 0, 0);
    }
}

GD_PIPELINE_NAMED(moe_prefill_shared, 256) {
    __shared__ ShLds sm;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t mode = a.c[0], lda = a.c[3], K = a.c[6], n = a.c[9], ldo = a.c[13];
    const uint32_t t0 = blockIdx.y * SH_TM, n0 = blockIdx.x * (mode == 0u ? 64u : SH_TN);
    const void *abase = gd_buf<const uint32_t>(a, a.c[1]) + a.c[2];
    const void *wbase = gd_buf<const uint32_t>(a, a.c[4]) + a.c[5];
    const uint32_t nk = K / 64u;

    // Lane offsets of the staged rows: activation row t0 + r (rows past n repeat the last one),
    // weight row n0 + r (mode 1) or gate row n0 + r, up row up_row0 + n0 + r - 64 (mode 0); the
    // global chunk of LDS position p of row r is p ^ ((r / 2) % 8).
    uint32_t aoff, woff[4];
    {
        const uint32_t r = wave * 8u + (lane >> 3), q = (lane & 7u) ^ ((r >> 1) & 7u);
        aoff = min(t0 + r, n - 1u) * lda * 2u + q * 16u;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t r = (wave * 4u + (uint32_t)i) * 8u + (lane >> 3), q = (lane & 7u) ^ ((r >> 1) & 7u);
        const uint32_t row = mode == 0u && r >= 64u ? a.c[10] + n0 + r - 64u : n0 + r;
        woff[i] = row * K * 2u + q * 16u;
    }
    sh_stage(sm, 0, wave, abase, aoff, wbase, woff, 0);
    for (uint32_t b = 1; b < nk && b < SH_NBUF - 1u; ++b) sh_stage(sm, b, wave, abase, aoff, wbase, woff, b);

    const uint32_t m = lane & 31u, h = lane >> 5;
    f32x16 acc = {};
    for (uint32_t kb = 0; kb < nk; kb += SH_NBUF) {
        sh_step<0>(sm, kb, nk, wave, m, h, abase, aoff, wbase, woff, acc);
        if (kb + 1u < nk) sh_step<1>(sm, kb + 1u, nk, wave, m, h, abase, aoff, wbase, woff, acc);
        if (kb + 2u < nk) sh_step<2>(sm, kb + 2u, nk, wave, m, h, abase, aoff, wbase, woff, acc);
        if (kb + 3u < nk) sh_step<3>(sm, kb + 3u, nk, wave, m, h, abase, aoff, wbase, woff, acc);
        if (kb + 4u < nk) sh_step<4>(sm, kb + 4u, nk, wave, m, h, abase, aoff, wbase, woff, acc);
    }
    gg_sync<0>();  // every wave is done with the buffers

    // Accumulator register r: token row 8 (r / 4) + 4 h + r % 4, staged row 32 w + m.
    const uint32_t rbase = h * 4u;
    if (mode == 0u) {
        // Up waves: u (scaled back) into LDS [32 tokens][64 columns] fp32; gate waves: silu(g) * u
        // rounded to binary16 into LDS rows of 64 values; then 16-byte row chunks to a[t][n0 ..].
        // Gate wave w (0, 1) and up wave w + 2 hold columns 32 w .. + 31.
        float *ub = reinterpret_cast<float *>(&sm.a[0][0]);
        _Float16 *ab = reinterpret_cast<_Float16 *>(&sm.b[0][0]);
        static_assert(sizeof(sm.a) >= SH_TM * 64 * 4, "u rows fit the activation buffers");
        const float sg = gd_bits_f32(a.c[11]), su = gd_bits_f32(a.c[12]);
        const uint32_t col = (wave & 1u) * 32u + m;
        if (wave >= 2u) {
#pragma unroll
            for (int r = 0; r < 16; ++r) ub[(rbase + (r / 4) * 8u + (r % 4)) * 64u + col] = acc[r] * su;
        }
        __syncthreads();
        if (wave < 2u) {
            bool bad = false;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t i = rbase + (r / 4) * 8u + (r % 4);
                const float v = gd_silu_rcp(acc[r] * sg) * ub[i * 64u + col];
                bad |= t0 + i < n && !gd_half_ok(v);
                ab[i * 64u + col] = (_Float16)v;
            }
            gd_range_flag(a.table, a.c[14], bad);
        }
        __syncthreads();
        uint32_t *out = gd_buf<uint32_t>(a, a.c[7]) + a.c[8];
        {
            const uint32_t i = tid >> 3, c = tid & 7u;  // 32 token rows of 8 chunks
            if (t0 + i < n)
                *reinterpret_cast<gd_u32x4 *>(out + (size_t)(t0 + i) * (ldo / 2u) + n0 / 2u + c * 4u) =
                    reinterpret_cast<const gd_u32x4 *>(ab)[i * 8u + c];
        }
    } else {
        // o (scaled back) into LDS [32 tokens][128 columns] fp32, then 16-byte row chunks to
        // o[t][n0 ..].
        float *res = reinterpret_cast<float *>(&sm.a[0][0]);
        static_assert(sizeof(sm) >= SH_TM * SH_TN * 4u, "result rows fit the K-loop buffers");
        const float sd = gd_bits_f32(a.c[11]);
#pragma unroll
        for (int r = 0; r < 16; ++r) res[(rbase + (r / 4) * 8u + (r % 4)) * 128u + wave * 32u + m] = acc[r] * sd;
        __syncthreads();
        float *out = gd_buf<float>(a, a.c[7]) + a.c[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t idx = tid + 256u * q, i = idx >> 5, c = idx & 31u;
            if (t0 + i < n)
                *reinterpret_cast<float4 *>(out + (size_t)(t0 + i) * ldo + n0 + c * 4u) =
                    *reinterpret_cast<const float4 *>(res + i * 128u + c * 4u);
        }
    }
}
