// Prefill path, step 4: grouped gate/up GEMM of the sorted slots with TQ2_T dequant fused into
// the fp16 MFMA B operand, SwiGLU and the down-input rotation in the epilogue.
//   g = W_g[e] . xh, u = W_u[e] . xh        src/engine.zig:567-602
//   a = H_128 (down_signs * silu(g) * u)    src/engine.zig:603-607
//
// A group takes one tile of the sort (expert e, up to 128 sorted rows) and one 128-column block
// of F. Eight waves: wave w owns F columns 32 (w % 4) .. + 31 of the block for the gate (w < 4)
// or the up projection (w >= 4), so no weight is decoded twice, and the gate and up waves of one
// column range share a SIMD: while one issues MFMAs the other decodes. Each decoded fragment
// feeds all of the tile's 32-row blocks (v_mfma_f32_32x32x16_f16, fp32 accumulation). K runs
// over the E / 128 Gyro blocks: the tile's activation rows (binary16 rows of the rotated input,
// gathered through route_order) and the 256 weight rows' blocks arrive in LDS by direct loads
// issued two blocks ahead (ggemm.h); each lane decodes the block of its own row into B operands.
// The fp16 products scale x codebook stay finite: the host checks every layer's scales.
// Epilogue: the up waves pass u through LDS (fp32); the gate waves form silu(g) * u times the
// down signs, rounded to binary16 into LDS rows; the 128-point Walsh-Hadamard transform of every
// row runs as one more fp16 MFMA product with H_128 (exact +-1 entries, fp32 accumulation, then
// x 1/sqrt(128)), split over the eight waves; binary16 rows go to act16[sorted row][F].
// Grid: (F / 128, max tiles); 512 threads, one group per CU (141 KB of LDS); groups start tile
// by tile in the sort's longest-first order, all column blocks of a tile together; the groups
// beyond the sort's tile count exit.
// Requires TQ2_T experts, E % 256 == 0 (rows start at 4-byte boundaries, an even block count),
// F % 128 == 0, |xh|, |act| < 65504.
// Constants: 0 meta_uav 1 order_uav 2 order_off 3 xh16_uav 4 xh16_off (words) 5 base_lo
// 6 base_hi 7 slot_stride 8 proj_bytes 9 codebook_srv 10 signs_srv (0xffffffff: none)
// 11 signs_off 12 act16_uav 13 act16_off (words) 14 E 15 F 16 n_used.
#include "ggemm.h"

struct GuState {
    const void *xbase, *wbase;  // activation rows; the layer's slot arena (expert bundles)
    uint32_t roff[4], woff[2];
    uint32_t nal;  // activation loads per block of this wave (0 or 4)
    uint32_t wave, m, h, sel, nk, wq;  // wq: the staged weight row this lane decodes
};

// Start of K block kb: this wave's loads of block kb have landed once at most the loads of
// block kb + 1 are outstanding (4 activation loads, plus 2 or 1 weight loads by wave class).
__device__ __forceinline__ void gu_sync(const GuState &t, uint32_t kb) {
    gg_sync_block(t.nal + (t.wave < 4u ? 2u : 1u), kb + 1u >= t.nk);
}

// K block kb from buffer BUF for NRB 32-row blocks; stages block kb + 2 into buffer
// (BUF + 2) % 3, the buffer of block kb - 1, which every wave has left once past the sync.
template <int BUF, int NRB>
__device__ __forceinline__ void gu_step(GgLds &sm, const GuState &t, uint32_t kb, f32x16 (&acc)[NRB]) {
    gu_sync(t, kb);
    if (kb + 2u < t.nk) {
        if (t.nal) gg_stage_a8(sm, (BUF + 2) % 3, t.wave, t.xbase, t.roff, kb + 2u);
        gg_stage_w8(sm, (BUF + 2) % 3, t.wave, t.wbase, t.woff, kb + 2u);
    }
    GgBlk wc;
    gg_read_w(sm, BUF, t.wq, wc);
    float sc;
    uint32_t q[8];
    tq2_unpack(wc.d, kb & 1u, sc, q);
    const half2_t sc2 = {(_Float16)sc, (_Float16)sc};
    // Software pipeline over the 8 K-steps with an explicit schedule (sched_barrier fences keep
    // the compiler from regrouping it): between the MFMAs of step s go the codebook gathers of
    // step s + 2 (one trellis state per piece, over the first two slots; two steps ahead, so a
    // one-block tile still hides their latency) and the A operands of step s + 1 (one per
    // slot). Gathers of even and odd steps use separate registers.
    uint32_t raw[2][4], pr[2] = {0u, 0u};
    gg_gather(q, 0, t.sel, sm.book, raw[0]);
    gg_gather(q, 1, t.sel, sm.book, raw[1]);
    f16x8 av[NRB];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) av[rb] = gg_a(sm, BUF, rb * 32u + t.m, 0, t.h);
    constexpr int kPieceSlots = NRB < 2 ? NRB : 2;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const f16x8 bv = gg_scale(raw[s & 1], sc2);
        f16x8 cur[NRB];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) cur[rb] = av[rb];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NRB; ++i) {
            acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur[i], bv, acc[i], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (s < 6) {
#pragma unroll
                for (int piece = 0; piece < 2; ++piece)
                    if (i < kPieceSlots && piece * kPieceSlots / 2 == i)
                        gg_gather_piece(q, s + 2, piece, t.sel, sm.book, pr[s & 1], raw[s & 1]);
            }
            if (s < 7) {
                av[i] = gg_a(sm, BUF, i * 32u + t.m, s + 1, t.h);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// The K loop and the epilogue of a tile with NRB 32-row blocks.
template <int NRB>
__device__ __forceinline__ void gu_tile(GgLds &sm, const GuState &t, const GdArgs &a, uint32_t row0, uint32_t rows,
                                        uint32_t fb, uint32_t F) {
    f32x16 acc[NRB];
#pragma unroll
    for (int r = 0; r < NRB; ++r) acc[r] = (f32x16){};
    // Blocks rotate through the three buffers: block kb in buffer kb % 3.
    for (uint32_t kb = 0; kb < t.nk; kb += 3u) {
        gu_step<0, NRB>(sm, t, kb, acc);
        if (kb + 1u < t.nk) gu_step<1, NRB>(sm, t, kb + 1u, acc);
        if (kb + 2u < t.nk) gu_step<2, NRB>(sm, t, kb + 2u, acc);
    }
    gg_sync<0>();  // every wave is done with the buffers
    const float *signs = a.c[10] != 0xffffffffu ? gd_buf<const float>(a, a.c[10]) + a.c[11] : nullptr;
    gg_gu_epilogue(sm, acc, t.wave, t.m, t.h, signs, gd_buf<uint32_t>(a, a.c[12]) + a.c[13], row0, rows, fb, F);
}

GD_PIPELINE_NAMED_OCC(moe_prefill_gu, 512, 2) {
    __shared__ GgLds sm;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
    const uint32_t *meta = gd_buf<const uint32_t>(a, a.c[0]);
    const uint32_t tile = blockIdx.y;
    if (tile >= __builtin_amdgcn_readfirstlane(meta[1023])) return;
    const uint4 td = reinterpret_cast<const uint4 *>(meta + 1024u)[tile];
    // Uniform per group: scalar branches over the row blocks.
    const uint32_t e = __builtin_amdgcn_readfirstlane(td.x), row0 = __builtin_amdgcn_readfirstlane(td.y),
                   rows = __builtin_amdgcn_readfirstlane(td.z);
    const uint32_t E = a.c[14], F = a.c[15], U = a.c[16], fb = blockIdx.x;

    const uint4 *cb = gd_buf<const uint4>(a, a.c[9]);
    reinterpret_cast<uint4 *>(sm.book)[tid] = cb[tid];
    if (tid < GG_TM) sm.src[tid] = gd_buf<const uint32_t>(a, a.c[1])[a.c[2] + row0 + min(tid, rows - 1u)] / U;
    __syncthreads();

    GuState t;
    t.wave = wave;
    t.m = lane & 31u;
    t.h = lane >> 5;
    t.sel = gg_sel(t.h);
    t.nk = E / 128u;
    t.wq = (wave >> 2) * 128u + (wave & 3u) * 32u + t.m;
    t.xbase = gd_buf<const uint32_t>(a, a.c[3]) + a.c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t r;
        const uint32_t c = gg_chunk8(wave, lane, i, r);
        t.roff[i] = sm.src[r] * (E * 2u) + c;
    }
    // Staged weight row q < 128: gate row fb * 128 + q; q >= 128: up row fb * 128 + q - 128.
    // Load L carries pieces 64 L + lane: row g / 3, 16-byte piece g % 3.
    const uint64_t base = ((uint64_t)a.c[6] << 32) | a.c[5];
    t.wbase = reinterpret_cast<const void *>(base);
    const uint32_t row_bytes = (E / 128u) * 34u, proj_bytes = a.c[8];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t g = gg_w8_load(wave, i) * 64u + lane, q = g / 3u, piece = g - q * 3u;
        t.woff[i] = e * a.c[7] + (q >> 7) * proj_bytes + (fb * 128u + (q & 127u)) * row_bytes + piece * 16u;
    }
    t.nal = gg_a_loads(wave, (rows + 31u) >> 5);
    if (t.nal) gg_stage_a8(sm, 0, wave, t.xbase, t.roff, 0);
    gg_stage_w8(sm, 0, wave, t.wbase, t.woff, 0);
    if (t.nk > 1u) {
        if (t.nal) gg_stage_a8(sm, 1, wave, t.xbase, t.roff, 1);
        gg_stage_w8(sm, 1, wave, t.wbase, t.woff, 1);
    }
    switch ((rows + 31u) >> 5) {
        case 1: gu_tile<1>(sm, t, a, row0, rows, fb, F); break;
        case 2: gu_tile<2>(sm, t, a, row0, rows, fb, F); break;
        case 3: gu_tile<3>(sm, t, a, row0, rows, fb, F); break;
        default: gu_tile<4>(sm, t, a, row0, rows, fb, F); break;
    }
}
