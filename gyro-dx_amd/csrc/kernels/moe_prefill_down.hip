// Prefill path, step 5: grouped down GEMM of the sorted slots with TQ2_T dequant fused into the
// fp16 MFMA B operand.
//   down[slot][r] = W_d[e][r] . a[slot]     src/engine.zig:608-633
//
// A group takes one tile of the sort (expert e, up to 128 sorted rows) and one 256-row block
// of the expert's down matrix (256 output columns); eight waves, wave w owns output columns
// 32 w .. + 31, two waves per SIMD. K runs over the F / 128 Gyro blocks of a down row; the
// tile's act16 rows (already contiguous in sorted order) and the 256 weight rows' blocks arrive
// in LDS by direct loads two blocks ahead, and each lane decodes its own down row into B
// operands, with the software pipeline of the gate/up kernel (ggemm.h). The results pass
// through LDS (fp32 [row][256 columns], 128 KB over the K-loop buffers) so that every sorted row
// leaves as 1 KB of 16-byte stores to its slot's row, down32[route_order[row]][E], in fp32 for
// the k-ordered combine.
// Grid: (E / 256, max tiles); 512 threads, one group per CU, started tile by tile in the sort's
// longest-first order; the groups beyond the sort's tile count exit. Requires TQ2_T experts,
// F % 256 == 0, E % 256 == 0.
// Constants: 0 meta_uav 1 order_uav 2 order_off 3 act16_uav 4 act16_off (words) 5 base_lo
// 6 base_hi 7 slot_stride 8 down_offset (bytes from the bundle start) 9 codebook_srv
// 10 down32_uav 11 down32_off (words) 12 E 13 F.
#include "ggemm.h"

struct DnState {
    const void *abase, *wbase;  // act16 rows; the layer's slot arena
    uint32_t roff[4], woff[2];
    uint32_t nal;  // activation loads per block of this wave (0 or 4)
    uint32_t wave, m, h, sel, nk;
};

// Start of K block kb (as the gate/up kernel: 4 activation loads, plus 2 or 1 weight loads by
// wave class, belong to the following block).
__device__ __forceinline__ void dn_sync(const DnState &t, uint32_t kb) {
    gg_sync_block(t.nal + (t.wave < 4u ? 2u : 1u), kb + 1u >= t.nk);
}

// K block kb from buffer BUF for NRB 32-row blocks (see gu_step of the gate/up kernel).
template <int BUF, int NRB>
__device__ __forceinline__ void dn_step(GgLds &sm, const DnState &t, uint32_t kb, f32x16 (&acc)[NRB]) {
    dn_sync(t, kb);
    if (kb + 2u < t.nk) {
        if (t.nal) gg_stage_a8(sm, (BUF + 2) % 3, t.wave, t.abase, t.roff, kb + 2u);
        gg_stage_w8(sm, (BUF + 2) % 3, t.wave, t.wbase, t.woff, kb + 2u);
    }
    GgBlk cur;
    gg_read_w(sm, BUF, t.wave * 32u + t.m, cur);
    float sc;
    uint32_t q[8];
    tq2_unpack(cur.d, kb & 1u, sc, q);
    const half2_t sc2 = {(_Float16)sc, (_Float16)sc};
    uint32_t raw[2][4], pr[2] = {0u, 0u};  // gathers of even and odd steps, two steps ahead
    gg_gather(q, 0, t.sel, sm.book, raw[0]);
    gg_gather(q, 1, t.sel, sm.book, raw[1]);
    f16x8 av[NRB];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) av[rb] = gg_a(sm, BUF, rb * 32u + t.m, 0, t.h);
    constexpr int kPieceSlots = NRB < 2 ? NRB : 2;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const f16x8 bv = gg_scale(raw[s & 1], sc2);
        f16x8 cur_a[NRB];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) cur_a[rb] = av[rb];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NRB; ++i) {
            acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur_a[i], bv, acc[i], 0, 0, 0);
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

template <int NRB>
__device__ __forceinline__ void dn_tile(GgLds &sm, const DnState &t, const GdArgs &a, uint32_t rows, uint32_t eb,
                                        uint32_t E) {
    f32x16 acc[NRB];
#pragma unroll
    for (int r = 0; r < NRB; ++r) acc[r] = (f32x16){};
    for (uint32_t kb = 0; kb < t.nk; kb += 3u) {
        dn_step<0, NRB>(sm, t, kb, acc);
        if (kb + 1u < t.nk) dn_step<1, NRB>(sm, t, kb + 1u, acc);
        if (kb + 2u < t.nk) dn_step<2, NRB>(sm, t, kb + 2u, acc);
    }
    gg_sync<0>();  // every wave is done with the buffers
    gg_down_epilogue(sm, acc, t.wave, t.m, t.h, gd_buf<float>(a, a.c[10]) + a.c[11], rows, eb, E);
}

GD_PIPELINE_NAMED_OCC(moe_prefill_down, 512, 2) {
    __shared__ GgLds sm;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
    const uint32_t *meta = gd_buf<const uint32_t>(a, a.c[0]);
    const uint32_t tile = blockIdx.y;
    if (tile >= __builtin_amdgcn_readfirstlane(meta[1023])) return;
    const uint4 td = reinterpret_cast<const uint4 *>(meta + 1024u)[tile];
    const uint32_t e = __builtin_amdgcn_readfirstlane(td.x), row0 = __builtin_amdgcn_readfirstlane(td.y),
                   rows = __builtin_amdgcn_readfirstlane(td.z);
    const uint32_t E = a.c[12], F = a.c[13], eb = blockIdx.x;

    const uint4 *cb = gd_buf<const uint4>(a, a.c[9]);
    reinterpret_cast<uint4 *>(sm.book)[tid] = cb[tid];
    if (tid < GG_TM) sm.src[tid] = gd_buf<const uint32_t>(a, a.c[1])[a.c[2] + row0 + min(tid, rows - 1u)];

    DnState t;
    t.wave = wave;
    t.m = lane & 31u;
    t.h = lane >> 5;
    t.sel = gg_sel(t.h);
    t.nk = F / 128u;
    t.abase = gd_buf<const uint32_t>(a, a.c[3]) + a.c[4];
    // Source row of each staged activation chunk: sorted row row0 + r; padding rows repeat the
    // last row.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t r;
        const uint32_t c = gg_chunk8(wave, lane, i, r);
        t.roff[i] = (row0 + min(r, rows - 1u)) * (F * 2u) + c;
    }
    // Staged weight row q: down row eb * 256 + q. Load L carries pieces 64 L + lane: row g / 3,
    // 16-byte piece g % 3.
    t.wbase = reinterpret_cast<const void *>(((uint64_t)a.c[6] << 32) | a.c[5]);
    const uint32_t row_bytes = (F / 128u) * 34u;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t g = gg_w8_load(wave, i) * 64u + lane, q = g / 3u, piece = g - q * 3u;
        t.woff[i] = e * a.c[7] + a.c[8] + (eb * 256u + q) * row_bytes + piece * 16u;
    }
    __syncthreads();  // codebook and slot numbers
    t.nal = gg_a_loads(wave, (rows + 31u) >> 5);
    if (t.nal) gg_stage_a8(sm, 0, wave, t.abase, t.roff, 0);
    gg_stage_w8(sm, 0, wave, t.wbase, t.woff, 0);
    if (t.nk > 1u) {
        if (t.nal) gg_stage_a8(sm, 1, wave, t.abase, t.roff, 1);
        gg_stage_w8(sm, 1, wave, t.wbase, t.woff, 1);
    }
    switch ((rows + 31u) >> 5) {
        case 1: dn_tile<1>(sm, t, a, rows, eb, E); break;
        case 2: dn_tile<2>(sm, t, a, rows, eb, E); break;
        case 3: dn_tile<3>(sm, t, a, rows, eb, E); break;
        default: dn_tile<4>(sm, t, a, rows, eb, E); break;
    }
}
