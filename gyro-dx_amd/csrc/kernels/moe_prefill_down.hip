// Prefill path, step 5: grouped down GEMM of the sorted slots with TQ2_T dequant fused into the
// fp16 MFMA B operand.
//   down[slot][r] = W_d[e][r] . a[slot]     src/engine.zig:608-633
//
// A group takes one tile of the sort (expert e, up to 128 sorted rows) and one 128-row block
// of the expert's down matrix (128 output columns); wave w owns output columns 32 w .. +31.
// K runs over the F / 128 Gyro blocks of a down row; the tile's act16 rows (already contiguous
// in sorted order) and the 128 weight rows' blocks arrive in LDS by direct loads two blocks
// ahead, and each lane decodes its own down row into B operands, with the software pipeline of
// the gate/up kernel (ggemm.h). Results go to the slot's own row, down32[route_order[row]][E],
// in fp32 for the k-ordered combine.
// Grid: (max tiles, E / 128); 256 threads, one group per CU; the groups beyond the sort's tile
// count exit. Requires TQ2_T experts, F % 256 == 0.
// Constants: 0 meta_uav 1 order_uav 2 order_off 3 act16_uav 4 act16_off (words) 5 base_lo
// 6 base_hi 7 slot_stride 8 down_offset (bytes from the bundle start) 9 codebook_srv
// 10 down32_uav 11 down32_off (words) 12 E 13 F.
#include "ggemm.h"

#define DN_LOADS 10  // global-to-LDS loads per wave and K block: 8 activation + 2 weight

struct DnState {
    const void *abase, *wbase;  // act16 rows; the layer's slot arena
    uint32_t roff[8], woff[2];
    uint32_t wave, m, h, sel, nk;
};

// K block kb from buffer BUF for NRB 32-row blocks (see gu_step of the gate/up kernel).
template <int BUF, int NRB>
__device__ __forceinline__ void dn_step(GgLds &sm, const DnState &t, uint32_t kb, f32x16 (&acc)[NRB]) {
    if (kb + 1u < t.nk) gg_sync<DN_LOADS>();
    else gg_sync<0>();
    if (kb + 2u < t.nk) {
        gg_stage_a(sm, (BUF + 2) % 3, t.wave, t.abase, t.roff, kb + 2u);
        gg_stage_w<2>(sm, (BUF + 2) % 3, t.wave, t.wbase, t.woff, kb + 2u);
    }
    GgBlk cur;
    gg_read_w(sm, BUF, t.wave * 32u + t.m, cur);
    float sc;
    uint32_t q[8];
    tq2_unpack(cur.d, kb & 1u, sc, q);
    const half2_t sc2 = {(_Float16)sc, (_Float16)sc};
    // Software pipeline as in gu_step, with one projection: the gathers of step s + 1 follow the
    // first MFMAs of step s, its A operands the last ones.
    uint32_t raw[4], pr = 0;
    gg_gather(q, 0, t.sel, sm.book, raw);
    f16x8 av[NRB];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) av[rb] = gg_a(sm, BUF, rb * 32u + t.m, 0, t.h);
    constexpr int kPieceSlots = NRB < 2 ? NRB : 2;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const f16x8 bv = gg_scale(raw, sc2);
        f16x8 cur_a[NRB];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) cur_a[rb] = av[rb];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NRB; ++i) {
            acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur_a[i], bv, acc[i], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (s < 7) {
#pragma unroll
                for (int piece = 0; piece < 2; ++piece)
                    if (i < kPieceSlots && piece * kPieceSlots / 2 == i)
                        gg_gather_piece(q, s + 1, piece, t.sel, sm.book, pr, raw);
                if (i == NRB - 1) {  // A operands after the gathers
#pragma unroll
                    for (int r = 0; r < NRB; ++r) av[r] = gg_a(sm, BUF, r * 32u + t.m, s + 1, t.h);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

template <int NRB>
__device__ __forceinline__ void dn_tile(GgLds &sm, const DnState &t, const GdArgs &a, uint32_t row0, uint32_t rows,
                                        uint32_t eb, uint32_t E) {
    (void)row0;
    f32x16 acc[NRB];
#pragma unroll
    for (int r = 0; r < NRB; ++r) acc[r] = (f32x16){};
    for (uint32_t kb = 0; kb < t.nk; kb += 3u) {
        dn_step<0, NRB>(sm, t, kb, acc);
        if (kb + 1u < t.nk) dn_step<1, NRB>(sm, t, kb + 1u, acc);
        if (kb + 2u < t.nk) dn_step<2, NRB>(sm, t, kb + 2u, acc);
    }
    // Rows go back to their slots (staged in sm.src): down32[slot][eb * 128 + 32 wave + m].
    float *out = gd_buf<float>(a, a.c[10]) + a.c[11];
    const uint32_t col = eb * 128u + t.wave * 32u + t.m;
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t i = rb * 32u + (r / 4) * 8u + t.h * 4u + (r % 4);
            if (i < rows) out[(size_t)sm.src[i] * E + col] = acc[rb][r];
        }
    }
}

GD_PIPELINE_NAMED_OCC(moe_prefill_down, 256, 1) {
    __shared__ GgLds sm;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
    const uint32_t *meta = gd_buf<const uint32_t>(a, a.c[0]);
    const uint32_t tile = blockIdx.x;
    if (tile >= __builtin_amdgcn_readfirstlane(meta[1023])) return;
    const uint4 td = reinterpret_cast<const uint4 *>(meta + 1024u)[tile];
    const uint32_t e = __builtin_amdgcn_readfirstlane(td.x), row0 = __builtin_amdgcn_readfirstlane(td.y),
                   rows = __builtin_amdgcn_readfirstlane(td.z);
    const uint32_t E = a.c[12], F = a.c[13], eb = blockIdx.y;

    const uint4 *cb = gd_buf<const uint4>(a, a.c[9]);
    reinterpret_cast<uint4 *>(sm.book)[tid] = cb[tid];
    reinterpret_cast<uint4 *>(sm.book)[tid + 256u] = cb[tid + 256u];
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
    for (int i = 0; i < 8; ++i) {
        uint32_t r;
        const uint32_t c = gg_chunk(wave, lane, i, r);
        t.roff[i] = (row0 + min(r, rows - 1u)) * (F * 2u) + c;
    }
    // Weight rows: down row eb * 128 + q (q < 128; the loads' surplus pieces repeat row 127 into
    // unused buffer rows).
    t.wbase = reinterpret_cast<const void *>(((uint64_t)a.c[6] << 32) | a.c[5]);
    const uint32_t row_bytes = (F / 128u) * 34u;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        uint32_t q, piece;
        gg_w_piece<2>(wave, lane, i, q, piece);
        t.woff[i] = e * a.c[7] + a.c[8] + (eb * 128u + min(q, 127u)) * row_bytes + piece * 16u;
    }
    __syncthreads();  // codebook and slot numbers
    gg_stage_a(sm, 0, wave, t.abase, t.roff, 0);
    gg_stage_w<2>(sm, 0, wave, t.wbase, t.woff, 0);
    if (t.nk > 1u) {
        gg_stage_a(sm, 1, wave, t.abase, t.roff, 1);
        gg_stage_w<2>(sm, 1, wave, t.wbase, t.woff, 1);
    }
    switch ((rows + 31u) >> 5) {
        case 1: dn_tile<1>(sm, t, a, row0, rows, eb, E); break;
        case 2: dn_tile<2>(sm, t, a, row0, rows, eb, E); break;
        case 3: dn_tile<3>(sm, t, a, row0, rows, eb, E); break;
        default: dn_tile<4>(sm, t, a, row0, rows, eb, E); break;
    }
}
