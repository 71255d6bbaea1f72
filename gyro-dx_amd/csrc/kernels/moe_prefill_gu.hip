// Prefill path, step 4: grouped gate/up GEMM of the sorted slots with TQ2_T dequant fused into
// the fp16 MFMA B operand, SwiGLU and the down-input rotation in the epilogue.
//   g = W_g[e] . xh, u = W_u[e] . xh        src/engine.zig:567-602
//   a = H_128 (down_signs * silu(g) * u)    src/engine.zig:603-607
//
// A group takes one tile of the sort (expert e, up to 128 sorted rows) and one 128-column block
// of F. Wave w owns F columns 32 w .. 32 w + 31 of the block for both gate and up, so no
// weight is decoded twice; each decoded fragment feeds all of the tile's 32-row blocks
// (v_mfma_f32_32x32x16_f16, fp32 accumulation). K runs over the E / 128 Gyro blocks: the
// tile's activation rows (binary16 rows of the rotated input, gathered through route_order)
// arrive in LDS by direct loads issued one block ahead (ggemm.h), and each lane decodes the
// block of its own weight row (loaded one block ahead into registers) into B operands.
// The fp16 products scale x codebook stay finite: the host checks every layer's scales.
// Epilogue: silu(g) * u times the down signs, through LDS into rows, one 128-point
// Walsh-Hadamard transform per row and wave, and binary16 rows act16[sorted row][F].
// Grid: (max tiles, F / 128); 256 threads, two groups per CU; the groups beyond the sort's tile
// count exit.
// Requires TQ2_T experts, E % 256 == 0 (rows start at 4-byte boundaries, an even block count),
// F % 128 == 0, |xh|, |act| < 65504.
// Constants: 0 meta_uav 1 order_uav 2 order_off 3 xh16_uav 4 xh16_off (words) 5 base_lo
// 6 base_hi 7 slot_stride 8 proj_bytes 9 codebook_srv 10 signs_srv (0xffffffff: none)
// 11 signs_off 12 act16_uav 13 act16_off (words) 14 E 15 F 16 n_used.
#include "fwht.h"
#include "ggemm.h"

#define GU_ACT_STRIDE 132  // floats per epilogue row

struct GuState {
    gd_guint *grow, *urow;  // this lane's gate and up rows
    const void *xbase;      // activation rows (byte offsets in roff)
    uint32_t roff[8];
    uint32_t wave, m, h, sel, nrb, nk;
};

// Block kb from buffer BUF with weights (gc, uc) for NRB 32-row blocks; prefetches block kb + 1
// into the other buffer and (gn, un). The current block is unpacked before the prefetch is
// issued (and the scheduler may not move it past), so waiting for it never waits for the
// prefetch: loads retire in order.
template <int BUF, int NRB>
__device__ __forceinline__ void gu_step(GgLds &sm, const GuState &t, uint32_t kb, const GgBlk &gc, const GgBlk &uc,
                                        GgBlk &gn, GgBlk &un, f32x16 (&accg)[NRB], f32x16 (&accu)[NRB]) {
    const bool odd = kb & 1u;
    float gs, us;
    uint32_t gq[8], uq[8];
    tq2_unpack(gc.d, odd, gs, gq);
    tq2_unpack(uc.d, odd, us, uq);
    const half2_t gs2 = {(_Float16)gs, (_Float16)gs}, us2 = {(_Float16)us, (_Float16)us};
    gg_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if (kb + 1u < t.nk) {
        gg_stage(sm, BUF ^ 1, t.wave, t.xbase, t.roff, kb + 1u);
        gg_load_blk(t.grow, kb + 1u, gn);
        gg_load_blk(t.urow, kb + 1u, un);
    }
    // Software pipeline over the 8 K-steps with an explicit schedule (sched_barrier fences keep
    // the compiler from regrouping it). Everything step s + 1 reads from LDS is issued during
    // step s, between its MFMAs: first the codebook gathers of its decode (one trellis state per
    // piece), then its A operands. LDS reads retire in order, so step s + 1 finds them complete
    // and never waits inside its MFMA sequence.
    uint32_t rg[4], ru[4], pg = 0, pu = 0;
    gg_gather(gq, 0, t.sel, sm.book, rg);
    gg_gather(uq, 0, t.sel, sm.book, ru);
    f16x8 av[NRB];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) av[rb] = gg_a(sm, BUF, rb * 32u + t.m, 0, t.h);
    constexpr int kSlots = 2 * NRB;
    constexpr int kPieceSlots = kSlots < 4 ? kSlots : 4;  // slots that carry gathers
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const f16x8 bg = gg_scale(rg, gs2), bu = gg_scale(ru, us2);
        f16x8 cur[NRB];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) cur[rb] = av[rb];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < kSlots; ++i) {
            const int rb = i >> 1;
            if ((i & 1) == 0) accg[rb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur[rb], bg, accg[rb], 0, 0, 0);
            else accu[rb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur[rb], bu, accu[rb], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (s < 7) {
                // Gathers: pieces 0..3 = (gate state a, gate state b, up a, up b) over the first
                // kPieceSlots slots.
#pragma unroll
                for (int piece = 0; piece < 4; ++piece) {
                    if (i < kPieceSlots && piece * kPieceSlots / 4 == i) {
                        if (piece < 2) gg_gather_piece(gq, s + 1, piece, t.sel, sm.book, pg, rg);
                        else gg_gather_piece(uq, s + 1, piece - 2, t.sel, sm.book, pu, ru);
                    }
                }
                // A operands of step s + 1 over the remaining slots (all in the last slot when
                // every slot carries gathers).
#pragma unroll
                for (int r = 0; r < NRB; ++r) {
                    const int slot = kSlots - NRB + r;
                    if (slot == i || (slot < kPieceSlots && i == kSlots - 1))
                        av[r] = gg_a(sm, BUF, r * 32u + t.m, s + 1, t.h);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// The K loop and the epilogue of a tile with NRB 32-row blocks.
template <int NRB>
__device__ __forceinline__ void gu_tile(GgLds &sm, const GuState &t, const GdArgs &a, uint32_t row0, uint32_t rows,
                                        uint32_t fb, uint32_t F) {
    const uint32_t lane = threadIdx.x & 63u;
    f32x16 accg[NRB], accu[NRB];
#pragma unroll
    for (int r = 0; r < NRB; ++r) {
        accg[r] = (f32x16){};
        accu[r] = (f32x16){};
    }
    GgBlk g0, u0, g1, u1;
    gg_load_blk(t.grow, 0, g0);
    gg_load_blk(t.urow, 0, u0);
    gg_stage(sm, 0, t.wave, t.xbase, t.roff, 0);
    // nk is even: blocks alternate between buffer 0 with (g0, u0) and buffer 1 with (g1, u1).
    for (uint32_t kb = 0; kb < t.nk; kb += 2u) {
        gu_step<0, NRB>(sm, t, kb, g0, u0, g1, u1, accg, accu);
        gu_step<1, NRB>(sm, t, kb + 1u, g1, u1, g0, u0, accg, accu);
    }
    gg_barrier();  // every wave is done with the activation buffers

    // Epilogue: act = down_signs * silu(g) * u into LDS rows (132-float stride, from offset 0).
    float *act = reinterpret_cast<float *>(&sm);
    const bool has_signs = a.c[10] != 0xffffffffu;
    const uint32_t col = t.wave * 32u + t.m;
    const float sgn = has_signs ? gd_buf<const float>(a, a.c[10])[a.c[11] + fb * 128u + col] : 1.0f;
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t i = rb * 32u + (r / 4) * 8u + t.h * 4u + (r % 4);
            act[i * GU_ACT_STRIDE + col] = gd_silu(accg[rb][r]) * accu[rb][r] * sgn;
        }
    }
    __syncthreads();
    uint32_t *out = gd_buf<uint32_t>(a, a.c[12]) + a.c[13];
    for (uint32_t i = t.wave; i < rows; i += 4u) {
        const float2 v = *reinterpret_cast<const float2 *>(act + i * GU_ACT_STRIDE + 2u * lane);
        float x0 = v.x, x1 = v.y;
        if (has_signs) {
            gd_fwht128_wave(x0, x1);
            x0 *= GD_INV_SQRT128;
            x1 *= GD_INV_SQRT128;
        }
        const uint32_t h0 = __builtin_bit_cast(uint16_t, (_Float16)x0);
        const uint32_t h1 = __builtin_bit_cast(uint16_t, (_Float16)x1);
        out[(size_t)(row0 + i) * (F / 2u) + fb * 64u + lane] = h0 | (h1 << 16);
    }
}

GD_PIPELINE_NAMED_OCC(moe_prefill_gu, 256, 2) {
    __shared__ GgLds sm;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t *meta = gd_buf<const uint32_t>(a, a.c[0]);
    const uint32_t tile = blockIdx.x;
    if (tile >= __builtin_amdgcn_readfirstlane(meta[1023])) return;
    const uint4 td = reinterpret_cast<const uint4 *>(meta + 1024u)[tile];
    // Uniform per group: scalar branches over the row blocks.
    const uint32_t e = __builtin_amdgcn_readfirstlane(td.x), row0 = __builtin_amdgcn_readfirstlane(td.y),
                   rows = __builtin_amdgcn_readfirstlane(td.z);
    const uint32_t E = a.c[14], F = a.c[15], U = a.c[16], fb = blockIdx.y;

    const uint4 *cb = gd_buf<const uint4>(a, a.c[9]);
    reinterpret_cast<uint4 *>(sm.book)[tid] = cb[tid];
    reinterpret_cast<uint4 *>(sm.book)[tid + 256u] = cb[tid + 256u];
    if (tid < GG_TM) sm.src[tid] = gd_buf<const uint32_t>(a, a.c[1])[a.c[2] + row0 + min(tid, rows - 1u)] / U;
    __syncthreads();

    GuState t;
    t.wave = wave;
    t.m = lane & 31u;
    t.h = lane >> 5;
    t.sel = gg_sel(t.h);
    t.nrb = (rows + 31u) >> 5;
    t.nk = E / 128u;
    t.xbase = gd_buf<const uint32_t>(a, a.c[3]) + a.c[4];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint32_t r;
        const uint32_t c = gg_chunk(wave, lane, i, r);
        t.roff[i] = sm.src[r] * (E * 2u) + c;
    }
    const uint64_t base = ((uint64_t)a.c[6] << 32) | a.c[5];
    const uint8_t *grow = reinterpret_cast<const uint8_t *>(base + (uint64_t)e * a.c[7]) +
                          (size_t)(fb * 128u + wave * 32u + t.m) * ((E / 128u) * 34u);
    t.grow = gd_global(reinterpret_cast<const uint32_t *>(grow));
    t.urow = gd_global(reinterpret_cast<const uint32_t *>(grow + a.c[8]));

    switch (t.nrb) {
        case 1: gu_tile<1>(sm, t, a, row0, rows, fb, F); break;
        case 2: gu_tile<2>(sm, t, a, row0, rows, fb, F); break;
        case 3: gu_tile<3>(sm, t, a, row0, rows, fb, F); break;
        default: gu_tile<4>(sm, t, a, row0, rows, fb, F); break;
    }
}
