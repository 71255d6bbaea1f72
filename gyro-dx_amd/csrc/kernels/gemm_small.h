// Units of the TQ2_T grouped GEMMs for sort tiles of at most SR rows (the prefill path's small
// expert segments: under a skewed router most hit experts receive 1 to 4 token slots, and a
// unit decodes its 256 weight rows whatever the tile's row count).
//
// The tile's activation rows, all of K, are staged into LDS once (SR rows x K binary16, XOR-
// swizzled 16-byte chunks: chunk c of row r at position c ^ r, so the A-operand reads of the
// tile's rows at one chunk index hit different bank groups), then the K loop runs without a
// barrier: each lane streams its weight row's blocks from HBM into registers, two blocks
// ahead in a ring of three, and decodes them into the B operand as the other units do
// (gg_gather_piece, gg_scale). The MFMA sequence per accumulator (K-steps in order) and the
// epilogues are those of gemm_units.h, so the results are bit-identical to theirs. MFMA rows
// at or past SR read row (m mod SR) and are never stored.
// LDS: the GhLds of the other units; the codebook at byte 0, the activation rows from byte 8192
// (SR K 2 bytes: 64 KB at K = 2048, SR = 16), addressed from the start of the struct.
#pragma once
#include "gemm_units.h"

static_assert(sizeof(GhLds) >= 8192u + 16u * 2048u * 2u, "small-unit activation rows fit the units' LDS");

// Rows a small unit takes for hidden width E (gate/up K) when E % 512 == 0; 0: none.
__host__ __device__ constexpr uint32_t gs_rows_for(uint32_t E) { return E % 512u ? 0u : (E <= 2048u ? 16u : (E <= 4096u ? 8u : 0u)); }

// Stages rows 0 .. rows - 1 of the tile (row r: rowp(r) words into `src`, K binary16 values)
// into LDS at byte 8192, 16-byte chunk positions r K / 8 + q holding chunk q ^ r. A wave's
// direct load writes 64 consecutive positions (one quarter, half, ... of a row).
template <class ROWF>
__device__ __forceinline__ void gs_stage_rows(GhLds &sm, uint32_t wave, uint32_t lane, const void *src, uint32_t K,
                                              uint32_t rows, ROWF rowp) {
    const uint32_t cpr = K / 8u, per_row = cpr / 64u, loads = rows * per_row;
    const uint32_t base = gg_lds_addr(&sm) + 8192u;
    for (uint32_t j = wave; j < loads; j += 8u) {  // uniform per wave
        const uint32_t r = j / per_row, q = (j - r * per_row) * 64u + lane;
        gg_dma16(base + (r * cpr + (q - lane)) * 16u, src, rowp(r) * 4u + ((q ^ r) * 16u));
    }
}

// A operand of K-step s for MFMA row m (chunk 2 s + h of row m mod SR).
template <uint32_t SR>
__device__ __forceinline__ f16x8 gs_a(const GhLds &sm, uint32_t cpr, uint32_t m, uint32_t s, uint32_t h) {
    const uint32_t r = m & (SR - 1u), c = 2u * s + h;
    const gd_u32x4 *a = reinterpret_cast<const gd_u32x4 *>(reinterpret_cast<const uint8_t *>(&sm) + 8192u);
    return __builtin_bit_cast(f16x8, a[r * cpr + (c ^ r)]);
}

// The 9 words from the 4-byte-aligned start of a 34-byte block.
__device__ __forceinline__ void gs_load_blk(gd_guint *p, uint32_t (&d)[9]) {
#pragma unroll
    for (int j = 0; j < 9; ++j) d[j] = p[j];
}

// One K block (8 K-steps) from the weight words d (block parity odd: its start is 2 bytes past
// the loaded words' first byte).
template <uint32_t SR>
__device__ __forceinline__ void gs_block(const GhLds &sm, const uint32_t (&d)[9], bool odd, uint32_t cpr, uint32_t kb,
                                         uint32_t m, uint32_t h, uint32_t sel, f32x16 &acc) {
    float sc;
    uint32_t q[8];
    tq2_unpack(d, odd, sc, q);
    const half2_t sc2 = {(_Float16)sc, (_Float16)sc};
    uint32_t raw[2][4], pr[2] = {0u, 0u};
    gg_gather(q, 0, sel, sm.book, raw[0]);
    gg_gather(q, 1, sel, sm.book, raw[1]);
    f16x8 av = gs_a<SR>(sm, cpr, m, 8u * kb, h);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const f16x8 bv = gg_scale(raw[s & 1], sc2);
        const f16x8 cur = av;
        __builtin_amdgcn_sched_barrier(0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur, bv, acc, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (s < 7) av = gs_a<SR>(sm, cpr, m, 8u * kb + (uint32_t)s + 1u, h);
        if (s < 6) {
            gg_gather_piece(q, s + 2, 0, sel, sm.book, pr[s & 1], raw[s & 1]);
            gg_gather_piece(q, s + 2, 1, sel, sm.book, pr[s & 1], raw[s & 1]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// The K loop over nk blocks: the lane's weight row at `row` (global words; block kb at byte
// 34 kb of the row, whose start parity is qpar), blocks two ahead in a ring of three registers
// sets. Ends with every wave past its last LDS read.
template <uint32_t SR>
__device__ __forceinline__ void gs_kloop(const GhLds &sm, const uint8_t *row, uint32_t qpar, uint32_t nk, uint32_t cpr,
                                         uint32_t m, uint32_t h, uint32_t sel, f32x16 &acc) {
    acc = (f32x16){};
    uint32_t d0[9], d1[9], d2[9];
    auto blk = [&](uint32_t kb) {
        return gd_global(reinterpret_cast<const uint32_t *>(row + ((int64_t)(kb * 34u) - 2 * (int64_t)((qpar + kb) & 1u))));
    };
    gs_load_blk(blk(0), d0);
    gs_load_blk(blk(1), d1);
    gg_sync<0>();  // the staged activation rows (every wave's direct loads) and the codebook
#pragma unroll 1
    for (uint32_t kb = 0; kb < nk; kb += 3u) {
        if (kb + 2u < nk) gs_load_blk(blk(kb + 2u), d2);
        gs_block<SR>(sm, d0, ((qpar + kb) & 1u) != 0u, cpr, kb, m, h, sel, acc);
        if (kb + 1u >= nk) break;
        if (kb + 3u < nk) gs_load_blk(blk(kb + 3u), d0);
        gs_block<SR>(sm, d1, ((qpar + kb + 1u) & 1u) != 0u, cpr, kb + 1u, m, h, sel, acc);
        if (kb + 2u >= nk) break;
        if (kb + 4u < nk) gs_load_blk(blk(kb + 4u), d1);
        gs_block<SR>(sm, d2, ((qpar + kb + 2u) & 1u) != 0u, cpr, kb + 2u, m, h, sel, acc);
    }
    gg_sync<0>();  // every wave is done with the activation rows and the codebook
}

// Small gate/up unit of tile descriptor td (rows <= SR) and column block fb: as gu_unit.
template <uint32_t SR, bool COHERENT>
__device__ __forceinline__ void gs_gu_unit(GhLds &sm, const GuUnitArgs &p, uint4 td, uint32_t fb) {
    uint32_t tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const uint32_t lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t e = __builtin_amdgcn_readfirstlane(td.x), row0 = __builtin_amdgcn_readfirstlane(td.y),
                   rows = __builtin_amdgcn_readfirstlane(td.z);
    const uint32_t E = p.E, F = p.F, U = p.U, m = lane & 31u, h = lane >> 5;
    reinterpret_cast<uint4 *>(sm.book)[tid] = p.codebook[tid];
    const uint32_t *order = p.order + row0;
    gs_stage_rows(sm, wave, lane, p.xh16, E, rows, [&](uint32_t r) { return order[r] / U * (E / 2u); });
    // Weight row wq of the unit: gate row fb * 128 + wq (wq < 128), up row fb * 128 + wq - 128.
    const uint32_t wq = (wave >> 2) * 128u + (wave & 3u) * 32u + m;
    const uint32_t row_bytes = (E / 128u) * 34u;
    const uint8_t *wrow = reinterpret_cast<const uint8_t *>(p.base) + (uint64_t)e * p.slot_stride +
                          (wq >> 7) * p.proj_bytes + (uint64_t)(fb * 128u + (wq & 127u)) * row_bytes;
    const bool signs = p.signs != nullptr;
    const float sgn = signs && wave < 4u ? gd_bits_f32(gd_global(p.signs)[fb * 128u + (wave & 3u) * 32u + m]) : 1.0f;
    uint32_t *out = p.act16;
    uint32_t *flag = p.flag;
    gh_settle(out, F);
    gh_settle(flag, rows);
    f32x16 acc[1];
    gs_kloop<SR>(sm, wrow, 0u, E / 128u, E / 8u, m, h, gg_sel(h), acc[0]);
    gh_gu_epilogue<1, COHERENT>(sm, acc, wave, m, h, signs, sgn, out, row0, rows, fb, F, flag);
}

// Small down unit of tile descriptor td (rows <= SR) and output column block eb: as dn_unit.
template <uint32_t SR>
__device__ __forceinline__ void gs_dn_unit(GhLds &sm, const DnUnitArgs &p, uint4 td, uint32_t eb) {
    uint32_t tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const uint32_t lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t e = __builtin_amdgcn_readfirstlane(td.x), row0 = __builtin_amdgcn_readfirstlane(td.y),
                   rows = __builtin_amdgcn_readfirstlane(td.z);
    const uint32_t E = p.E, F = p.F, m = lane & 31u, h = lane >> 5;
    reinterpret_cast<uint4 *>(sm.book)[tid] = p.codebook[tid];
    const uint32_t my_slot = gd_global(p.order)[row0 + min(tid & 127u, rows - 1u)];
    gs_stage_rows(sm, wave, lane, p.act16, F, rows, [&](uint32_t r) { return (row0 + r) * (F / 2u); });
    const uint32_t nk = F / 128u, q = eb * 256u + wave * 32u + m;  // this lane's down row
    const uint8_t *wrow = reinterpret_cast<const uint8_t *>(p.base) + (uint64_t)e * p.slot_stride + p.down_off +
                          (uint64_t)q * (nk * 34u);
    float *out = p.down32;
    gh_settle(out, E);
    f32x16 acc[1];
    gs_kloop<SR>(sm, wrow, (q * nk) & 1u, nk, F / 8u, m, h, gg_sel(h), acc[0]);
    gh_down_epilogue<1>(sm, acc, my_slot, wave, m, h, out, rows, eb, E);
}
