// The work units of the TQ2_T grouped GEMMs of the prefill path (src/engine.zig:567-633), shared
// by the one-unit-per-group kernels (moe_prefill_gu, moe_prefill_down) and the persistent kernel
// that runs both kinds from one queue (moe_prefill_gemm).
//
// Gate/up unit (tile, fb): one tile of the sort (expert e, up to 128 sorted rows) against the
// 128-column block fb of F, gate and up: g = W_g[e] . xh, u = W_u[e] . xh, then
// a = H_128(down_signs * silu(g) * u) rounded to binary16 into act16[sorted row][F].
// Down unit (tile, eb): the same tile against output columns eb * 256 .. + 255 of the expert's
// down matrix: down32[slot][r] = W_d[e][r] . a[slot], fp32.
// Both take 512 threads (eight waves), the 80 KB GhLds and at most 128 VGPRs; the layout, the
// pipeline and the epilogues are those of ggemm.h.
#pragma once
#include "ggemm.h"

struct GuUnitArgs {
    const uint32_t *order;     // route_order (sorted row -> slot)
    const void *xh16;          // rotated input rows, binary16 pairs, E / 2 words per token
    uint64_t base;             // the layer's expert arena
    uint32_t slot_stride, proj_bytes;
    const uint4 *codebook;
    const uint32_t *signs;     // down signs (fp32 bits, F values) or nullptr
    uint32_t *act16;           // [sorted row][F / 2] words
    uint32_t *flag;            // range flag word or nullptr
    uint32_t E, F, U;
};

struct DnUnitArgs {
    const uint32_t *order;
    const void *act16;         // [sorted row][F / 2] words
    uint64_t base;
    uint32_t slot_stride, down_off;  // down_off: bytes from an expert's bundle start
    const uint4 *codebook;
    float *down32;             // [slot][E]
    uint32_t E, F;
};

template <int NRB, bool COHERENT>
__device__ __forceinline__ void gu_tile(GhLds &sm, const GhState &t, bool signs, float sgn, uint32_t *out,
                                        uint32_t row0, uint32_t rows, uint32_t fb, uint32_t F, uint32_t *flag) {
    f32x16 acc[NRB];
    gh_kloop<NRB>(sm, t, acc);
    gh_gu_epilogue<NRB, COHERENT>(sm, acc, t.wave, t.m, t.h, signs, sgn, out, row0, rows, fb, F, flag);
}

template <int NRB>
__device__ __forceinline__ void dn_tile(GhLds &sm, const GhState &t, float *out, uint32_t my_slot, uint32_t rows,
                                        uint32_t eb, uint32_t E) {
    f32x16 acc[NRB];
    gh_kloop<NRB>(sm, t, acc);
    gh_down_epilogue<NRB>(sm, acc, my_slot, t.wave, t.m, t.h, out, rows, eb, E);
}

// Gate/up unit of tile descriptor td = {expert, first sorted row, rows, 0} and column block fb.
// The group's LDS must be free on entry. COHERENT: act16 goes out as device-scope stores, for
// down units of the same launch on other XCDs.
template <bool COHERENT>
__device__ __forceinline__ void gu_unit(GhLds &sm, const GuUnitArgs &p, uint4 td, uint32_t fb) {
    // The thread index, opaque to the compiler, so that nothing derived from it is hoisted out
    // of a persistent caller's loop and held live through the K loop.
    uint32_t tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const uint32_t lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
    // Uniform per group: scalar branches over the row blocks.
    const uint32_t e = __builtin_amdgcn_readfirstlane(td.x), row0 = __builtin_amdgcn_readfirstlane(td.y),
                   rows = __builtin_amdgcn_readfirstlane(td.z);
    const uint32_t E = p.E, F = p.F, U = p.U;
    __builtin_assume(E >= 256u);  // K = E / 128 >= 2 blocks: no short-loop versions
    reinterpret_cast<uint4 *>(sm.book)[tid] = p.codebook[tid];

    GhState t;
    t.wave = wave;
    t.m = lane & 31u;
    t.h = lane >> 5;
    t.sel = gg_sel(t.h);
    t.nk = E / 128u;
    t.wq = (wave >> 2) * 128u + (wave & 3u) * 32u + t.m;
    t.arow = gh_arow(sm, t.m, t.h);
    t.abase = p.xh16;
    // Activation rows staged by this lane: sorted row r (padding rows repeat the last row) is
    // the xh16 row of token route_order[row0 + r] / n_used.
    const uint32_t *order = p.order + row0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        uint32_t r;
        const uint32_t c = gh_chunk(wave, lane, i, r);
        t.roff[i] = order[min(r, rows - 1u)] / U * (E * 2u) + c;
    }
    // Staged weight row q < 128: gate row fb * 128 + q; q >= 128: up row fb * 128 + q - 128.
    // Load L carries pieces 64 L + lane: row g / 3, 16-byte piece g % 3.
    t.wbase = reinterpret_cast<const void *>(p.base);
    const uint32_t row_bytes = (E / 128u) * 34u;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t g = gg_w8_load(wave, i) * 64u + lane, q = g / 3u, piece = g - q * 3u;
        t.woff[i] = e * p.slot_stride + (q >> 7) * p.proj_bytes + (fb * 128u + (q & 127u)) * row_bytes + piece * 16u;
        t.wpar[i] = 0u;  // E / 128 is even: every row starts on a 4-byte boundary
    }
    t.qpar = 0u;
    t.nwl = wave < 4u ? 2u : 1u;
    t.nal = wave < 2u * ((rows + 31u) >> 5) ? 2u : 0u;  // waves whose 16 rows lie in the tile's row blocks
    // Epilogue operands, loaded now so that no load of the epilogue is issued in the K loop; as
    // global (not flat) loads, which leave the LDS wait counts of the K loop exact.
    const bool signs = p.signs != nullptr;
    const float sgn = signs && wave < 4u ? gd_bits_f32(gd_global(p.signs)[fb * 128u + (wave & 3u) * 32u + t.m]) : 1.0f;
    uint32_t *out = p.act16;
    uint32_t *flag = p.flag;
    gh_settle(out, F);
    gh_settle(flag, rows);
    __syncthreads();  // codebook
    gh_prologue(sm, t);
    switch ((rows + 31u) >> 5) {
        case 1: gu_tile<1, COHERENT>(sm, t, signs, sgn, out, row0, rows, fb, F, flag); break;
        case 2: gu_tile<2, COHERENT>(sm, t, signs, sgn, out, row0, rows, fb, F, flag); break;
        case 3: gu_tile<3, COHERENT>(sm, t, signs, sgn, out, row0, rows, fb, F, flag); break;
        default: gu_tile<4, COHERENT>(sm, t, signs, sgn, out, row0, rows, fb, F, flag); break;
    }
}

// Down unit of tile descriptor td and output column block eb. The group's LDS must be free on
// entry, and the tile's act16 rows written.
__device__ __forceinline__ void dn_unit(GhLds &sm, const DnUnitArgs &p, uint4 td, uint32_t eb) {
    // The thread index, opaque to the compiler, so that nothing derived from it is hoisted out
    // of a persistent caller's loop and held live through the K loop.
    uint32_t tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const uint32_t lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
    const uint32_t e = __builtin_amdgcn_readfirstlane(td.x), row0 = __builtin_amdgcn_readfirstlane(td.y),
                   rows = __builtin_amdgcn_readfirstlane(td.z);
    const uint32_t E = p.E, F = p.F;
    __builtin_assume(F >= 256u);  // K = F / 128 >= 2 blocks: no short-loop versions
    reinterpret_cast<uint4 *>(sm.book)[tid] = p.codebook[tid];
    // Slot of sorted row tid (threads < 128), for the epilogue: a global (not flat) load, which
    // leaves the LDS wait counts of the K loop exact.
    const uint32_t my_slot = gd_global(p.order)[row0 + min(tid & 127u, rows - 1u)];

    GhState t;
    t.wave = wave;
    t.m = lane & 31u;
    t.h = lane >> 5;
    t.sel = gg_sel(t.h);
    t.nk = F / 128u;
    t.wq = wave * 32u + t.m;
    t.arow = gh_arow(sm, t.m, t.h);
    t.abase = p.act16;
    // Activation rows staged by this lane: sorted row row0 + r; padding rows repeat the last row.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        uint32_t r;
        const uint32_t c = gh_chunk(wave, lane, i, r);
        t.roff[i] = (row0 + min(r, rows - 1u)) * (F * 2u) + c;
    }
    // Staged weight row q: down row eb * 256 + q. Load L carries pieces 64 L + lane: row g / 3,
    // 16-byte piece g % 3.
    t.wbase = reinterpret_cast<const void *>(p.base);
    const uint32_t row_bytes = (F / 128u) * 34u;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t g = gg_w8_load(wave, i) * 64u + lane, q = g / 3u, piece = g - q * 3u;
        t.woff[i] = e * p.slot_stride + p.down_off + (eb * 256u + q) * row_bytes + piece * 16u;
        t.wpar[i] = ((eb * 256u + q) * t.nk) & 1u;  // F / 128 odd: odd rows start 2 bytes off
    }
    t.qpar = ((eb * 256u + t.wq) * t.nk) & 1u;
    t.nwl = wave < 4u ? 2u : 1u;
    t.nal = wave < 2u * ((rows + 31u) >> 5) ? 2u : 0u;  // waves whose 16 rows lie in the tile's row blocks
    float *out = p.down32;
    gh_settle(out, E);
    __syncthreads();  // codebook
    gh_prologue(sm, t);
    switch ((rows + 31u) >> 5) {
        case 1: dn_tile<1>(sm, t, out, my_slot, rows, eb, E); break;
        case 2: dn_tile<2>(sm, t, out, my_slot, rows, eb, E); break;
        case 3: dn_tile<3>(sm, t, out, my_slot, rows, eb, E); break;
        default: dn_tile<4>(sm, t, out, my_slot, rows, eb, E); break;
    }
}
