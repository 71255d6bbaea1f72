// The work units of the type-generic grouped GEMMs of the prefill path (experts and projections
// of any of the eight Gyro types, src/engine.zig:567-633 with the types of src/gyro.zig:32-41),
// shared by the one-unit-per-group kernels (moe_prefill_gu_x, moe_prefill_down_x) and the
// persistent kernel that runs both kinds from one queue (moe_prefill_gemm_x).
//
// Gate/up unit (tile, fb): one tile of the sort (expert e, up to 128 sorted rows) against the
// 128-column block fb of F, gate and up, each matrix decoded in its own type from the layer's
// expert table: g = W_g[e] . xh, u = W_u[e] . xh, a = H_128(down_signs * silu(g) * u) rounded to
// binary16 into act16[sorted row][F]. Wave w owns F columns 32 (w % 4) .. + 31 of the block for
// the gate (w < 4) or the up projection (w >= 4). Staged weight rows: the gate half first (128
// rows of Pg pieces of 16 bytes), then the up half (128 rows of Pu pieces) at LDS byte 2048 Pg;
// the 2 (Pg + Pu) <= 16 loads of 64 pieces per block go to waves w (load w) and w (load w + 8,
// where it exists). A load never straddles the halves (each half is 2 P whole loads), so its
// matrix and K-block advance are uniform.
// Down unit (tile, eb): the same tile against output rows eb * 256 .. + 255 of the expert's down
// matrix, in its type: down32[slot][r] = W_d[e][r] . a[slot], fp32. Wave w owns output columns
// 32 w .. + 31; staged weight rows: 256 rows of P pieces, the 4 P <= 16 loads as above.
// Both take 512 threads and the 152.5 KB GxLds (one group per CU); K loop, B-operand decode and
// epilogues as ggemm.h describes. The fp16 products scale x codebook stay finite: the host
// checks every layer's scales.
#pragma once
#include "ggemm.h"

struct GuxArgs {
    const uint32_t *order;     // route_order (sorted row -> slot)
    const void *xh16;          // rotated input rows, binary16 pairs, E / 2 words per token
    const ExpertDesc *xtab;    // the layer's expert table
    const uint4 *codebook;
    const float *signs;        // down signs (F values) or nullptr
    uint32_t *act16;           // [sorted row][F / 2] words
    uint32_t *flag;            // range flag word or nullptr
    uint32_t E, F, U;
};

struct DnxArgs {
    const uint32_t *order;
    const void *act16;         // [sorted row][F / 2] words
    const ExpertDesc *xtab;
    const uint4 *codebook;
    float *down32;             // [slot][E]
    uint32_t E, F;
};

template <int NRB, bool COHERENT>
__device__ __forceinline__ void gux_tile(GxLds &sm, const GxState &t, uint32_t type, const GuxArgs &p,
                                         uint32_t row0, uint32_t rows, uint32_t fb) {
    f32x16 acc[NRB];
    gx_run<NRB>(sm, t, type, acc);
    gg_gu_epilogue<GxLds, NRB, COHERENT>(sm, acc, t.wave, t.m, t.h, p.signs, p.act16, row0, rows, fb, p.F, p.flag);
}

template <int NRB>
__device__ __forceinline__ void dnx_tile(GxLds &sm, const GxState &t, uint32_t type, const DnxArgs &p, uint32_t rows,
                                         uint32_t eb) {
    f32x16 acc[NRB];
    gx_run<NRB>(sm, t, type, acc);
    gg_down_epilogue(sm, acc, t.wave, t.m, t.h, p.down32, rows, eb, p.E);
}

// Gate/up unit of tile descriptor td = {expert, first sorted row, rows, 0} and column block fb.
// The group's LDS must be free on entry. COHERENT: act16 goes out as device-scope stores, for
// down units of the same launch on other XCDs.
template <bool COHERENT>
__device__ __forceinline__ void gux_unit(GxLds &sm, const GuxArgs &p, uint4 td, uint32_t fb) {
    // The thread index, opaque to the compiler, so that nothing derived from it is hoisted out
    // of a persistent caller's loop and held live through the K loop.
    uint32_t tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const uint32_t lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
    const uint32_t e = __builtin_amdgcn_readfirstlane(td.x), row0 = __builtin_amdgcn_readfirstlane(td.y),
                   rows = __builtin_amdgcn_readfirstlane(td.z);
    const uint32_t E = p.E, U = p.U;

    const ExpertDesc *xt = p.xtab + e;
    const uint32_t types = __builtin_amdgcn_readfirstlane(xt->types);
    const uint32_t tg = types & 0xffu, tu = (types >> 8) & 0xffu;
    GyroType gtg, gtu;
    if (!gd_type(tg, gtg) || !gd_type(tu, gtu)) return;  // uniform, before any barrier
    const uint32_t bbg = gtg.block_bytes, bbu = gtu.block_bytes;
    const uint32_t Pg = gx_pieces_of(bbg), Pu = gx_pieces_of(bbu);

    reinterpret_cast<uint4 *>(sm.book)[tid] = p.codebook[tid];
    if (tid < GG_TM) sm.src[tid] = p.order[row0 + min(tid, rows - 1u)] / U;
    __syncthreads();

    GxState t;
    t.wave = wave;
    t.m = lane & 31u;
    t.h = lane >> 5;
    t.nk = E / 128u;
    t.xbase = p.xh16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t r;
        const uint32_t c = gg_chunk8(wave, lane, i, r);
        t.roff[i] = sm.src[r] * (E * 2u) + c;
    }
    // This lane decodes staged row q = 32 (w % 4) + m of its wave's half.
    const uint32_t q = (wave & 3u) * 32u + t.m;
    t.wrow = wave < 4u ? q * 16u * Pg : 2048u * Pg + q * 16u * Pu;
    // Weight load L carries pieces 64 L' + lane of its half (L' = L, or L - 2 Pg in the up
    // half): row g / P (gate or up row fb * 128 + g / P), 16-byte piece g % P.
    const uint32_t nload = 2u * (Pg + Pu);
    t.nwl = wave + 8u < nload ? 2u : 1u;
    const uint64_t gate = xt->gate, upm = xt->up;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t L = wave + 8u * (uint32_t)i;
        const bool is_up = L >= 2u * Pg;
        const uint32_t Lh = is_up ? L - 2u * Pg : L, P = is_up ? Pu : Pg, bb = is_up ? bbu : bbg;
        const uint32_t g = Lh * 64u + lane, r = g / P, piece = g - r * P;
        t.wb[i] = reinterpret_cast<const void *>(is_up ? upm : gate);
        t.wbb[i] = bb;
        t.woff[i] = (fb * 128u + r) * ((E / 128u) * bb) + piece * 16u;
        t.wpar[i] = 0u;  // E / 128 is even: every row starts on a 4-byte boundary
    }
    t.qpar = 0u;
    t.nal = gg_a_loads(wave, (rows + 31u) >> 5);
    gx_stage(sm, 0, t, 0);
    if (t.nk > 1u) gx_stage(sm, 1, t, 1);
    const uint32_t type = wave < 4u ? tg : tu;
    switch ((rows + 31u) >> 5) {
        case 1: gux_tile<1, COHERENT>(sm, t, type, p, row0, rows, fb); break;
        case 2: gux_tile<2, COHERENT>(sm, t, type, p, row0, rows, fb); break;
        case 3: gux_tile<3, COHERENT>(sm, t, type, p, row0, rows, fb); break;
        default: gux_tile<4, COHERENT>(sm, t, type, p, row0, rows, fb); break;
    }
}

// Down unit of tile descriptor td and output row block eb. The group's LDS must be free on
// entry, and the tile's act16 rows written.
__device__ __forceinline__ void dnx_unit(GxLds &sm, const DnxArgs &p, uint4 td, uint32_t eb) {
    uint32_t tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const uint32_t lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
    const uint32_t e = __builtin_amdgcn_readfirstlane(td.x), row0 = __builtin_amdgcn_readfirstlane(td.y),
                   rows = __builtin_amdgcn_readfirstlane(td.z);
    const uint32_t F = p.F;

    const ExpertDesc *xt = p.xtab + e;
    const uint32_t type = (__builtin_amdgcn_readfirstlane(xt->types) >> 16) & 0xffu;
    GyroType gt;
    if (!gd_type(type, gt)) return;  // uniform, before any barrier
    const uint32_t bb = gt.block_bytes, P = gx_pieces_of(bb);

    reinterpret_cast<uint4 *>(sm.book)[tid] = p.codebook[tid];
    if (tid < GG_TM) sm.src[tid] = p.order[row0 + min(tid, rows - 1u)];

    GxState t;
    t.wave = wave;
    t.m = lane & 31u;
    t.h = lane >> 5;
    t.nk = F / 128u;
    t.xbase = p.act16;
    // Source row of each staged activation chunk: sorted row row0 + r; padding rows repeat the
    // last row.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t r;
        const uint32_t c = gg_chunk8(wave, lane, i, r);
        t.roff[i] = (row0 + min(r, rows - 1u)) * (F * 2u) + c;
    }
    // This lane decodes staged row 32 w + m (down row eb * 256 + 32 w + m). Weight load L carries
    // pieces 64 L + lane: row g / P, 16-byte piece g % P.
    t.wrow = (wave * 32u + t.m) * 16u * P;
    t.nwl = wave + 8u < 4u * P ? 2u : 1u;
    const uint32_t row_bytes = (F / 128u) * bb;
    const void *down = reinterpret_cast<const void *>(xt->down);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t g = (wave + 8u * (uint32_t)i) * 64u + lane, r = g / P, piece = g - r * P;
        t.wb[i] = down;
        t.wbb[i] = bb;
        t.woff[i] = (eb * 256u + r) * row_bytes + piece * 16u;
        t.wpar[i] = ((eb * 256u + r) * t.nk) & 1u;  // F / 128 odd: odd rows start 2 bytes off
    }
    t.qpar = ((eb * 256u + wave * 32u + t.m) * t.nk) & 1u;
    __syncthreads();  // codebook and slot numbers
    t.nal = gg_a_loads(wave, (rows + 31u) >> 5);
    gx_stage(sm, 0, t, 0);
    if (t.nk > 1u) gx_stage(sm, 1, t, 1);
    switch ((rows + 31u) >> 5) {
        case 1: dnx_tile<1>(sm, t, type, p, rows, eb); break;
        case 2: dnx_tile<2>(sm, t, type, p, rows, eb); break;
        case 3: dnx_tile<3>(sm, t, type, p, rows, eb); break;
        default: dnx_tile<4>(sm, t, type, p, rows, eb); break;
    }
}
