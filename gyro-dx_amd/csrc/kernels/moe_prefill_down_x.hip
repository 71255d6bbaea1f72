// Prefill path for layers whose experts and projections mix Gyro types, step 5: the grouped down
// GEMM of moe_prefill_down with each expert's down matrix and its type taken from the layer's
// expert table (ExpertDesc).
//   down[slot][r] = W_d[e][r] . a[slot]     src/engine.zig:608-633 (dotRow of the matrix's type,
//                                           src/kernels.zig:201-210)
//
// A group takes one tile of the sort and one 256-row block of the expert's down matrix; wave w
// owns output columns 32 w .. + 31. Staged weight rows: 256 rows of P pieces of 16 bytes; the
// 4 P <= 16 loads of 64 pieces per block go to waves w (load w) and w (load w + 8, where it
// exists). K loop, B-operand decode and epilogue as the TQ2_T kernel (ggemm.h).
// Grid: (E / 256, max tiles); 512 threads, one group per CU. Requires Gyro types 144..151,
// F % 256 == 0, E % 256 == 0.
// Constants: 0 meta_uav 1 order_uav 2 order_off 3 act16_uav 4 act16_off (words) 5 xtab_srv
// 6 codebook_srv 7 down32_uav 8 down32_off (words) 9 E 10 F.
#include "ggemm.h"

template <int NRB>
__device__ __forceinline__ void dnx_tile(GxLds &sm, const GxState &t, uint32_t type, const GdArgs &a, uint32_t rows,
                                         uint32_t eb, uint32_t E) {
    f32x16 acc[NRB];
    gx_run<NRB>(sm, t, type, acc);
    gg_down_epilogue(sm, acc, t.wave, t.m, t.h, gd_buf<float>(a, a.c[7]) + a.c[8], rows, eb, E);
}

GD_PIPELINE_NAMED_OCC(moe_prefill_down_x, 512, 2) {
    __shared__ GxLds sm;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
    const uint32_t *meta = gd_buf<const uint32_t>(a, a.c[0]);
    const uint32_t tile = blockIdx.y;
    if (tile >= __builtin_amdgcn_readfirstlane(meta[1023])) return;
    const uint4 td = reinterpret_cast<const uint4 *>(meta + 1024u)[tile];
    const uint32_t e = __builtin_amdgcn_readfirstlane(td.x), row0 = __builtin_amdgcn_readfirstlane(td.y),
                   rows = __builtin_amdgcn_readfirstlane(td.z);
    const uint32_t E = a.c[9], F = a.c[10], eb = blockIdx.x;

    const ExpertDesc *xt = gd_buf<const ExpertDesc>(a, a.c[5]) + e;
    const uint32_t type = (__builtin_amdgcn_readfirstlane(xt->types) >> 16) & 0xffu;
    GyroType gt;
    if (!gd_type(type, gt)) return;  // uniform, before any barrier
    const uint32_t bb = gt.block_bytes, P = gx_pieces_of(bb);

    const uint4 *cb = gd_buf<const uint4>(a, a.c[6]);
    reinterpret_cast<uint4 *>(sm.book)[tid] = cb[tid];
    if (tid < GG_TM) sm.src[tid] = gd_buf<const uint32_t>(a, a.c[1])[a.c[2] + row0 + min(tid, rows - 1u)];

    GxState t;
    t.wave = wave;
    t.m = lane & 31u;
    t.h = lane >> 5;
    t.nk = F / 128u;
    t.xbase = gd_buf<const uint32_t>(a, a.c[3]) + a.c[4];
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
        case 1: dnx_tile<1>(sm, t, type, a, rows, eb, E); break;
        case 2: dnx_tile<2>(sm, t, type, a, rows, eb, E); break;
        case 3: dnx_tile<3>(sm, t, type, a, rows, eb, E); break;
        default: dnx_tile<4>(sm, t, type, a, rows, eb, E); break;
    }
}
