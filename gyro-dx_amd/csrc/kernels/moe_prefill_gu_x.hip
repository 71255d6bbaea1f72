// Prefill path for layers whose experts and projections mix Gyro types, step 4: the grouped
// gate/up GEMM of moe_prefill_gu with each expert's matrices and their types taken from the
// layer's expert table (ExpertDesc).
//   g = W_g[e] . xh, u = W_u[e] . xh        src/engine.zig:567-602 (dotRow of each matrix's
//                                           type, src/kernels.zig:201-210)
//   a = H_128 (down_signs * silu(g) * u)    src/engine.zig:603-607
//
// A group takes one tile of the sort (expert e, up to 128 sorted rows) and one 128-column block
// of F; wave w owns F columns 32 (w % 4) .. + 31 of the block for the gate (w < 4) or the up
// projection (w >= 4) and decodes blocks of that matrix's type, so gate and up may differ.
// Staged weight rows: the gate half first (128 rows of Pg pieces of 16 bytes), then the up half
// (128 rows of Pu pieces) at LDS byte 2048 Pg; the 2 (Pg + Pu) <= 16 loads of 64 pieces per
// block go to waves w (load w) and w (load w + 8, where it exists). A load never straddles the
// halves (each half is 2 P whole loads), so its matrix and K-block advance are uniform.
// K loop, B-operand decode and epilogue as the TQ2_T kernel (ggemm.h); the fp16 products
// scale x codebook stay finite: the host checks every layer's scales.
// Grid: (F / 128, max tiles); 512 threads, one group per CU (152.5 KB of LDS).
// Requires Gyro types 144..151, E % 256 == 0, F % 128 == 0, activations within the binary16 range (checked: the range flag).
// Constants: 0 meta_uav 1 order_uav 2 order_off 3 xh16_uav 4 xh16_off (words) 5 xtab_srv
// 6 codebook_srv 7 signs_srv (0xffffffff: none) 8 signs_off 9 act16_uav 10 act16_off (words)
// 11 E 12 F 13 n_used 14 range flag (1: word 1022 of meta is set to 1 when an activation of a
// tile row leaves the binary16 range; 0: none).
#include "ggemm.h"

template <int NRB>
__device__ __forceinline__ void gux_tile(GxLds &sm, const GxState &t, uint32_t type, const GdArgs &a, uint32_t row0,
                                         uint32_t rows, uint32_t fb, uint32_t F, uint32_t *flag) {
    f32x16 acc[NRB];
    gx_run<NRB>(sm, t, type, acc);
    const float *signs = a.c[7] != 0xffffffffu ? gd_buf<const float>(a, a.c[7]) + a.c[8] : nullptr;
    gg_gu_epilogue(sm, acc, t.wave, t.m, t.h, signs, gd_buf<uint32_t>(a, a.c[9]) + a.c[10], row0, rows, fb, F, flag);
}

GD_PIPELINE_NAMED_OCC(moe_prefill_gu_x, 512, 2) {
    __shared__ GxLds sm;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
    const uint32_t *meta = gd_buf<const uint32_t>(a, a.c[0]);
    const uint32_t tile = blockIdx.y;
    if (tile >= __builtin_amdgcn_readfirstlane(meta[1023])) return;
    const uint4 td = reinterpret_cast<const uint4 *>(meta + 1024u)[tile];
    const uint32_t e = __builtin_amdgcn_readfirstlane(td.x), row0 = __builtin_amdgcn_readfirstlane(td.y),
                   rows = __builtin_amdgcn_readfirstlane(td.z);
    const uint32_t E = a.c[11], F = a.c[12], U = a.c[13], fb = blockIdx.x;

    const ExpertDesc *xt = gd_buf<const ExpertDesc>(a, a.c[5]) + e;
    const uint32_t types = __builtin_amdgcn_readfirstlane(xt->types);
    const uint32_t tg = types & 0xffu, tu = (types >> 8) & 0xffu;
    GyroType gtg, gtu;
    if (!gd_type(tg, gtg) || !gd_type(tu, gtu)) return;  // uniform, before any barrier
    const uint32_t bbg = gtg.block_bytes, bbu = gtu.block_bytes;
    const uint32_t Pg = gx_pieces_of(bbg), Pu = gx_pieces_of(bbu);

    const uint4 *cb = gd_buf<const uint4>(a, a.c[6]);
    reinterpret_cast<uint4 *>(sm.book)[tid] = cb[tid];
    if (tid < GG_TM) sm.src[tid] = gd_buf<const uint32_t>(a, a.c[1])[a.c[2] + row0 + min(tid, rows - 1u)] / U;
    __syncthreads();

    GxState t;
    t.wave = wave;
    t.m = lane & 31u;
    t.h = lane >> 5;
    t.nk = E / 128u;
    t.xbase = gd_buf<const uint32_t>(a, a.c[3]) + a.c[4];
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
    uint32_t *flag = a.c[14] ? const_cast<uint32_t *>(meta) + 1022u : nullptr;
    switch ((rows + 31u) >> 5) {
        case 1: gux_tile<1>(sm, t, type, a, row0, rows, fb, F, flag); break;
        case 2: gux_tile<2>(sm, t, type, a, row0, rows, fb, F, flag); break;
        case 3: gux_tile<3>(sm, t, type, a, row0, rows, fb, F, flag); break;
        default: gux_tile<4>(sm, t, type, a, row0, rows, fb, F, flag); break;
    }
}
