// Prefill path for layers whose experts and projections mix Gyro types, step 4: the grouped
// gate/up GEMM of moe_prefill_gu with each expert's matrices and their types taken from the
// layer's expert table (ExpertDesc).
//   g = W_g[e] . xh, u = W_u[e] . xh        src/engine.zig:567-602 (dotRow of each matrix's
//                                           type, src/kernels.zig:201-210)
//   a = H_128 (down_signs * silu(g) * u)    src/engine.zig:603-607
//
// Group (fb, tile) runs the gate/up unit (tile, fb) of gemm_units_x.h: one tile of the sort
// (expert e, up to 128 sorted rows) against one 128-column block of F, each matrix decoded in
// its own type, so gate and up may differ.
// Grid: (F / 128, max tiles); 512 threads, one group per CU (152.5 KB of LDS).
// Requires Gyro types 144..151, E % 256 == 0, F % 128 == 0, activations within the binary16 range (checked: the range flag).
// Constants: 0 meta_uav 1 order_uav 2 order_off 3 xh16_uav 4 xh16_off (words) 5 xtab_srv
// 6 codebook_srv 7 signs_srv (0xffffffff: none) 8 signs_off 9 act16_uav 10 act16_off (words)
// 11 E 12 F 13 n_used 14 range flag (1: word 1022 of meta is set to 1 when an activation of a
// tile row leaves the binary16 range; 0: none).
#include "gemm_units_x.h"

GD_PIPELINE_NAMED_OCC(moe_prefill_gu_x, 512, 2) {
    __shared__ GxLds sm;
    const uint32_t *meta = gd_buf<const uint32_t>(a, a.c[0]);
    const uint32_t tile = blockIdx.y;
    if (tile >= __builtin_amdgcn_readfirstlane(meta[1023])) return;
    GuxArgs p;
    p.order = gd_buf<const uint32_t>(a, a.c[1]) + a.c[2];
    p.xh16 = gd_buf<const uint32_t>(a, a.c[3]) + a.c[4];
    p.xtab = gd_buf<const ExpertDesc>(a, a.c[5]);
    p.codebook = gd_buf<const uint4>(a, a.c[6]);
    p.signs = a.c[7] != 0xffffffffu ? gd_buf<const float>(a, a.c[7]) + a.c[8] : nullptr;
    p.act16 = gd_buf<uint32_t>(a, a.c[9]) + a.c[10];
    p.flag = a.c[14] ? const_cast<uint32_t *>(meta) + 1022u : nullptr;
    p.E = a.c[11];
    p.F = a.c[12];
    p.U = a.c[13];
    gux_unit<false>(sm, p, reinterpret_cast<const uint4 *>(meta + 1024u)[tile], blockIdx.x);
}
