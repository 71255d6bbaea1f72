// Prefill path for layers whose experts and projections mix Gyro types, step 5: the grouped down
// GEMM of moe_prefill_down with each expert's down matrix and its type taken from the layer's
// expert table (ExpertDesc).
//   down[slot][r] = W_d[e][r] . a[slot]     src/engine.zig:608-633 (dotRow of the matrix's type,
//                                           src/kernels.zig:201-210)
//
// Group (eb, tile) runs the down unit (tile, eb) of gemm_units_x.h: one tile of the sort against
// one 256-row block of the expert's down matrix, decoded in its type.
// Grid: (E / 256, max tiles); 512 threads, one group per CU. Requires Gyro types 144..151,
// E % 256 == 0, F % 128 == 0 with F >= 256 (an odd F / 128 is handled: odd rows start 2 bytes
// past a 4-byte boundary).
// Constants: 0 meta_uav 1 order_uav 2 order_off 3 act16_uav 4 act16_off (words) 5 xtab_srv
// 6 codebook_srv 7 down32_uav 8 down32_off (words) 9 E 10 F.
#include "gemm_units_x.h"

GD_PIPELINE_NAMED_OCC(moe_prefill_down_x, 512, 2) {
    __shared__ GxLds sm;
    const uint32_t *meta = gd_buf<const uint32_t>(a, a.c[0]);
    const uint32_t tile = blockIdx.y;
    if (tile >= __builtin_amdgcn_readfirstlane(meta[1023])) return;
    DnxArgs p;
    p.order = gd_buf<const uint32_t>(a, a.c[1]) + a.c[2];
    p.act16 = gd_buf<const uint32_t>(a, a.c[3]) + a.c[4];
    p.xtab = gd_buf<const ExpertDesc>(a, a.c[5]);
    p.codebook = gd_buf<const uint4>(a, a.c[6]);
    p.down32 = gd_buf<float>(a, a.c[7]) + a.c[8];
    p.E = a.c[9];
    p.F = a.c[10];
    dnx_unit(sm, p, reinterpret_cast<const uint4 *>(meta + 1024u)[tile], blockIdx.x);
}
