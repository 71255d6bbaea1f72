// Prefill path, step 5: grouped down GEMM of the sorted slots with TQ2_T dequant fused into the
// fp16 MFMA B operand.
//   down[slot][r] = W_d[e][r] . a[slot]     src/engine.zig:608-633
//
// A group takes one tile of the sort (expert e, up to 128 sorted rows) and one 256-row block
// of the expert's down matrix (256 output columns); eight waves, wave w owns output columns
// 32 w .. + 31. K runs over the F / 128 Gyro blocks of a down row; the tile's act16 rows
// (already contiguous in sorted order) and the 256 weight rows' blocks arrive in LDS by direct
// loads (the half-block pipeline of ggemm.h), and each lane decodes its own down row into B
// operands, with the software pipeline of the gate/up kernel. Each result goes from the
// accumulators to its slot's row, down32[route_order[row]][E] (32 lanes: 128 contiguous bytes),
// in fp32 for the k-ordered combine.
// Grid: (E / 256, max tiles); 512 threads, two groups per CU (80 KB of LDS, at most 128 VGPRs),
// started tile by tile in the sort's longest-first order; the groups beyond the sort's tile
// count exit. Requires TQ2_T experts, F % 128 == 0 with F >= 256 (an odd block count per down
// row puts odd rows 2 bytes off a 4-byte boundary; the staging and the unpack follow each row's
// parity), E % 256 == 0.
// Constants: 0 meta_uav 1 order_uav 2 order_off 3 act16_uav 4 act16_off (words) 5 base_lo
// 6 base_hi 7 slot_stride 8 down_offset (bytes from the bundle start) 9 codebook_srv
// 10 down32_uav 11 down32_off (words) 12 E 13 F.
#include "gemm_units.h"

GD_PIPELINE_NAMED_OCC(moe_prefill_down, 512, 4) {
    __shared__ GhLds sm;
    const uint32_t *meta = gd_buf<const uint32_t>(a, a.c[0]);
    const uint32_t tile = blockIdx.y;
    if (tile >= __builtin_amdgcn_readfirstlane(meta[1023])) return;
    const uint4 td = reinterpret_cast<const uint4 *>(meta + 1024u)[tile];
    DnUnitArgs p;
    p.order = gd_buf<const uint32_t>(a, a.c[1]) + a.c[2];
    p.act16 = gd_buf<const uint32_t>(a, a.c[3]) + a.c[4];
    p.base = ((uint64_t)a.c[6] << 32) | a.c[5];
    p.slot_stride = a.c[7];
    p.down_off = a.c[8];
    p.codebook = gd_buf<const uint4>(a, a.c[9]);
    p.down32 = gd_buf<float>(a, a.c[10]) + a.c[11];
    p.E = a.c[12];
    p.F = a.c[13];
    dn_unit(sm, p, td, blockIdx.x);
}
