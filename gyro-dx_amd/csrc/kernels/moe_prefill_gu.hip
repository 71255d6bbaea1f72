// Prefill path, step 4: grouped gate/up GEMM of the sorted slots with TQ2_T dequant fused into
// the fp16 MFMA B operand, SwiGLU and the down-input rotation in the epilogue.
//   g = W_g[e] . xh, u = W_u[e] . xh        src/engine.zig:567-602
//   a = H_128 (down_signs * silu(g) * u)    src/engine.zig:603-607
//
// A group takes one tile of the sort (expert e, up to 128 sorted rows) and one 128-column block
// of F. Eight waves: wave w owns F columns 32 (w % 4) .. + 31 of the block for the gate (w < 4)
// or the up projection (w >= 4), so no weight is decoded twice, and the gate and up waves of one
// column range share a SIMD: while one issues MFMAs the other decodes. Each decoded fragment
// feeds all of the tile's 32-row blocks (v_mfma_f32_32x32x16_f16, fp32 accumulation). K runs
// over the E / 128 Gyro blocks: the tile's activation rows (binary16 rows of the rotated input,
// gathered through route_order) arrive in LDS in sub-blocks of 64 K two sub-blocks ahead, the
// 256 weight rows' blocks a block ahead (direct loads, the half-block pipeline of ggemm.h); each
// lane decodes the block of its own row into B operands.
// The fp16 products scale x codebook stay finite: the host checks every layer's scales.
// Epilogue: the up waves pass u through LDS (fp32, 64 rows at a time); the gate waves form
// silu(g) * u times the down signs, rounded to binary16 into LDS rows; the 128-point
// Walsh-Hadamard transform of every row runs as one more fp16 MFMA product with H_128 (exact
// +-1 entries, fp32 accumulation, then x 1/sqrt(128)), split over the eight waves; binary16
// rows go to act16[sorted row][F].
// Grid: (F / 128, max tiles); 512 threads, two groups per CU (80 KB of LDS, at most 128 VGPRs);
// groups start tile by tile in the sort's longest-first order, all column blocks of a tile
// together; the groups beyond the sort's tile count exit.
// Requires TQ2_T experts, E % 256 == 0 (rows start at 4-byte boundaries, an even block count
// of at least 2), F % 128 == 0, activations within the binary16 range (checked: the range flag).
// Constants: 0 meta_uav 1 order_uav 2 order_off 3 xh16_uav 4 xh16_off (words) 5 base_lo
// 6 base_hi 7 slot_stride 8 proj_bytes 9 codebook_srv 10 signs_srv (0xffffffff: none)
// 11 signs_off 12 act16_uav 13 act16_off (words) 14 E 15 F 16 n_used 17 range flag (1: word 1022
// of meta is set to 1 when an activation of a tile row leaves the binary16 range; 0: none).
#include "gemm_units.h"

GD_PIPELINE_NAMED_OCC(moe_prefill_gu, 512, 4) {
    __shared__ GhLds sm;
    const uint32_t *meta = gd_buf<const uint32_t>(a, a.c[0]);
    const uint32_t tile = blockIdx.y;
    if (tile >= __builtin_amdgcn_readfirstlane(meta[1023])) return;
    const uint4 td = reinterpret_cast<const uint4 *>(meta + 1024u)[tile];
    GuUnitArgs p;
    p.order = gd_buf<const uint32_t>(a, a.c[1]) + a.c[2];
    p.xh16 = gd_buf<const uint32_t>(a, a.c[3]) + a.c[4];
    p.base = ((uint64_t)a.c[6] << 32) | a.c[5];
    p.slot_stride = a.c[7];
    p.proj_bytes = a.c[8];
    p.codebook = gd_buf<const uint4>(a, a.c[9]);
    p.signs = a.c[10] != 0xffffffffu ? gd_buf<const uint32_t>(a, a.c[10]) + a.c[11] : nullptr;
    p.act16 = gd_buf<uint32_t>(a, a.c[12]) + a.c[13];
    p.flag = a.c[17] ? const_cast<uint32_t *>(meta) + 1022u : nullptr;
    p.E = a.c[14];
    p.F = a.c[15];
    p.U = a.c[16];
    gu_unit<false>(sm, p, td, blockIdx.x);
}
