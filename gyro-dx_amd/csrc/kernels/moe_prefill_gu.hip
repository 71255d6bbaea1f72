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
#include "ggemm.h"

template <int NRB>
__device__ __forceinline__ void gu_tile(GhLds &sm, const GhState &t, bool signs, float sgn, uint32_t *out,
                                        uint32_t row0, uint32_t rows, uint32_t fb, uint32_t F, uint32_t *flag) {
    f32x16 acc[NRB];
    gh_kloop<NRB>(sm, t, acc);
    gh_gu_epilogue<NRB>(sm, acc, t.wave, t.m, t.h, signs, sgn, out, row0, rows, fb, F, flag);
}

GD_PIPELINE_NAMED_OCC(moe_prefill_gu, 512, 4) {
    __shared__ GhLds sm;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
    const uint32_t *meta = gd_buf<const uint32_t>(a, a.c[0]);
    const uint32_t tile = blockIdx.y;
    if (tile >= __builtin_amdgcn_readfirstlane(meta[1023])) return;
    const uint4 td = reinterpret_cast<const uint4 *>(meta + 1024u)[tile];
    // Uniform per group: scalar branches over the row blocks.
    const uint32_t e = __builtin_amdgcn_readfirstlane(td.x), row0 = __builtin_amdgcn_readfirstlane(td.y),
                   rows = __builtin_amdgcn_readfirstlane(td.z);
    const uint32_t E = a.c[14], F = a.c[15], U = a.c[16], fb = blockIdx.x;

    const uint4 *cb = gd_buf<const uint4>(a, a.c[9]);
    reinterpret_cast<uint4 *>(sm.book)[tid] = cb[tid];

    GhState t;
    t.wave = wave;
    t.m = lane & 31u;
    t.h = lane >> 5;
    t.sel = gg_sel(t.h);
    t.nk = E / 128u;
    t.wq = (wave >> 2) * 128u + (wave & 3u) * 32u + t.m;
    t.arow = gh_arow(sm, t.m, t.h);
    t.abase = gd_buf<const uint32_t>(a, a.c[3]) + a.c[4];
    // Activation rows staged by this lane: sorted row r (padding rows repeat the last row) is
    // the xh16 row of token route_order[row0 + r] / n_used.
    const uint32_t *order = gd_buf<const uint32_t>(a, a.c[1]) + a.c[2] + row0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        uint32_t r;
        const uint32_t c = gh_chunk(wave, lane, i, r);
        t.roff[i] = order[min(r, rows - 1u)] / U * (E * 2u) + c;
    }
    // Staged weight row q < 128: gate row fb * 128 + q; q >= 128: up row fb * 128 + q - 128.
    // Load L carries pieces 64 L + lane: row g / 3, 16-byte piece g % 3.
    t.wbase = reinterpret_cast<const void *>(((uint64_t)a.c[6] << 32) | a.c[5]);
    const uint32_t row_bytes = (E / 128u) * 34u, proj_bytes = a.c[8];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t g = gg_w8_load(wave, i) * 64u + lane, q = g / 3u, piece = g - q * 3u;
        t.woff[i] = e * a.c[7] + (q >> 7) * proj_bytes + (fb * 128u + (q & 127u)) * row_bytes + piece * 16u;
        t.wpar[i] = 0u;  // E / 128 is even: every row starts on a 4-byte boundary
    }
    t.qpar = 0u;
    t.nwl = wave < 4u ? 2u : 1u;
    t.nal = wave < 2u * ((rows + 31u) >> 5) ? 2u : 0u;  // waves whose 16 rows lie in the tile's row blocks
    // Epilogue operands, loaded now so that no load of the epilogue is issued in the K loop; as
    // global (not flat) loads, which leave the LDS wait counts of the K loop exact.
    const bool signs = a.c[10] != 0xffffffffu;
    const float sgn = signs && wave < 4u ? gd_bits_f32(gd_global(gd_buf<const uint32_t>(a, a.c[10]))
                                                           [a.c[11] + fb * 128u + (wave & 3u) * 32u + t.m])
                                        : 1.0f;
    uint32_t *out = gd_buf<uint32_t>(a, a.c[12]) + a.c[13];
    uint32_t *flag = a.c[17] ? const_cast<uint32_t *>(meta) + 1022u : nullptr;
    gh_settle(out, F);
    gh_settle(flag, rows);
    __syncthreads();  // codebook
    gh_prologue(sm, t);
    switch ((rows + 31u) >> 5) {
        case 1: gu_tile<1>(sm, t, signs, sgn, out, row0, rows, fb, F, flag); break;
        case 2: gu_tile<2>(sm, t, signs, sgn, out, row0, rows, fb, F, flag); break;
        case 3: gu_tile<3>(sm, t, signs, sgn, out, row0, rows, fb, F, flag); break;
        default: gu_tile<4>(sm, t, signs, sgn, out, row0, rows, fb, F, flag); break;
    }
}
