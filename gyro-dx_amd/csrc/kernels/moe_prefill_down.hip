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
#include "ggemm.h"

template <int NRB>
__device__ __forceinline__ void dn_tile(GhLds &sm, const GhState &t, float *out, uint32_t my_slot, uint32_t rows,
                                        uint32_t eb, uint32_t E) {
    f32x16 acc[NRB];
    gh_kloop<NRB>(sm, t, acc);
    gh_down_epilogue<NRB>(sm, acc, my_slot, t.wave, t.m, t.h, out, rows, eb, E);
}

GD_PIPELINE_NAMED_OCC(moe_prefill_down, 512, 4) {
    __shared__ GhLds sm;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
    const uint32_t *meta = gd_buf<const uint32_t>(a, a.c[0]);
    const uint32_t tile = blockIdx.y;
    if (tile >= __builtin_amdgcn_readfirstlane(meta[1023])) return;
    const uint4 td = reinterpret_cast<const uint4 *>(meta + 1024u)[tile];
    const uint32_t e = __builtin_amdgcn_readfirstlane(td.x), row0 = __builtin_amdgcn_readfirstlane(td.y),
                   rows = __builtin_amdgcn_readfirstlane(td.z);
    const uint32_t E = a.c[12], F = a.c[13], eb = blockIdx.x;

    const uint4 *cb = gd_buf<const uint4>(a, a.c[9]);
    reinterpret_cast<uint4 *>(sm.book)[tid] = cb[tid];
    // Slot of sorted row tid (threads < 128), for the epilogue: a global (not flat) load, which
    // leaves the LDS wait counts of the K loop exact.
    const uint32_t my_slot = gd_global(gd_buf<const uint32_t>(a, a.c[1]))[a.c[2] + row0 + min(tid & 127u, rows - 1u)];

    GhState t;
    t.wave = wave;
    t.m = lane & 31u;
    t.h = lane >> 5;
    t.sel = gg_sel(t.h);
    t.nk = F / 128u;
    t.wq = wave * 32u + t.m;
    t.arow = gh_arow(sm, t.m, t.h);
    t.abase = gd_buf<const uint32_t>(a, a.c[3]) + a.c[4];
    // Activation rows staged by this lane: sorted row row0 + r; padding rows repeat the last row.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        uint32_t r;
        const uint32_t c = gh_chunk(wave, lane, i, r);
        t.roff[i] = (row0 + min(r, rows - 1u)) * (F * 2u) + c;
    }
    // Staged weight row q: down row eb * 256 + q. Load L carries pieces 64 L + lane: row g / 3,
    // 16-byte piece g % 3.
    t.wbase = reinterpret_cast<const void *>(((uint64_t)a.c[6] << 32) | a.c[5]);
    const uint32_t row_bytes = (F / 128u) * 34u;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t g = gg_w8_load(wave, i) * 64u + lane, q = g / 3u, piece = g - q * 3u;
        t.woff[i] = e * a.c[7] + a.c[8] + (eb * 256u + q) * row_bytes + piece * 16u;
        t.wpar[i] = ((eb * 256u + q) * t.nk) & 1u;  // F / 128 odd: odd rows start 2 bytes off
    }
    t.qpar = ((eb * 256u + t.wq) * t.nk) & 1u;
    t.nwl = wave < 4u ? 2u : 1u;
    t.nal = wave < 2u * ((rows + 31u) >> 5) ? 2u : 0u;  // waves whose 16 rows lie in the tile's row blocks
    float *out = gd_buf<float>(a, a.c[10]) + a.c[11];
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
