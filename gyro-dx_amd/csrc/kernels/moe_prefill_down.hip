// Prefill path, step 5: grouped down GEMM of the sorted slots with TQ2_T dequant fused into the
// fp16 MFMA B operand.
//   down[slot][r] = W_d[e][r] . a[slot]     src/engine.zig:608-633
//
// A group takes one tile of the sort (expert e, up to 128 sorted rows) and one 128-row block
// of the expert's down matrix (128 output columns); wave w owns output columns 32 w .. +31.
// K runs over the F / 128 Gyro blocks of a down row; per block the tile's act16 rows (already
// contiguous in sorted order) arrive in LDS by direct loads one block ahead, and each lane
// decodes its own down row into the B operand, as in the gate/up kernel (ggemm.h). Results go
// to the slot's own row, down32[route_order[row]][E], in fp32 for the k-ordered combine.
// Grid: (max tiles, E / 128); 256 threads, two groups per CU; the groups beyond the sort's tile
// count exit. Requires TQ2_T experts, F % 256 == 0.
// Constants: 0 meta_uav 1 order_uav 2 order_off 3 act16_uav 4 act16_off (words) 5 base_lo
// 6 base_hi 7 slot_stride 8 down_offset (bytes from the bundle start) 9 codebook_srv
// 10 down32_uav 11 down32_off (words) 12 E 13 F.
#include "ggemm.h"

struct DnState {
    gd_guint *drow;     // this lane's down row
    const void *abase;  // act16 rows (byte offsets in roff)
    uint32_t roff[8];
    uint32_t wave, m, h, sel, nk;
};

// Block kb from buffer BUF with weights `cur` for NRB 32-row blocks; prefetches block kb + 1
// (see gu_step of the gate/up kernel).
template <int BUF, int NRB>
__device__ __forceinline__ void dn_step(GgLds &sm, const DnState &t, uint32_t kb, const GgBlk &cur, GgBlk &nxt,
                                        f32x16 (&acc)[NRB]) {
    float sc;
    uint32_t q[8];
    tq2_unpack(cur.d, kb & 1u, sc, q);
    const half2_t sc2 = {(_Float16)sc, (_Float16)sc};
    gg_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if (kb + 1u < t.nk) {
        gg_stage(sm, BUF ^ 1, t.wave, t.abase, t.roff, kb + 1u);
        gg_load_blk(t.drow, kb + 1u, nxt);
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const f16x8 bv = gg_b(q, s, t.sel, sc2, sm.book);
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb)
            acc[rb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(gg_a(sm, BUF, rb * 32u + t.m, s, t.h), bv, acc[rb], 0, 0, 0);
    }
}

template <int NRB>
__device__ __forceinline__ void dn_tile(GgLds &sm, const DnState &t, const GdArgs &a, uint32_t row0, uint32_t rows,
                                        uint32_t eb, uint32_t E) {
    f32x16 acc[NRB];
#pragma unroll
    for (int r = 0; r < NRB; ++r) acc[r] = (f32x16){};
    GgBlk c0, c1;
    gg_load_blk(t.drow, 0, c0);
    gg_stage(sm, 0, t.wave, t.abase, t.roff, 0);
    // nk is even: blocks alternate between buffer 0 with c0 and buffer 1 with c1.
    for (uint32_t kb = 0; kb < t.nk; kb += 2u) {
        dn_step<0, NRB>(sm, t, kb, c0, c1, acc);
        dn_step<1, NRB>(sm, t, kb + 1u, c1, c0, acc);
    }
    // Rows go back to their slots: down32[slot][eb * 128 + 32 wave + m].
    const uint32_t *order = gd_buf<const uint32_t>(a, a.c[1]) + a.c[2];
    float *out = gd_buf<float>(a, a.c[10]) + a.c[11];
    const uint32_t col = eb * 128u + t.wave * 32u + t.m;
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t i = rb * 32u + (r / 4) * 8u + t.h * 4u + (r % 4);
            if (i < rows) out[(size_t)order[row0 + i] * E + col] = acc[rb][r];
        }
    }
}

GD_PIPELINE_NAMED_OCC(moe_prefill_down, 256, 2) {
    __shared__ GgLds sm;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t *meta = gd_buf<const uint32_t>(a, a.c[0]);
    const uint32_t tile = blockIdx.x;
    if (tile >= __builtin_amdgcn_readfirstlane(meta[1023])) return;
    const uint4 td = reinterpret_cast<const uint4 *>(meta + 1024u)[tile];
    const uint32_t e = __builtin_amdgcn_readfirstlane(td.x), row0 = __builtin_amdgcn_readfirstlane(td.y),
                   rows = __builtin_amdgcn_readfirstlane(td.z);
    const uint32_t E = a.c[12], F = a.c[13], eb = blockIdx.y;

    const uint4 *cb = gd_buf<const uint4>(a, a.c[9]);
    reinterpret_cast<uint4 *>(sm.book)[tid] = cb[tid];
    reinterpret_cast<uint4 *>(sm.book)[tid + 256u] = cb[tid + 256u];
    __syncthreads();

    DnState t;
    t.wave = wave;
    t.m = lane & 31u;
    t.h = lane >> 5;
    t.sel = gg_sel(t.h);
    t.nk = F / 128u;
    t.abase = gd_buf<const uint32_t>(a, a.c[3]) + a.c[4];
    // Source row of each staged chunk: sorted row row0 + r; padding rows repeat the last row.
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint32_t r;
        const uint32_t c = gg_chunk(wave, lane, i, r);
        t.roff[i] = (row0 + min(r, rows - 1u)) * (F * 2u) + c;
    }
    const uint64_t base = ((uint64_t)a.c[6] << 32) | a.c[5];
    t.drow = gd_global(reinterpret_cast<const uint32_t *>(reinterpret_cast<const uint8_t *>(base + (uint64_t)e * a.c[7] + a.c[8]) +
                                                         (size_t)(eb * 128u + wave * 32u + t.m) * ((F / 128u) * 34u)));
    switch ((rows + 31u) >> 5) {
        case 1: dn_tile<1>(sm, t, a, row0, rows, eb, E); break;
        case 2: dn_tile<2>(sm, t, a, row0, rows, eb, E); break;
        case 3: dn_tile<3>(sm, t, a, row0, rows, eb, E); break;
        default: dn_tile<4>(sm, t, a, row0, rows, eb, E); break;
    }
}
