// Prefill path, step 5: grouped down GEMM of the sorted slots with TQ2_T dequant fused into the
// fp16 MFMA B operand.
//   down[slot][r] = W_d[e][r] . a[slot]     src/engine.zig:608-633
//
// A group takes one tile of the sort (expert e, up to 128 sorted rows) and one 128-row block
// of the expert's down matrix (128 output columns); wave w owns output columns 32 w .. +31.
// K runs over the F / 128 Gyro blocks of a down row; per block the tile's act16 rows (already
// contiguous in sorted order) are staged into LDS as in the gate/up kernel, and each lane
// decodes its own down row into the B operand (see moe_prefill_gu.hip). Results go to the
// slot's own row, down32[route_order[row]][E], in fp32 for the k-ordered combine.
// Grid: (max tiles, E / 128); 256 threads; the groups beyond the sort's tile count exit.
// Requires TQ2_T experts, F % 256 == 0.
// Constants: 0 meta_uav 1 order_uav 2 order_off 3 act16_uav 4 act16_off (words) 5 base_lo
// 6 base_hi 7 slot_stride 8 down_offset (bytes from the bundle start) 9 codebook_srv
// 10 down32_uav 11 down32_off (words) 12 E 13 F.
#include "gyro_fast.h"

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define DN_TM 128
#define DN_ROW_BYTES 272
#define DN_ABUF (DN_TM * DN_ROW_BYTES)

__device__ __forceinline__ void dn_load_blk(const uint8_t *row, uint32_t kb, uint32_t d[9]) {
    const uint32_t *p = reinterpret_cast<const uint32_t *>(row + ((kb * 34u) & ~3u));
#pragma unroll
    for (int j = 0; j < 9; ++j) d[j] = p[j];
}

__device__ __forceinline__ f16x8 dn_b_operand(const uint32_t q[8], int s, uint32_t h, half2_t scale2,
                                              const uint32_t *book) {
    const uint32_t pr = h ? tq2_pair23(q[s]) : tq2_pair01(q[s], q[(s + 7) & 7]);
    const uint32_t sa = pr & 0x7fffu, sb = __builtin_amdgcn_ubfe(pr, 16, 15);
    uint32_t a0, a1, b0, b1;
    cb_addr(sa, a0, a1);
    cb_addr(sb, b0, b1);
    u32x4 v;
    v[0] = __builtin_bit_cast(uint32_t, as_half2(lds_word(book, a0)) * scale2);
    v[1] = __builtin_bit_cast(uint32_t, as_half2(lds_word(book, a1)) * scale2);
    v[2] = __builtin_bit_cast(uint32_t, as_half2(lds_word(book, b0)) * scale2);
    v[3] = __builtin_bit_cast(uint32_t, as_half2(lds_word(book, b1)) * scale2);
    return __builtin_bit_cast(f16x8, v);
}

GD_PIPELINE_NAMED(moe_prefill_down, 256) {
    __shared__ __attribute__((aligned(16))) uint8_t abuf[2 * DN_ABUF];
    __shared__ uint4 book4[512];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t *meta = gd_buf<const uint32_t>(a, a.c[0]);
    const uint32_t tile = blockIdx.x;
    if (tile >= meta[1023]) return;
    const uint4 td = reinterpret_cast<const uint4 *>(meta + 1024u)[tile];
    const uint32_t e = td.x, row0 = td.y, rows = td.z;
    const uint32_t E = a.c[12], F = a.c[13];
    const uint32_t nrb = (rows + 31u) >> 5, nk = F / 128u, eb = blockIdx.y;

    book4[tid] = gd_buf<const uint4>(a, a.c[9])[tid];
    book4[tid + 256u] = gd_buf<const uint4>(a, a.c[9])[tid + 256u];
    const uint32_t *book = reinterpret_cast<const uint32_t *>(book4);

    const uint32_t m = lane & 31u, h = lane >> 5;
    const uint64_t base = ((uint64_t)a.c[6] << 32) | a.c[5];
    const uint32_t row_bytes = nk * 34u;
    const uint8_t *drow = reinterpret_cast<const uint8_t *>(base + (uint64_t)e * a.c[7] + a.c[8]) +
                          (size_t)(eb * 128u + wave * 32u + m) * row_bytes;

    // A staging: thread tid loads half of sorted row tid / 2 (64 words) of K block kb.
    const uint32_t sr = tid >> 1, shalf = tid & 1u;
    const bool srow = sr < rows;
    const uint32_t *asrc = gd_buf<const uint32_t>(a, a.c[3]) + a.c[4] + (size_t)(row0 + (srow ? sr : 0u)) * (F / 2u) +
                           shalf * 32u;
    u32x4 stage[8];

    f32x16 acc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = (f32x16){};
    uint32_t cur[9], nxt[9];
    dn_load_blk(drow, 0, cur);
    if (srow) {
#pragma unroll
        for (int j = 0; j < 8; ++j) stage[j] = reinterpret_cast<const u32x4 *>(asrc + 0u * 64u)[j];
    }
    if (srow) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            reinterpret_cast<u32x4 *>(abuf + 0u * DN_ABUF + sr * DN_ROW_BYTES + shalf * 128u)[j] = stage[j];
    }
    for (uint32_t kb = 0; kb < nk; ++kb) {
        const bool more = kb + 1u < nk;
        if (more) {
            if (srow) {
#pragma unroll
                for (int j = 0; j < 8; ++j) stage[j] = reinterpret_cast<const u32x4 *>(asrc + (kb + 1u) * 64u)[j];
            }
            dn_load_blk(drow, kb + 1u, nxt);
        }
        __syncthreads();
        float sc;
        uint32_t q[8];
        tq2_unpack(cur, kb & 1u, sc, q);
        const half2_t sc2 = {(_Float16)sc, (_Float16)sc};
        const uint8_t *ab = abuf + (kb & 1u) * DN_ABUF + m * DN_ROW_BYTES + h * 16u;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const f16x8 bv = dn_b_operand(q, s, h, sc2, book);
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                if ((uint32_t)rb < nrb) {
                    const f16x8 av = *reinterpret_cast<const f16x8 *>(ab + rb * 32 * DN_ROW_BYTES + s * 32);
                    acc[rb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc[rb], 0, 0, 0);
                }
            }
        }
        if (more) {
            if (srow) {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    reinterpret_cast<u32x4 *>(abuf + ((kb + 1u) & 1u) * DN_ABUF + sr * DN_ROW_BYTES + shalf * 128u)[j] = stage[j];
            }
#pragma unroll
            for (int j = 0; j < 9; ++j) cur[j] = nxt[j];
        }
    }

    // Rows go back to their slots: down32[slot][eb * 128 + 32 wave + m].
    const uint32_t *order = gd_buf<const uint32_t>(a, a.c[1]) + a.c[2];
    float *out = gd_buf<float>(a, a.c[10]) + a.c[11];
    const uint32_t col = eb * 128u + wave * 32u + m;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
        if ((uint32_t)rb < nrb) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t i = rb * 32u + (r / 4) * 8u + h * 4u + (r % 4);
                if (i < rows) out[(size_t)order[row0 + i] * E + col] = acc[rb][r];
            }
        }
    }
}
