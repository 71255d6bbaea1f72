// Prefill path, step 4: grouped gate/up GEMM of the sorted slots with TQ2_T dequant fused into
// the fp16 MFMA B operand, SwiGLU and the down-input rotation in the epilogue.
//   g = W_g[e] . xh, u = W_u[e] . xh        src/engine.zig:567-602
//   a = H_128 (down_signs * silu(g) * u)    src/engine.zig:603-607
//
// A group takes one tile of the sort (expert e, up to 128 sorted rows) and one 128-column block
// of F. Wave w owns F columns 32 w .. 32 w + 31 of the block for both gate and up, so no
// weight is decoded twice; every wave multiplies its decoded fragment into all of the tile's
// 32-row blocks (v_mfma_f32_32x32x16_f16, fp32 accumulation).
// K runs over the E / 128 Gyro blocks. Per block the tile's activations (binary16 rows of the
// rotated input, gathered through route_order) are staged into LDS, double-buffered, rows
// padded to 272 bytes so that the 16-byte A-operand reads are bank-conflict free. Each lane
// decodes the block of its own weight row: lane half h needs the trellis steps 4s + 2h and
// 4s + 2h + 1 of K-step s, two states from one v_perm of stream word s; each state names two
// codebook pairs (LDS gathers), which are exactly the B operand's binary16 pairs at
// consecutive k; one v_pk_mul_f16 by the block scale makes the weights. (The fp16 products
// scale * codebook stay finite: the host checks every layer's scales.)
// Epilogue: silu(g) * u and the down signs per value, through LDS into rows, one 128-point
// Walsh-Hadamard transform per row and wave, and binary16 rows act16[sorted row][F].
// Grid: (max tiles, F / 128); 256 threads; the groups beyond the sort's tile count exit.
// Requires TQ2_T experts, E % 128 == 0, F % 128 == 0, |xh|, |act| < 65504.
// Constants: 0 meta_uav 1 order_uav 2 order_off 3 xh16_uav 4 xh16_off (words) 5 base_lo
// 6 base_hi 7 slot_stride 8 proj_bytes 9 codebook_srv 10 signs_srv (0xffffffff: none)
// 11 signs_off 12 act16_uav 13 act16_off (words) 14 E 15 F 16 n_used.
#include "fwht.h"
#include "gyro_fast.h"

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define GU_TM 128
#define GU_ROW_BYTES 272                  // 256 bytes of K plus 16 bytes of padding
#define GU_ABUF (GU_TM * GU_ROW_BYTES)    // 34,816 bytes per buffer
#define GU_ACT_STRIDE 132                 // floats per epilogue row

// One lane's trellis block: scale and the 8 stream words (bytes 4i..4i+3 in word i).
struct Blk {
    uint32_t d[9];
};

__device__ __forceinline__ void load_blk(const uint8_t *row, uint32_t kb, Blk &b) {
    const uint32_t *p = reinterpret_cast<const uint32_t *>(row + ((kb * 34u) & ~3u));
#pragma unroll
    for (int j = 0; j < 9; ++j) b.d[j] = p[j];
}

// B operand of K-step s for lane half h: 8 binary16 weights (k = 16 s + 8 h .. + 7).
__device__ __forceinline__ f16x8 b_operand(const uint32_t q[8], int s, uint32_t h, half2_t scale2,
                                           const uint32_t *book) {
    const uint32_t pr = h ? tq2_pair23(q[s]) : tq2_pair01(q[s], q[(s + 7) & 7]);
    const uint32_t sa = pr & 0x7fffu, sb = __builtin_amdgcn_ubfe(pr, 16, 15);
    uint32_t a0, a1, b0, b1;
    cb_addr(sa, a0, a1);
    cb_addr(sb, b0, b1);
    const half2_t w0 = as_half2(lds_word(book, a0)) * scale2;
    const half2_t w1 = as_half2(lds_word(book, a1)) * scale2;
    const half2_t w2 = as_half2(lds_word(book, b0)) * scale2;
    const half2_t w3 = as_half2(lds_word(book, b1)) * scale2;
    u32x4 v;
    v[0] = __builtin_bit_cast(uint32_t, w0);
    v[1] = __builtin_bit_cast(uint32_t, w1);
    v[2] = __builtin_bit_cast(uint32_t, w2);
    v[3] = __builtin_bit_cast(uint32_t, w3);
    return __builtin_bit_cast(f16x8, v);
}

GD_PIPELINE_NAMED(moe_prefill_gu, 256) {
    __shared__ __attribute__((aligned(16))) uint8_t abuf[2 * GU_ABUF];
    __shared__ uint4 book4[512];
    __shared__ uint32_t tok[GU_TM];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t *meta = gd_buf<const uint32_t>(a, a.c[0]);
    const uint32_t tile = blockIdx.x;
    if (tile >= meta[1023]) return;
    const uint4 td = reinterpret_cast<const uint4 *>(meta + 1024u)[tile];
    const uint32_t e = td.x, row0 = td.y, rows = td.z;
    const uint32_t E = a.c[14], F = a.c[15], U = a.c[16];
    const uint32_t nrb = (rows + 31u) >> 5, nk = E / 128u, fb = blockIdx.y;

    book4[tid] = gd_buf<const uint4>(a, a.c[9])[tid];
    book4[tid + 256u] = gd_buf<const uint4>(a, a.c[9])[tid + 256u];
    if (tid < GU_TM) {
        const uint32_t r = tid < rows ? tid : 0u;
        tok[tid] = gd_buf<const uint32_t>(a, a.c[1])[a.c[2] + row0 + r] / U;
    }
    __syncthreads();
    const uint32_t *book = reinterpret_cast<const uint32_t *>(book4);

    // Weight rows of this lane: F row fb * 128 + 32 wave + (lane % 32) of gate and of up.
    const uint32_t m = lane & 31u, h = lane >> 5;
    const uint64_t base = ((uint64_t)a.c[6] << 32) | a.c[5];
    const uint32_t row_bytes = (E / 128u) * 34u;
    const uint8_t *grow = reinterpret_cast<const uint8_t *>(base + (uint64_t)e * a.c[7]) +
                          (size_t)(fb * 128u + wave * 32u + m) * row_bytes;
    const uint8_t *urow = grow + a.c[8];

    // A staging: thread tid loads half a row (64 words = 128 bytes) of K block kb.
    const uint32_t sr = tid >> 1, shalf = tid & 1u;
    const uint32_t *xsrc = gd_buf<const uint32_t>(a, a.c[3]) + a.c[4] + (size_t)tok[sr] * (E / 2u) + shalf * 32u;
    const bool srow = sr < rows;
    u32x4 stage[8];

    f32x16 accg[4], accu[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        accg[r] = (f32x16){};
        accu[r] = (f32x16){};
    }
    Blk gb, ub, gn, un;
    load_blk(grow, 0, gb);
    load_blk(urow, 0, ub);
    if (srow) {
#pragma unroll
        for (int j = 0; j < 8; ++j) stage[j] = reinterpret_cast<const u32x4 *>(xsrc + 0u * 64u)[j];
    }
    if (srow) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            reinterpret_cast<u32x4 *>(abuf + 0u * GU_ABUF + sr * GU_ROW_BYTES + shalf * 128u)[j] = stage[j];
    }
    for (uint32_t kb = 0; kb < nk; ++kb) {
        const bool more = kb + 1u < nk;
        if (more) {
            if (srow) {
#pragma unroll
                for (int j = 0; j < 8; ++j) stage[j] = reinterpret_cast<const u32x4 *>(xsrc + (kb + 1u) * 64u)[j];
            }
            load_blk(grow, kb + 1u, gn);
            load_blk(urow, kb + 1u, un);
        }
        __syncthreads();
        // This lane's gate and up blocks kb: scale and stream words.
        const bool odd = kb & 1u;
        float gs, us;
        uint32_t gq[8], uq[8];
        tq2_unpack(gb.d, odd, gs, gq);
        tq2_unpack(ub.d, odd, us, uq);
        const half2_t gs2 = {(_Float16)gs, (_Float16)gs}, us2 = {(_Float16)us, (_Float16)us};
        const uint8_t *ab = abuf + (kb & 1u) * GU_ABUF + m * GU_ROW_BYTES + h * 16u;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const f16x8 bg = b_operand(gq, s, h, gs2, book);
            const f16x8 bu = b_operand(uq, s, h, us2, book);
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                if ((uint32_t)rb < nrb) {
                    const f16x8 av = *reinterpret_cast<const f16x8 *>(ab + rb * 32 * GU_ROW_BYTES + s * 32);
                    accg[rb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bg, accg[rb], 0, 0, 0);
                    accu[rb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bu, accu[rb], 0, 0, 0);
                }
            }
        }
        if (more) {
            if (srow) {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    reinterpret_cast<u32x4 *>(abuf + ((kb + 1u) & 1u) * GU_ABUF + sr * GU_ROW_BYTES + shalf * 128u)[j] = stage[j];
            }
            gb = gn;
            ub = un;
        }
    }
    __syncthreads();  // every wave is done with the A buffers

    // Epilogue: act = down_signs * silu(g) * u into LDS rows (132-float stride).
    float *act = reinterpret_cast<float *>(abuf);
    const bool has_signs = a.c[10] != 0xffffffffu;
    const uint32_t col = wave * 32u + m;
    const float sgn = has_signs ? gd_buf<const float>(a, a.c[10])[a.c[11] + fb * 128u + col] : 1.0f;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
        if ((uint32_t)rb < nrb) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t i = rb * 32u + (r / 4) * 8u + h * 4u + (r % 4);
                act[i * GU_ACT_STRIDE + col] = gd_silu(accg[rb][r]) * accu[rb][r] * sgn;
            }
        }
    }
    __syncthreads();
    uint32_t *out = gd_buf<uint32_t>(a, a.c[12]) + a.c[13];
    for (uint32_t i = wave; i < rows; i += 4u) {
        const float2 v = *reinterpret_cast<const float2 *>(act + i * GU_ACT_STRIDE + 2u * lane);
        float x0 = v.x, x1 = v.y;
        if (has_signs) {
            gd_fwht128_wave(x0, x1);
            x0 *= GD_INV_SQRT128;
            x1 *= GD_INV_SQRT128;
        }
        const uint32_t h0 = __builtin_bit_cast(uint16_t, (_Float16)x0);
        const uint32_t h1 = __builtin_bit_cast(uint16_t, (_Float16)x1);
        out[(size_t)(row0 + i) * (F / 2u) + fb * 64u + lane] = h0 | (h1 << 16);
    }
}
