// Shared pieces of the grouped GEMMs of the prefill path (moe_prefill_gu, moe_prefill_down):
// fp16 MFMA 32x32x16 tiles whose B operand is decoded from TQ2_T trellis blocks in registers
// and whose A operand (activation rows of one sort tile) is staged in LDS by direct
// global-to-LDS loads.
//
// LDS of a group (one struct, so the codebook sits at offset 0 and its gather addresses need no
// base add): the codebook (8 KB), two activation buffers of 128 rows x 256 bytes (one K block
// of 128 binary16 values per row), and the tile's 128 source rows. A row's sixteen 16-byte
// chunks are XOR-swizzled, chunk c of row r at position c ^ (r % 16), so that the A-operand
// reads of 16 consecutive rows at one chunk hit 16 different bank groups.
#pragma once
#include "gyro_fast.h"

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define GG_TM 128
#define GG_ROW 256
#define GG_ABUF (GG_TM * GG_ROW)

struct __attribute__((aligned(16))) GgLds {
    uint32_t book[2048];
    gd_u32x4 a[2][GG_ABUF / 16];  // 16-byte chunks
    uint32_t src[GG_TM];
};

// Full barrier of the group: waits for every outstanding load of this wave (global loads into
// registers and global-to-LDS loads) and its LDS traffic, then synchronises the waves.
__device__ __forceinline__ void gg_barrier() { asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// One global_load_lds_dwordx4: lane l writes the 16 bytes at gbase + voff into LDS byte
// lds + 16 l (lds is uniform). Issued from inline assembly so that the compiler neither
// reorders it with LDS accesses nor adds waits of its own: gg_barrier is the only wait for it.
// M0 is set and used inside the one statement; the kernels that stage this way use M0 nowhere
// else.
__device__ __forceinline__ void gg_dma16(uint32_t lds, const void *gbase, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff), "s"(gbase) : "memory", "m0");
}

// Stages K block kb of the tile's 128 rows into buffer `buf`: wave w fills rows 32 w .. 32 w + 31
// with 8 loads of 4 rows each. row_off[i] is the byte offset (from gbase) of this lane's source
// row for load i plus its swizzled chunk, so block kb adds kb * 256 bytes.
__device__ __forceinline__ void gg_stage(GgLds &sm, uint32_t buf, uint32_t wave, const void *gbase,
                                         const uint32_t row_off[8], uint32_t kb) {
    // LDS byte address, uniform per wave (M0 takes a scalar).
    const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sm.a[buf][0] + wave * 32u * GG_ROW);
#pragma unroll
    for (int i = 0; i < 8; ++i) gg_dma16(base + i * 4u * GG_ROW, gbase, row_off[i] + kb * 256u);
}

// Byte offset of the 16-byte chunk that lane `lane` of wave `wave` stages for load i: row
// r = 32 w + 4 i + lane / 16, LDS position p = lane % 16, source chunk p ^ (r % 16).
__device__ __forceinline__ uint32_t gg_chunk(uint32_t wave, uint32_t lane, int i, uint32_t &row) {
    row = wave * 32u + (uint32_t)i * 4u + (lane >> 4);
    return ((lane & 15u) ^ (row & 15u)) * 16u;
}

// A operand of K-step s (k = 16 s + 8 h .. + 7) for tile row r: chunk 2 s + h of the row.
__device__ __forceinline__ f16x8 gg_a(const GgLds &sm, uint32_t buf, uint32_t r, int s, uint32_t h) {
    const uint32_t p = ((uint32_t)(2 * s) + h) ^ (r & 15u);
    return __builtin_bit_cast(f16x8, sm.a[buf][r * 16u + p]);
}

// One lane's trellis block: scale and the 8 stream words (bytes 4i..4i+3 in word i).
struct GgBlk {
    uint32_t d[9];
};

// Block kb of a row that starts at a 4-byte boundary: 9 words from byte (34 kb) & ~3.
__device__ __forceinline__ void gg_load_blk(gd_guint *row, uint32_t kb, GgBlk &b) {
    const uint32_t w = (kb * 34u) >> 2;
#pragma unroll
    for (int j = 0; j < 9; ++j) b.d[j] = row[w + j];
}

// LDS byte addresses of the codebook pairs of a 15-bit state (as cb_addr of gyro_fast.h). The
// multiply-add stays a v_mad_u32_u24: written in C, the compiler drops the state mask (only low
// bits reach the result) and with it the 24-bit range, and emits a quarter-rate 64-bit mad.
__device__ __forceinline__ void gg_cb_addr(uint32_t s, uint32_t &a0, uint32_t &a1) {
    const uint32_t p = __umul24(s, 0x3779B1u);
    uint32_t t;
    asm("v_mad_u32_u24 %0, %1, %2, %3" : "=v"(t) : "v"(s), "s"(0x13C0u), "v"(p >> 19));
    a0 = t & 0x1ffcu;
    a1 = (p >> 8) & 0x1ffcu;
}

// B operand of K-step s for this lane (k = 16 s + 8 h .. + 7): the two trellis steps 4 s + 2 h
// and 4 s + 2 h + 1 come from one v_perm of stream words s and s - 1 (selector `sel`: pair of
// steps 4i, 4i+1 for h = 0, 4i+2, 4i+3 for h = 1); each state names two codebook pairs, the
// weights at consecutive k, scaled by the block scale in binary16.
__device__ __forceinline__ f16x8 gg_b(const uint32_t q[8], int s, uint32_t sel, half2_t scale2,
                                      const uint32_t *book) {
    const uint32_t pr = __builtin_amdgcn_perm(q[s], q[(s + 7) & 7], sel);
    const uint32_t sa = pr & 0x7fffu, sb = __builtin_amdgcn_ubfe(pr, 16, 15);
    uint32_t a0, a1, b0, b1;
    gg_cb_addr(sa, a0, a1);
    gg_cb_addr(sb, b0, b1);
    gd_u32x4 v;
    v[0] = __builtin_bit_cast(uint32_t, as_half2(book[a0 >> 2]) * scale2);
    v[1] = __builtin_bit_cast(uint32_t, as_half2(book[a1 >> 2]) * scale2);
    v[2] = __builtin_bit_cast(uint32_t, as_half2(book[b0 >> 2]) * scale2);
    v[3] = __builtin_bit_cast(uint32_t, as_half2(book[b1 >> 2]) * scale2);
    return __builtin_bit_cast(f16x8, v);
}

// The two halves of gg_b, for software pipelining: gg_gather issues the four codebook reads of
// K-step s into raw[4]; gg_scale turns them into the B operand once they have arrived.
__device__ __forceinline__ void gg_gather(const uint32_t q[8], int s, uint32_t sel, const uint32_t *book,
                                          uint32_t raw[4]) {
    const uint32_t pr = __builtin_amdgcn_perm(q[s], q[(s + 7) & 7], sel);
    const uint32_t sa = pr & 0x7fffu, sb = __builtin_amdgcn_ubfe(pr, 16, 15);
    uint32_t a0, a1, b0, b1;
    gg_cb_addr(sa, a0, a1);
    gg_cb_addr(sb, b0, b1);
    raw[0] = book[a0 >> 2];
    raw[1] = book[a1 >> 2];
    raw[2] = book[b0 >> 2];
    raw[3] = book[b1 >> 2];
}
// One state's half of gg_gather (piece 0 also forms the state pair pr), for finer interleaving.
__device__ __forceinline__ void gg_gather_piece(const uint32_t q[8], int s, int piece, uint32_t sel,
                                                const uint32_t *book, uint32_t &pr, uint32_t raw[4]) {
    if (piece == 0) pr = __builtin_amdgcn_perm(q[s], q[(s + 7) & 7], sel);
    const uint32_t st = piece == 0 ? (pr & 0x7fffu) : __builtin_amdgcn_ubfe(pr, 16, 15);
    uint32_t a0, a1;
    gg_cb_addr(st, a0, a1);
    raw[2 * piece] = book[a0 >> 2];
    raw[2 * piece + 1] = book[a1 >> 2];
}
__device__ __forceinline__ f16x8 gg_scale(const uint32_t raw[4], half2_t scale2) {
    gd_u32x4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = __builtin_bit_cast(uint32_t, as_half2(raw[j]) * scale2);
    return __builtin_bit_cast(f16x8, v);
}

// v_perm selectors of gg_b: lane half 0 takes steps 4i, 4i+1, lane half 1 steps 4i+2, 4i+3.
__device__ __forceinline__ uint32_t gg_sel(uint32_t h) { return h ? 0x06070506u : 0x04050304u; }
