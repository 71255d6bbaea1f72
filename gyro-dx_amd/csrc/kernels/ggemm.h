// Shared pieces of the grouped GEMMs of the prefill path (moe_prefill_gu, moe_prefill_down):
// fp16 MFMA 32x32x16 tiles whose B operand is decoded from TQ2_T trellis blocks in registers
// and whose A operand (activation rows of one sort tile) is read from LDS.
//
// Every global load of the K loop is a direct global-to-LDS load (global_load_lds_dwordx4)
// issued from inline assembly, two K blocks ahead into one of three LDS buffers; the only wait
// for them is the counted vmcnt of gg_sync at the start of each block. (Compiler-visible loads
// would make the compiler insert waits of its own, which retire loads in order and would wait
// for the newest prefetch too.)
//
// LDS of a group (one struct, so the codebook sits at offset 0 and its gather addresses need no
// base add): the codebook (8 KB); three activation buffers of 128 rows x 256 bytes (one K block
// of 128 binary16 values per row), a row's sixteen 16-byte chunks XOR-swizzled (chunk c of row
// r at position c ^ (r % 16)) so that the A-operand reads of 16 rows at one chunk hit 16
// different bank groups; three weight buffers of up to 256 rows x 48 bytes (the 34-byte Gyro
// block of K block kb of each weight row, from its 4-byte-aligned start); the tile's source rows.
#pragma once
#include "gyro_fast.h"

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define GG_TM 128
#define GG_ROW 256
#define GG_ABUF (GG_TM * GG_ROW)
#define GG_WROW 48
#define GG_WROWS 256
#define GG_NBUF 3

struct __attribute__((aligned(16))) GgLds {
    uint32_t book[2048];
    gd_u32x4 a[GG_NBUF][GG_ABUF / 16];                // 16-byte chunks
    gd_u32x4 w[GG_NBUF][GG_WROWS * GG_WROW / 16];     // 16-byte chunks
    uint32_t src[GG_TM];
};

// Start of K block kb: waits until at most NEWER of this wave's global-to-LDS loads are
// outstanding (the loads of the following block), then for LDS traffic, and synchronises the
// group, so that every wave's loads of block kb have landed.
template <int NEWER>
__device__ __forceinline__ void gg_sync() {
    if constexpr (NEWER == 0) asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(NEWER) : "memory");
}

// One global_load_lds_dwordx4: lane l writes the 16 bytes at gbase + voff into LDS byte
// lds + 16 l (lds is uniform). M0 is set and used inside the one statement; the kernels that
// stage this way use M0 nowhere else.
__device__ __forceinline__ void gg_dma16(uint32_t lds, const void *gbase, uint32_t voff) {
    // The base and the LDS address are uniform; readfirstlane keeps them in scalar registers even
    // where the compiler has moved them to vector registers (it folds away otherwise). Its result
    // is a signed int: each half goes through uint32_t so that the low half is zero-extended.
    const uint64_t b = (uint64_t)(uintptr_t)gbase;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    const uint64_t sb = ((uint64_t)hi << 32) | (uint64_t)lo;
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff),
                 "s"(sb)
                 : "memory", "m0");
}

__device__ __forceinline__ uint32_t gg_lds_addr(const void *p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}

// Activations of K block kb into buffer buf: wave w fills rows 32 w .. 32 w + 31 with 8 loads of
// 4 rows each; roff[i] is the byte offset (from gbase) of this lane's source row for load i plus
// its swizzled chunk, so block kb adds kb * 256 bytes.
__device__ __forceinline__ void gg_stage_a(GgLds &sm, uint32_t buf, uint32_t wave, const void *gbase,
                                           const uint32_t roff[8], uint32_t kb) {
    const uint32_t base = gg_lds_addr(&sm.a[buf][0]) + wave * 32u * GG_ROW;
#pragma unroll
    for (int i = 0; i < 8; ++i) gg_dma16(base + i * 4u * GG_ROW, gbase, roff[i] + kb * 256u);
}

// Chunk offset of activation load i for a lane: row r = 32 w + 4 i + lane / 16, LDS position
// p = lane % 16, source chunk p ^ (r % 16).
__device__ __forceinline__ uint32_t gg_chunk(uint32_t wave, uint32_t lane, int i, uint32_t &row) {
    row = wave * 32u + (uint32_t)i * 4u + (lane >> 4);
    return ((lane & 15u) ^ (row & 15u)) * 16u;
}

// Eight-wave groups: wave w fills activation rows 16 w .. 16 w + 15 with 4 loads of 4 rows.
__device__ __forceinline__ void gg_stage_a8(GgLds &sm, uint32_t buf, uint32_t wave, const void *gbase,
                                            const uint32_t roff[4], uint32_t kb) {
    const uint32_t base = gg_lds_addr(&sm.a[buf][0]) + wave * 16u * GG_ROW;
#pragma unroll
    for (int i = 0; i < 4; ++i) gg_dma16(base + i * 4u * GG_ROW, gbase, roff[i] + kb * 256u);
}
__device__ __forceinline__ uint32_t gg_chunk8(uint32_t wave, uint32_t lane, int i, uint32_t &row) {
    row = wave * 16u + (uint32_t)i * 4u + (lane >> 4);
    return ((lane & 15u) ^ (row & 15u)) * 16u;
}

// Eight-wave groups, 256 weight rows (768 pieces of 16 bytes): waves 0..3 issue loads 2 w and
// 2 w + 1, waves 4..7 load 4 + w; load L covers pieces 64 L .. 64 L + 63 at LDS byte 1024 L of
// the buffer.
__device__ __forceinline__ uint32_t gg_w8_load(uint32_t wave, int i) { return wave < 4u ? wave * 2u + (uint32_t)i : wave + 4u; }
__device__ __forceinline__ void gg_stage_w8(GgLds &sm, uint32_t buf, uint32_t wave, const void *wbase,
                                            const uint32_t woff[2], uint32_t kb) {
    const uint32_t base = gg_lds_addr(&sm.w[buf][0]);
    const uint32_t kbo = (kb * 34u) & ~3u;
    gg_dma16(base + gg_w8_load(wave, 0) * 1024u, wbase, woff[0] + kbo);
    if (wave < 4u) gg_dma16(base + gg_w8_load(wave, 1) * 1024u, wbase, woff[1] + kbo);
}

// Weight blocks of K block kb into buffer buf: NW loads per wave of 64 lanes, 3 lanes (48 bytes)
// per weight row, so the 4 waves cover 4 NW 64 / 3 rows; woff[i] is the byte offset (from
// wbase) of this lane's 16 bytes of block 0, and block kb adds (34 kb) & ~3.
template <int NW>
__device__ __forceinline__ void gg_stage_w(GgLds &sm, uint32_t buf, uint32_t wave, const void *wbase,
                                           const uint32_t woff[NW], uint32_t kb) {
    const uint32_t base = gg_lds_addr(&sm.w[buf][0]) + wave * NW * 1024u;
    const uint32_t kbo = (kb * 34u) & ~3u;
#pragma unroll
    for (int i = 0; i < NW; ++i) gg_dma16(base + i * 1024u, wbase, woff[i] + kbo);
}

// The weight row and 16-byte piece that lane `lane` of wave `wave` stages with load i.
template <int NW>
__device__ __forceinline__ void gg_w_piece(uint32_t wave, uint32_t lane, int i, uint32_t &row, uint32_t &piece) {
    const uint32_t g = (wave * NW + (uint32_t)i) * 64u + lane;
    row = g / 3u;
    piece = g - row * 3u;
}

// Weight row q's 9 words of a staged block (scale and stream from the block's 4-byte-aligned
// start, as tq2_unpack expects).
struct GgBlk {
    uint32_t d[9];
};
__device__ __forceinline__ void gg_read_w(const GgLds &sm, uint32_t buf, uint32_t q, GgBlk &b) {
    const gd_u32x4 lo = sm.w[buf][q * 3u], mid = sm.w[buf][q * 3u + 1u];
    const gd_u32x4 hi = sm.w[buf][q * 3u + 2u];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        b.d[j] = lo[j];
        b.d[4 + j] = mid[j];
    }
    b.d[8] = hi[0];
}

// A operand of K-step s (k = 16 s + 8 h .. + 7) for tile row r: chunk 2 s + h of the row.
__device__ __forceinline__ f16x8 gg_a(const GgLds &sm, uint32_t buf, uint32_t r, int s, uint32_t h) {
    const uint32_t p = ((uint32_t)(2 * s) + h) ^ (r & 15u);
    return __builtin_bit_cast(f16x8, sm.a[buf][r * 16u + p]);
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

// Decode of the B operand of K-step s for this lane (k = 16 s + 8 h .. + 7) in two phases, for
// software pipelining. The two trellis steps 4 s + 2 h and 4 s + 2 h + 1 come from one v_perm of
// stream words s and s - 1 (selector gg_sel(h)); each state names two codebook pairs, the
// weights at consecutive k. gg_gather_piece issues the reads of one state (piece 0 also forms
// the state pair pr) into raw[2 piece], raw[2 piece + 1]; gg_scale turns the four raw pairs into
// the B operand, scaled by the block scale in binary16.
__device__ __forceinline__ void gg_gather_piece(const uint32_t q[8], int s, int piece, uint32_t sel,
                                                const uint32_t *book, uint32_t &pr, uint32_t raw[4]) {
    if (piece == 0) pr = __builtin_amdgcn_perm(q[s], q[(s + 7) & 7], sel);
    const uint32_t st = piece == 0 ? (pr & 0x7fffu) : __builtin_amdgcn_ubfe(pr, 16, 15);
    uint32_t a0, a1;
    gg_cb_addr(st, a0, a1);
    raw[2 * piece] = book[a0 >> 2];
    raw[2 * piece + 1] = book[a1 >> 2];
}
__device__ __forceinline__ void gg_gather(const uint32_t q[8], int s, uint32_t sel, const uint32_t *book,
                                          uint32_t raw[4]) {
    uint32_t pr = 0;
    gg_gather_piece(q, s, 0, sel, book, pr, raw);
    gg_gather_piece(q, s, 1, sel, book, pr, raw);
}
__device__ __forceinline__ f16x8 gg_scale(const uint32_t raw[4], half2_t scale2) {
    gd_u32x4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = __builtin_bit_cast(uint32_t, as_half2(raw[j]) * scale2);
    return __builtin_bit_cast(f16x8, v);
}

// v_perm selectors of gg_gather_piece: lane half 0 takes steps 4i, 4i+1, lane half 1 steps
// 4i+2, 4i+3.
__device__ __forceinline__ uint32_t gg_sel(uint32_t h) { return h ? 0x06070506u : 0x04050304u; }
