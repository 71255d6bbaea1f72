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

template <int WROW>
struct __attribute__((aligned(16))) GgLdsT {
    uint32_t book[2048];
    gd_u32x4 a[GG_NBUF][GG_ABUF / 16];             // 16-byte chunks
    gd_u32x4 w[GG_NBUF][GG_WROWS * WROW / 16];     // 16-byte chunks
    uint32_t src[GG_TM];
};
typedef GgLdsT<GG_WROW> GgLds;  // TQ2_T: 3 pieces of 16 bytes per staged block
typedef GgLdsT<64> GxLds;       // every Gyro type: up to 4 pieces (152.5 KB in all)

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

// Start of a K block for a wave that issues `newer` loads per block (activation and weight):
// at most the loads of the following block stay outstanding (none before the last block).
// newer is 1, 2, 5 or 6 (0 or 4 activation loads, 1 or 2 weight loads), uniform per wave.
__device__ __forceinline__ void gg_sync_block(uint32_t newer, bool last) {
    if (last) {
        gg_sync<0>();
        return;
    }
    switch (newer) {
        case 6: gg_sync<6>(); break;
        case 5: gg_sync<5>(); break;
        case 2: gg_sync<2>(); break;
        default: gg_sync<1>(); break;
    }
}

// Activation loads per block of wave w for a tile of nrb 32-row blocks: the waves whose 16 rows
// lie in the tile's row blocks stage them (4 loads), the others none.
__device__ __forceinline__ uint32_t gg_a_loads(uint32_t wave, uint32_t nrb) { return wave < 2u * nrb ? 4u : 0u; }

__device__ __forceinline__ uint32_t gg_lds_addr(const void *p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}

// Eight-wave groups: wave w fills activation rows 16 w .. 16 w + 15 with 4 loads of 4 rows.
template <class LDS>
__device__ __forceinline__ void gg_stage_a8(LDS &sm, uint32_t buf, uint32_t wave, const void *gbase,
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
template <class LDS>
__device__ __forceinline__ f16x8 gg_a(const LDS &sm, uint32_t buf, uint32_t r, int s, uint32_t h) {
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

// ---- Every Gyro type (the type-generic grouped GEMMs) ------------------------------------
// A staged weight row holds the block of K block kb from its 4-byte-aligned start (kb BB) & ~3
// (every Gyro block size is 2 mod 4, so the block starts at byte 2 (kb % 2) of it) in
// P = ceil((BB + 2) / 16) pieces of 16 bytes; the rows of one matrix are packed at 16 P bytes.
__device__ __forceinline__ uint32_t gx_pieces_of(uint32_t bb) { return (bb + 2u + 15u) / 16u; }

// LDS byte address of the codebook pair idx0 of a 15-bit state (as gg_cb_addr).
__device__ __forceinline__ uint32_t gg_cb_addr0(uint32_t s) {
    const uint32_t p = __umul24(s, 0x3779B1u);
    uint32_t t;
    asm("v_mad_u32_u24 %0, %1, %2, %3" : "=v"(t) : "v"(s), "s"(0x13C0u), "v"(p >> 19));
    return t & 0x1ffcu;
}

// Stream words of a k-bit block as lane half h reads them. The B operand of K-step s for half h
// covers k = 16 s + 8 h .. + 7: trellis steps 4 s + 2 h, + 1 of a 32-step type (two pairs per
// step), 8 s + 4 h .. + 3 of a 64-step type (one pair per step). Half 1's steps are D = 2 or 4
// steps after half 0's, i.e. its windows sit D K bits lower in the circular stream; rotating
// the stream up by D K bits (< 32) for half 1 gives both halves the same window offsets.
template <int ID>
__device__ __forceinline__ void gx_half_stream(uint32_t (&w)[gyro_nw<ID>()], uint32_t h) {
    constexpr int NW = gyro_nw<ID>(), R = (GyroT<ID>::S == 32 ? 2 : 4) * GyroT<ID>::K;
    uint32_t r[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) r[i] = __builtin_amdgcn_alignbit(w[i], w[(i + NW - 1) % NW], 32 - R);
#pragma unroll
    for (int i = 0; i < NW; ++i) w[i] = h ? r[i] : w[i];
}

// Codebook reads of piece p (0, 1) of K-step s from the half-adjusted stream words: a 32-step
// type's state of step 4 s + p (pairs idx0, idx1), a 64-step type's states of steps 8 s + 2 p
// and + 1 (pair idx0 each); into raw[2 p], raw[2 p + 1], the weights in k order.
template <int ID>
__device__ __forceinline__ void gx_gather_piece(const uint32_t (&w)[gyro_nw<ID>()], int s, int p, const uint32_t *book,
                                                uint32_t raw[4]) {
    if constexpr (GyroT<ID>::S == 32) {
        uint32_t a0, a1;
        gg_cb_addr(gyro_kstate<ID>(w, 4 * s + p), a0, a1);
        raw[2 * p] = book[a0 >> 2];
        raw[2 * p + 1] = book[a1 >> 2];
    } else {
        raw[2 * p] = book[gg_cb_addr0(gyro_kstate<ID>(w, 8 * s + 2 * p)) >> 2];
        raw[2 * p + 1] = book[gg_cb_addr0(gyro_kstate<ID>(w, 8 * s + 2 * p + 1)) >> 2];
    }
}

// K loop of the type-generic grouped GEMMs (moe_prefill_gu_x, moe_prefill_down_x): eight waves,
// 128 activation rows and 256 staged weight rows per K block in the three-buffer direct-load
// pipeline of the TQ2_T kernels; each wave decodes blocks of one (uniform) Gyro type.
struct GxState {
    const void *xbase;                   // activation rows
    const void *wb[2];                   // matrix of each of this wave's weight loads
    uint32_t roff[4], woff[2], wbb[2];   // per load: lane offset at block 0 (the row's first byte), block bytes
    uint32_t wpar[2], qpar;              // row start parity (2 bytes past a 4-byte boundary) per load, decode row
    uint32_t nwl;                        // weight loads per block of this wave (1 or 2)
    uint32_t nal;                        // activation loads per block of this wave (0 or 4)
    uint32_t wave, m, h, nk;
    uint32_t wrow;                       // LDS byte offset (in a weight buffer) of this lane's row
};

// Start of K block kb: the wave's loads of block kb have landed once at most the loads of block
// kb + 1 (nal activation loads and nwl weight loads) are outstanding.
__device__ __forceinline__ void gx_sync(const GxState &t, uint32_t kb) { gg_sync_block(t.nal + t.nwl, kb + 1u >= t.nk); }

// Stages K block kb into buffer buf: the wave's activation loads (if any), then its weight loads w and
// (nwl == 2) w + 8 at LDS byte 1024 L of the weight buffer; block kb of a row starts at its
// row's byte kb BB (every BB is 2 mod 4), whose 4-byte-aligned start lies 2 bytes earlier when the
// row's start parity plus kb is odd.
__device__ __forceinline__ void gx_stage(GxLds &sm, uint32_t buf, const GxState &t, uint32_t kb) {
    if (t.nal) gg_stage_a8(sm, buf, t.wave, t.xbase, t.roff, kb);
    const uint32_t base = gg_lds_addr(&sm.w[buf][0]);
    gg_dma16(base + t.wave * 1024u, t.wb[0], t.woff[0] + kb * t.wbb[0] - 2u * ((t.wpar[0] + kb) & 1u));
    if (t.nwl == 2u)
        gg_dma16(base + (t.wave + 8u) * 1024u, t.wb[1], t.woff[1] + kb * t.wbb[1] - 2u * ((t.wpar[1] + kb) & 1u));
}

// K block kb from buffer BUF for NRB 32-row blocks with blocks of Gyro type ID, in the software
// pipeline of the TQ2_T kernels: between the MFMAs of K-step s go the codebook reads of step
// s + 2 (two pieces over the first two slots) and the A operands of step s + 1 (one per slot).
template <int ID, int BUF, int NRB>
__device__ __forceinline__ void gx_step(GxLds &sm, const GxState &t, uint32_t kb, f32x16 (&acc)[NRB]) {
    gx_sync(t, kb);
    if (kb + 2u < t.nk) gx_stage(sm, (BUF + 2) % 3, t, kb + 2u);
    constexpr int NW = gyro_nw<ID>(), NQ = (NW + 1 + 3) / 4;
    const gd_u32x4 *rq = reinterpret_cast<const gd_u32x4 *>(reinterpret_cast<const uint8_t *>(&sm.w[BUF][0]) + t.wrow);
    uint32_t d[4 * NQ];
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
        const gd_u32x4 v = rq[j];
#pragma unroll
        for (int c = 0; c < 4; ++c) d[4 * j + c] = v[c];
    }
    float sc;
    uint32_t w[NW], raw[2][4], pr[2] = {0u, 0u};  // gathers of even and odd steps, two steps ahead
    const uint32_t sel = gg_sel(t.h);
    if constexpr (ID == 144) {
        tq2_unpack(d, ((t.qpar + kb) & 1u) != 0u, sc, w);
        gg_gather(w, 0, sel, sm.book, raw[0]);
        gg_gather(w, 1, sel, sm.book, raw[1]);
    } else {
        gyro_unpack<ID>(d, ((t.qpar + kb) & 1u) != 0u, sc, w);
        gx_half_stream<ID>(w, t.h);
#pragma unroll
        for (int s0 = 0; s0 < 2; ++s0) {
            gx_gather_piece<ID>(w, s0, 0, sm.book, raw[s0]);
            gx_gather_piece<ID>(w, s0, 1, sm.book, raw[s0]);
        }
    }
    const half2_t sc2 = {(_Float16)sc, (_Float16)sc};
    f16x8 av[NRB];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) av[rb] = gg_a(sm, BUF, rb * 32u + t.m, 0, t.h);
    constexpr int kPieceSlots = NRB < 2 ? NRB : 2;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const f16x8 bv = gg_scale(raw[s & 1], sc2);
        f16x8 cur[NRB];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) cur[rb] = av[rb];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NRB; ++i) {
            acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur[i], bv, acc[i], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (s < 6) {
#pragma unroll
                for (int piece = 0; piece < 2; ++piece) {
                    if (i < kPieceSlots && piece * kPieceSlots / 2 == i) {
                        if constexpr (ID == 144) gg_gather_piece(w, s + 2, piece, sel, sm.book, pr[s & 1], raw[s & 1]);
                        else gx_gather_piece<ID>(w, s + 2, piece, sm.book, raw[s & 1]);
                    }
                }
            }
            if (s < 7) av[i] = gg_a(sm, BUF, i * 32u + t.m, s + 1, t.h);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// The whole K loop of a tile for the wave's Gyro type `type` (uniform per wave; the callers
// admit only the eight types, so every wave takes one case and reaches every sync). Blocks
// rotate through the three buffers: block kb in buffer kb % 3.
template <int ID, int NRB>
__device__ __forceinline__ void gx_kloop(GxLds &sm, const GxState &t, f32x16 (&acc)[NRB]) {
    for (uint32_t kb = 0; kb < t.nk; kb += 3u) {
        gx_step<ID, 0, NRB>(sm, t, kb, acc);
        if (kb + 1u < t.nk) gx_step<ID, 1, NRB>(sm, t, kb + 1u, acc);
        if (kb + 2u < t.nk) gx_step<ID, 2, NRB>(sm, t, kb + 2u, acc);
    }
}
template <int NRB>
__device__ __forceinline__ void gx_run(GxLds &sm, const GxState &t, uint32_t type, f32x16 (&acc)[NRB]) {
#pragma unroll
    for (int r = 0; r < NRB; ++r) acc[r] = (f32x16){};
#define GX_KLOOP(ID) gx_kloop<ID, NRB>(sm, t, acc)
    GYRO_TYPE_SWITCH(type, GX_KLOOP)
#undef GX_KLOOP
    gg_sync<0>();  // every wave is done with the buffers
}

// ---- Epilogues shared by the TQ2_T and the type-generic kernels ---------------------------
// Gate/up epilogue of a tile of NRB 32-row blocks after the K loop (every wave past its last
// sync): wave w holds, for rows rb * 32 + 8 (r / 4) + 4 h + r % 4 and F-block column
// 32 (w % 4) + m, the gate (w < 4) or up (w >= 4) products in acc[rb][r].
// (1) The up waves store u, fp32 [row][column], over activation buffers 0 and 1 (64 KB).
// (2) The gate waves form act = down_signs * silu(g) * u, rounded to binary16, into activation
//     buffer 2 in the A-operand layout.
// (3) With down signs, the 128-point Walsh-Hadamard transform of every row as a GEMM with H_128
//     (entries (-1)^popcount(k & j), exact in binary16): wave w computes output columns
//     32 (w % 4) .. + 31 of the row blocks rb with rb % 2 == w / 4. The B operand of lane (j, h)
//     at K-step s holds H[16 s + 8 h + e][j] for e = 0..7, the lane's fixed pattern
//     (-1)^popcount(e & j) times (-1)^popcount((16 s + 8 h) & j). Scaled rows go to activation
//     buffer 0 (same layout).
// (4) Rows of 128 binary16 values (16 swizzled chunks) to out[row0 + i][fb * 128 ..]; COHERENT:
//     as device-scope stores, for readers on other XCDs within the same launch.
template <class LDS, int NRB, bool COHERENT = false>
__device__ __forceinline__ void gg_gu_epilogue(LDS &sm, const f32x16 (&acc)[NRB], uint32_t wave, uint32_t m,
                                               uint32_t h, const float *signs, uint32_t *out, uint32_t row0,
                                               uint32_t rows, uint32_t fb, uint32_t F, uint32_t *flag) {
    bool bad = false;  // a tile row's activation outside the binary16 range
    const bool up = wave >= 4u;
    const uint32_t cq = wave & 3u, col = cq * 32u + m;
    float *ubuf = reinterpret_cast<float *>(&sm.a[0][0]);
    if (up) {
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
            for (int r = 0; r < 16; ++r) ubuf[(rb * 32u + (r / 4) * 8u + h * 4u + (r % 4)) * 128u + col] = acc[rb][r];
    }
    __syncthreads();
    _Float16 *act = reinterpret_cast<_Float16 *>(&sm.a[2][0]);
    if (!up) {
        const float sgn = signs ? signs[fb * 128u + col] : 1.0f;
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t i = rb * 32u + (r / 4) * 8u + h * 4u + (r % 4);
                const float v = gd_silu_rcp(acc[rb][r]) * ubuf[i * 128u + col] * sgn;
                bad |= i < rows && !gd_half_ok(v);
                act[i * 128u + ((((col >> 3) ^ (i & 15u)) << 3) | (col & 7u))] = (_Float16)v;
            }
        }
    }
    __syncthreads();
    if (signs) {
        const uint32_t j = col, half = wave >> 2;
        f16x8 hp, hn;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            hp[e] = (__builtin_popcount((uint32_t)e & j) & 1) ? (_Float16)-1.0f : (_Float16)1.0f;
            hn[e] = -hp[e];
        }
        _Float16 *res = reinterpret_cast<_Float16 *>(&sm.a[0][0]);
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
            if ((uint32_t)(rb & 1) != half) continue;  // uniform per wave
            f32x16 rot = (f32x16){};
#pragma unroll
            for (int s8 = 0; s8 < 8; ++s8) {
                const f16x8 hb = (__builtin_popcount((16u * s8 + 8u * h) & j) & 1) ? hn : hp;
                rot = __builtin_amdgcn_mfma_f32_32x32x16_f16(gg_a(sm, 2, rb * 32u + m, s8, h), hb, rot, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t i = rb * 32u + (r / 4) * 8u + h * 4u + (r % 4);
                const float v = rot[r] * GD_INV_SQRT128;
                bad |= i < rows && !gd_half_ok(v);
                res[i * 128u + ((((j >> 3) ^ (i & 15u)) << 3) | (j & 7u))] = (_Float16)v;
            }
        }
        __syncthreads();
    }
    if (flag && bad) *flag = 1u;
    const gd_u32x4 *rows_src = signs ? &sm.a[0][0] : &sm.a[2][0];
    for (uint32_t idx = threadIdx.x; idx < rows * 16u; idx += 512u) {
        const uint32_t i = idx >> 4, c = idx & 15u;
        const gd_u32x4 v = rows_src[i * 16u + (c ^ (i & 15u))];
        uint32_t *dst = out + (size_t)(row0 + i) * (F / 2u) + fb * 64u + c * 4u;
        if constexpr (COHERENT) {
            __attribute__((address_space(1))) uint64_t *d =
                (__attribute__((address_space(1))) uint64_t *)(uintptr_t)dst;
            __hip_atomic_store(d, (uint64_t)v[0] | ((uint64_t)v[1] << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(d + 1, (uint64_t)v[2] | ((uint64_t)v[3] << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            *reinterpret_cast<gd_u32x4 *>(dst) = v;
        }
    }
}

// Down epilogue: wave w holds output columns 32 w + m of rows rb * 32 + 8 (r / 4) + 4 h + r % 4.
// The results pass through LDS rows of 256 floats (the 128-byte half of row i's 64-column pair
// at half (w ^ (i >> 2)) & 1, so that the two lane halves, rows i and i + 4, write different
// banks), then every sorted row i leaves as 64 chunks of 16 bytes to out[src[i]][eb * 256 ..].
template <class LDS, int NRB>
__device__ __forceinline__ void gg_down_epilogue(LDS &sm, const f32x16 (&acc)[NRB], uint32_t wave, uint32_t m,
                                                 uint32_t h, float *out, uint32_t rows, uint32_t eb, uint32_t E) {
    float *res = reinterpret_cast<float *>(&sm.a[0][0]);
    static_assert(sizeof(sm.a) + sizeof(sm.w) >= 128u * 256u * 4u, "result rows fit the K-loop buffers");
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t i = rb * 32u + (r / 4) * 8u + h * 4u + (r % 4);
            const uint32_t w = wave ^ ((i >> 2) & 1u);
            res[i * 256u + w * 32u + m] = acc[rb][r];
        }
    }
    __syncthreads();
    for (uint32_t idx = threadIdx.x; idx < rows * 64u; idx += 512u) {
        const uint32_t i = idx >> 6, c = idx & 63u;    // chunk c: columns 4 c .. 4 c + 3
        const uint32_t w = (c >> 3) ^ ((i >> 2) & 1u);  // the 32-column group's stored half
        const float4 v = *reinterpret_cast<const float4 *>(res + i * 256u + w * 32u + (c & 7u) * 4u);
        *reinterpret_cast<float4 *>(out + (size_t)sm.src[i] * E + eb * 256u + c * 4u) = v;
    }
}

// ---- Two groups per CU: the half-block pipeline of the TQ2_T kernels ----------------------
// The same tiles and decode as above in 80 KB of LDS and at most 128 VGPRs, so that two groups
// share a CU (four waves per SIMD): while one group waits at a barrier or on its gathers, the
// other issues. Activations are staged in sub-blocks of 64 K (128 bytes of a row, 16 KB for
// 128 rows) into three buffers, two sub-blocks ahead; weight blocks (128 K) go to two buffers,
// issued three sub-blocks ahead: the buffer of block b - 1 is free once every wave has passed
// the first sub-block of block b - 1, where each lane reads its block into registers.
// Issue order per wave: prologue A0 W0 A1 W1; sub-block j (after its sync) stages A(j + 2) and,
// for odd j, W((j + 3) / 2). A row's eight 16-byte chunks are XOR-swizzled (chunk c of row r
// at position c ^ ((r >> 1) & 7)), so that the A-operand reads of 16 rows (one chunk index,
// rows of even and odd parity in the two 128-byte bank halves) hit 16 different bank groups,
// and the chunk of K-step s (0..3) of a sub-block sits at byte (lane's step-0 byte) ^ 32 s.
#define GH_AROW 128
#define GH_ABUF (GG_TM * GH_AROW)

struct __attribute__((aligned(16))) GhLds {
    uint32_t book[2048];                             // 8 KB, at offset 0
    gd_u32x4 a[GG_NBUF][GH_ABUF / 16];               // 3 x 16 KB
    gd_u32x4 w[2][GG_WROWS * GG_WROW / 16];          // 2 x 12 KB
};
static_assert(sizeof(GhLds) == 81920, "two groups fill the CU's 160 KB");

struct GhState {
    const void *abase, *wbase;  // activation rows; the layer's slot arena
    uint32_t roff[2], woff[2];  // per load: lane offset at sub-block / block 0 (woff: the row's first byte)
    uint32_t wpar[2];           // per load: 1 if its row starts 2 bytes past a 4-byte boundary
    uint32_t nal, nwl;          // activation loads per sub-block (0 or 2), weight loads per block (1 or 2)
    uint32_t wave, m, h, sel, nk;
    uint32_t wq, qpar;          // staged weight row this lane decodes, and its row's start parity
    uint32_t arow;              // byte of this lane's step-0 A chunk of rows m + 32 rb in buffer 0
};

// Start of sub-block j of nj: at most the loads issued after the wave's loads of sub-block j
// (and of its weight block) stay outstanding: A(j + 1) and a weight block before the last two
// sub-blocks, A(j + 1) before the last one, none at the last.
__device__ __forceinline__ void gh_sync(const GhState &t, uint32_t j, uint32_t nj) {
    const uint32_t newer = j + 3u <= nj ? t.nal + t.nwl : (j + 2u == nj ? t.nal : 0u);
    switch (newer) {
        case 4: gg_sync<4>(); break;
        case 3: gg_sync<3>(); break;
        case 2: gg_sync<2>(); break;
        case 1: gg_sync<1>(); break;
        default: gg_sync<0>(); break;
    }
}

// Activation sub-block j of rows 16 w .. 16 w + 15: two loads of 8 rows x 128 bytes; lane l
// writes position l % 8 of row 16 w + 8 i + l / 8 (roff holds the swizzled source chunk).
__device__ __forceinline__ void gh_stage_a(GhLds &sm, uint32_t buf, const GhState &t, uint32_t j) {
    const uint32_t base = gg_lds_addr(&sm.a[0][0]) + buf * GH_ABUF + t.wave * 16u * GH_AROW;
    gg_dma16(base, t.abase, t.roff[0] + j * GH_AROW);
    gg_dma16(base + 8u * GH_AROW, t.abase, t.roff[1] + j * GH_AROW);
}
// Swizzled source chunk offset of load i for lane `lane` of wave `wave`, and its row.
__device__ __forceinline__ uint32_t gh_chunk(uint32_t wave, uint32_t lane, int i, uint32_t &row) {
    row = wave * 16u + (uint32_t)i * 8u + (lane >> 3);
    return ((lane & 7u) ^ ((row >> 1) & 7u)) * 16u;
}
// Weight block kb of the 256 staged rows (as gg_stage_w8). Block kb of a row starts at byte
// 34 kb of it; with an odd block count per row, odd rows start 2 bytes past a 4-byte boundary,
// so the 4-byte-aligned start of the block lies 2 bytes earlier when (row parity + kb) is odd.
__device__ __forceinline__ void gh_stage_w(GhLds &sm, uint32_t buf, const GhState &t, uint32_t kb) {
    const uint32_t base = gg_lds_addr(&sm.w[0][0]) + buf * (uint32_t)sizeof(sm.w[0]);
    gg_dma16(base + gg_w8_load(t.wave, 0) * 1024u, t.wbase, t.woff[0] + kb * 34u - 2u * ((t.wpar[0] + kb) & 1u));
    if (t.nwl == 2u)
        gg_dma16(base + gg_w8_load(t.wave, 1) * 1024u, t.wbase, t.woff[1] + kb * 34u - 2u * ((t.wpar[1] + kb) & 1u));
}
// Step-0 A byte of lane (m, h) in buffer 0 (row m, chunk h).
__device__ __forceinline__ uint32_t gh_arow(const GhLds &sm, uint32_t m, uint32_t h) {
    return (uint32_t)((const uint8_t *)&sm.a[0][0] - (const uint8_t *)&sm) + m * GH_AROW +
           ((h ^ ((m >> 1) & 7u)) << 4);
}
__device__ __forceinline__ f16x8 gh_a(const GhLds &sm, uint32_t byte) {
    return *reinterpret_cast<const f16x8 *>(reinterpret_cast<const uint8_t *>(&sm) + byte);
}

// Half HALF (K-steps 4 HALF .. 4 HALF + 3) of a weight block for NRB 32-row blocks, from the
// activation buffer at byte offset abyte of buffer 0 plus this lane's row: MFMAs of step s, with
// the codebook gathers of step s + 2 and the A operands of step s + 1 between them (as gu_step).
template <int HALF, int NRB>
__device__ __forceinline__ void gh_half(const GhLds &sm, uint32_t arow, const uint32_t (&q)[8], uint32_t sel,
                                        half2_t sc2, uint32_t (&raw)[2][4], uint32_t (&pr)[2], f32x16 (&acc)[NRB]) {
    f16x8 av[NRB];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) av[rb] = gh_a(sm, arow + rb * 32u * GH_AROW);
    constexpr int kPieceSlots = NRB < 2 ? NRB : 2;
#pragma unroll
    for (int sl = 0; sl < 4; ++sl) {
        const int s = 4 * HALF + sl;
        const f16x8 bv = gg_scale(raw[s & 1], sc2);
        f16x8 cur[NRB];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) cur[rb] = av[rb];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NRB; ++i) {
            acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur[i], bv, acc[i], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            // The A operand first: LDS reads retire in order, so the wait for it before the next
            // MFMA then leaves the (younger) gathers of step s + 2 in flight.
            if (sl < 3) av[i] = gh_a(sm, (arow ^ (32u * (uint32_t)(sl + 1))) + (uint32_t)i * 32u * GH_AROW);
            if (s < 6) {
#pragma unroll
                for (int piece = 0; piece < 2; ++piece)
                    if (i < kPieceSlots && piece * kPieceSlots / 2 == i)
                        gg_gather_piece(q, s + 2, piece, sel, sm.book, pr[s & 1], raw[s & 1]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// Weight row q's 9 words of staged block buffer buf.
__device__ __forceinline__ void gh_read_w(const GhLds &sm, uint32_t buf, uint32_t q, GgBlk &b) {
    const gd_u32x4 lo = sm.w[buf][q * 3u], mid = sm.w[buf][q * 3u + 1u];
    const gd_u32x4 hi = sm.w[buf][q * 3u + 2u];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        b.d[j] = lo[j];
        b.d[4 + j] = mid[j];
    }
    b.d[8] = hi[0];
}

// The K loop: blocks of 128 K as two sub-blocks, A(j) in buffer j % 3 and W(b) in buffer b % 2.
// Requires nk >= 2 and the prologue (A0 W0 A1 W1) issued; ends with every load landed and every
// wave past its last LDS read.
template <int NRB>
__device__ __forceinline__ void gh_kloop(GhLds &sm, const GhState &t, f32x16 (&acc)[NRB]) {
#pragma unroll
    for (int r = 0; r < NRB; ++r) acc[r] = (f32x16){};
    const uint32_t nj = 2u * t.nk;
    uint32_t abuf = 0;  // buffer of sub-block j: j % 3
#pragma unroll 1
    for (uint32_t kb = 0; kb < t.nk; ++kb) {
        const uint32_t j = 2u * kb;
        // Even sub-block: stage A(j + 2); read and unpack the weight block, first gathers.
        gh_sync(t, j, nj);
        if (j + 2u < nj && t.nal) gh_stage_a(sm, abuf == 0u ? 2u : abuf - 1u, t, j + 2u);
        GgBlk wc;
        gh_read_w(sm, kb & 1u, t.wq, wc);
        float sc;
        uint32_t q[8];
        tq2_unpack(wc.d, ((t.qpar + kb) & 1u) != 0u, sc, q);
        const half2_t sc2 = {(_Float16)sc, (_Float16)sc};
        uint32_t raw[2][4], pr[2] = {0u, 0u};
        gg_gather(q, 0, t.sel, sm.book, raw[0]);
        gg_gather(q, 1, t.sel, sm.book, raw[1]);
        gh_half<0, NRB>(sm, t.arow + abuf * GH_ABUF, q, t.sel, sc2, raw, pr, acc);
        abuf = abuf == 2u ? 0u : abuf + 1u;
        // Odd sub-block: stage A(j + 3) and W(kb + 2) (into the buffer of block kb, read above).
        gh_sync(t, j + 1u, nj);
        if (j + 3u < nj && t.nal) gh_stage_a(sm, abuf == 0u ? 2u : abuf - 1u, t, j + 3u);
        if (kb + 2u < t.nk) gh_stage_w(sm, kb & 1u, t, kb + 2u);
        gh_half<1, NRB>(sm, t.arow + abuf * GH_ABUF, q, t.sel, sc2, raw, pr, acc);
        abuf = abuf == 2u ? 0u : abuf + 1u;
    }
    gg_sync<0>();  // every wave is done with the buffers
}

// Makes the epilogue's scalar operands (an output pointer and a size) arrive before the K loop:
// a scalar load still outstanding there would turn every counted LDS wait of the loop into a
// wait for all LDS traffic (scalar loads return out of order).
template <class T>
__device__ __forceinline__ void gh_settle(T *ptr, uint32_t n) {
    asm volatile("" ::"s"(ptr), "s"(n));
}

// Prologue of the K loop: A0 W0 A1 W1.
__device__ __forceinline__ void gh_prologue(GhLds &sm, const GhState &t) {
    if (t.nal) gh_stage_a(sm, 0, t, 0);
    gh_stage_w(sm, 0, t, 0);
    if (t.nal) gh_stage_a(sm, 1, t, 1);
    gh_stage_w(sm, 1, t, 1);
}

// Gate/up epilogue in the 80 KB: bytes [0, 32 K) hold u (fp32, 64 rows x 128 columns, one half
// of the tile at a time) and later the rotated rows; bytes [32 K, 64 K) the act rows (binary16,
// 128 rows of 16 chunks, chunk c of row i at position c ^ (i % 16)). Otherwise as
// gg_gu_epilogue: act = down_signs * silu(g) * u rounded to binary16, then (with down signs)
// the 128-point Walsh-Hadamard transform of every row as an MFMA product with H_128, and rows
// of 128 binary16 values to out[row0 + i][fb * 128 ..].
// sgn: the down sign of this gate lane's column (1 without signs), loaded before the K loop.
template <int NRB, bool COHERENT = false>
__device__ __forceinline__ void gh_gu_epilogue(GhLds &sm, const f32x16 (&acc)[NRB], uint32_t wave, uint32_t m,
                                               uint32_t h, bool signs, float sgn, uint32_t *out, uint32_t row0,
                                               uint32_t rows, uint32_t fb, uint32_t F, uint32_t *flag) {
    bool bad = false;  // a tile row's activation outside the binary16 range
    uint8_t *lds = reinterpret_cast<uint8_t *>(&sm);
    float *ubuf = reinterpret_cast<float *>(lds);
    _Float16 *act = reinterpret_cast<_Float16 *>(lds + 32768);
    gd_u32x4 *actc = reinterpret_cast<gd_u32x4 *>(lds + 32768);
    const bool up = wave >= 4u;
    const uint32_t cq = wave & 3u, col = cq * 32u + m;
#pragma unroll
    for (int p = 0; p < (NRB + 1) / 2; ++p) {
        if (up) {
#pragma unroll
            for (int rb = 2 * p; rb < NRB && rb < 2 * p + 2; ++rb)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    ubuf[((rb - 2 * p) * 32u + (r / 4) * 8u + h * 4u + (r % 4)) * 128u + col] = acc[rb][r];
        }
        __syncthreads();
        if (!up) {
#pragma unroll
            for (int rb = 2 * p; rb < NRB && rb < 2 * p + 2; ++rb) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t iu = (rb - 2 * p) * 32u + (r / 4) * 8u + h * 4u + (r % 4), i = iu + 64u * p;
                    const float v = gd_silu_rcp(acc[rb][r]) * ubuf[iu * 128u + col] * sgn;
                    bad |= i < rows && !gd_half_ok(v);
                    act[i * 128u + ((((col >> 3) ^ (i & 15u)) << 3) | (col & 7u))] = (_Float16)v;
                }
            }
        }
        __syncthreads();
    }
    if (signs) {
        const uint32_t j = col, half = wave >> 2;
        f16x8 hp, hn;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            hp[e] = (__builtin_popcount((uint32_t)e & j) & 1) ? (_Float16)-1.0f : (_Float16)1.0f;
            hn[e] = -hp[e];
        }
        _Float16 *res = reinterpret_cast<_Float16 *>(lds);
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
            if ((uint32_t)(rb & 1) != half) continue;  // uniform per wave
            f32x16 rot = (f32x16){};
            const uint32_t i0 = rb * 32u + m;
#pragma unroll
            for (int s8 = 0; s8 < 8; ++s8) {
                const f16x8 hb = (__builtin_popcount((16u * s8 + 8u * h) & j) & 1) ? hn : hp;
                const f16x8 av = __builtin_bit_cast(f16x8, actc[i0 * 16u + (((uint32_t)(2 * s8) + h) ^ (i0 & 15u))]);
                rot = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, hb, rot, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t i = rb * 32u + (r / 4) * 8u + h * 4u + (r % 4);
                const float v = rot[r] * GD_INV_SQRT128;
                bad |= i < rows && !gd_half_ok(v);
                res[i * 128u + ((((j >> 3) ^ (i & 15u)) << 3) | (j & 7u))] = (_Float16)v;
            }
        }
        __syncthreads();
    }
    if (flag && bad) *flag = 1u;
    // Global (not flat) stores: a flat access also counts as LDS traffic in the wait counters.
    const gd_u32x4 *rows_src = reinterpret_cast<const gd_u32x4 *>(signs ? lds : lds + 32768);
    __attribute__((address_space(1))) gd_u32x4 *og =
        (__attribute__((address_space(1))) gd_u32x4 *)(uintptr_t)(out + (size_t)row0 * (F / 2u) + fb * 64u);
    for (uint32_t idx = threadIdx.x; idx < rows * 16u; idx += 512u) {
        const uint32_t i = idx >> 4, c = idx & 15u;
        const gd_u32x4 v = rows_src[i * 16u + (c ^ (i & 15u))];
        if constexpr (COHERENT) {
            // Device-scope stores (written through to the point of coherence), for readers on
            // other XCDs within the same launch.
            __attribute__((address_space(1))) uint64_t *d =
                reinterpret_cast<__attribute__((address_space(1))) uint64_t *>(og + (size_t)i * (F / 8u) + c);
            __hip_atomic_store(d, (uint64_t)v[0] | ((uint64_t)v[1] << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(d + 1, (uint64_t)v[2] | ((uint64_t)v[3] << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            og[(size_t)i * (F / 8u) + c] = v;
        }
    }
}

// Down epilogue: wave w holds output columns 32 w + m of rows rb * 32 + 8 (r / 4) + 4 h + r % 4;
// each value goes straight to out[slot of row i][eb * 256 + 32 w + m] (lanes m: 128 contiguous
// bytes of a row). my_slot: the slot of sorted row threadIdx.x (threads < 128), passed through
// LDS.
template <int NRB>
__device__ __forceinline__ void gh_down_epilogue(GhLds &sm, const f32x16 (&acc)[NRB], uint32_t my_slot,
                                                 uint32_t wave, uint32_t m, uint32_t h, float *out, uint32_t rows,
                                                 uint32_t eb, uint32_t E) {
    uint32_t *slot = reinterpret_cast<uint32_t *>(&sm);
    if (threadIdx.x < GG_TM) slot[threadIdx.x] = my_slot;
    __syncthreads();
    // Global (not flat) stores: a flat access also counts as LDS traffic in the wait counters.
    __attribute__((address_space(1))) float *o =
        (__attribute__((address_space(1))) float *)(uintptr_t)(out + eb * 256u + wave * 32u + m);
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t i = rb * 32u + (r / 4) * 8u + h * 4u + (r % 4);
            if (i < rows) o[(size_t)slot[i] * E] = acc[rb][r];
        }
    }
}
