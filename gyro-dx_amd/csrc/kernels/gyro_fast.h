// Building blocks of the MI355X fast paths: TQ2_T trellis states from packed stream words,
// the hash and LDS codebook addressing in 24-bit integer arithmetic, and the per-layer
// expert descriptor table.
#pragma once
#include "gd_kernel.h"

// Expert descriptor: device addresses of one expert's gate, up and down rows, and their Gyro
// types (one byte each, projection p in bits 8p..8p+7). 32 bytes per expert.
struct ExpertDesc {
    uint64_t gate, up, down;
    uint32_t types;
    uint32_t pad;
};

// Two 15-bit TQ2_T states from stream word q (bytes 4i..4i+3) and the previous word qp:
// lo16 = state of step 4i (+0) or 4i+2 (+2), hi16 = the following step, before masking.
// v_perm_b32 picks bytes from {q : qp}; pool bytes 0-3 are qp, 4-7 are q.
__device__ __forceinline__ uint32_t tq2_pair01(uint32_t q, uint32_t qp) {
    return __builtin_amdgcn_perm(q, qp, 0x04050304u);  // [b4i, b4i-1, b4i+1, b4i]
}
__device__ __forceinline__ uint32_t tq2_pair23(uint32_t q) {
    return __builtin_amdgcn_perm(q, q, 0x06070506u);   // [b4i+2, b4i+1, b4i+3, b4i+2]
}

// LDS byte addresses of the two codebook pairs of a 15-bit state s (SPEC section 5):
// x = s * 0x9E3779B1 mod 2^32 = p + ((s * 0x9E) << 24) with p = s * 0x3779B1 (24-bit product);
// idx1 * 4 = (x >> 8) & 0x1ffc only sees p; idx0 * 4 = (x >> 19) & 0x1ffc
//          = ((p >> 19) + s * (0x9E << 5)) & 0x1ffc.
__device__ __forceinline__ void cb_addr(uint32_t s, uint32_t &a0, uint32_t &a1) {
    const uint32_t p = __umul24(s, 0x3779B1u);
    a1 = (p >> 8) & 0x1ffcu;
    a0 = (__umul24(s, 0x13C0u) + (p >> 19)) & 0x1ffcu;
}
__device__ __forceinline__ uint32_t cb_addr0(uint32_t s) {
    const uint32_t p = __umul24(s, 0x3779B1u);
    return (__umul24(s, 0x13C0u) + (p >> 19)) & 0x1ffcu;
}

__device__ __forceinline__ uint32_t lds_word(const uint32_t *book_base, uint32_t byte_addr) {
    return *reinterpret_cast<const uint32_t *>(reinterpret_cast<const uint8_t *>(book_base) + byte_addr);
}

// fp16 half of a codebook word times an fp32 activation, accumulated in fp32 (v_fma_mix_f32).
__device__ __forceinline__ float fma_lo(uint32_t w, float x, float acc) {
    return __builtin_fmaf(gd_half(w & 0xffffu), x, acc);
}
__device__ __forceinline__ float fma_hi(uint32_t w, float x, float acc) {
    return __builtin_fmaf(gd_half(w >> 16), x, acc);
}

// Read-only global data viewed through the constant address space: wave-uniform loads of it
// become scalar loads (the scalar cache is invalidated at every dispatch). Only for buffers
// that no wave writes during the dispatch.
typedef const __attribute__((address_space(4))) float cfloat;
typedef const __attribute__((address_space(4))) uint32_t cuint;
__device__ __forceinline__ cfloat *as_const(const float *p) { return (cfloat *)(uintptr_t)p; }
__device__ __forceinline__ cuint *as_const(const uint32_t *p) { return (cuint *)(uintptr_t)p; }

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ half2_t as_half2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }

// Dot of one TQ2_T block's 32 steps with 128 activations, given the 8 stream words; returns
// the unscaled sum of codebook * x. X is a uniform cfloat* (scalar loads), an LDS pointer or a
// register array.
template <typename XP>
__device__ __forceinline__ float tq2_block_dot(const uint32_t q[8], const uint32_t *book, XP x) {
    float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t qp = q[(i + 7) & 7];
        const uint32_t p01 = tq2_pair01(q[i], qp), p23 = tq2_pair23(q[i]);
        const uint32_t s[4] = {p01 & 0x7fffu, __builtin_amdgcn_ubfe(p01, 16, 15), p23 & 0x7fffu,
                               __builtin_amdgcn_ubfe(p23, 16, 15)};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t a0, a1;
            cb_addr(s[j], a0, a1);
            const uint32_t w0 = lds_word(book, a0), w1 = lds_word(book, a1);
            const XP xs = x + (i * 4 + j) * 4;
            acc0 = fma_lo(w0, xs[0], acc0);
            acc1 = fma_hi(w0, xs[1], acc1);
            acc0 = fma_lo(w1, xs[2], acc0);
            acc1 = fma_hi(w1, xs[3], acc1);
        }
    }
    return acc0 + acc1;
}

// Half of tq2_block_dot: trellis steps 16 half .. 16 half + 15 (stream words 4 half .. + 3, and
// the word before them for the first state) against x[64 half .. 64 half + 63].
template <typename XP>
__device__ __forceinline__ float tq2_half_dot(const uint32_t q[8], uint32_t half, const uint32_t *book, XP x) {
    float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t qi = half ? q[4 + i] : q[i];
        const uint32_t qp = half ? q[3 + i] : q[(i + 7) & 7];
        const uint32_t p01 = tq2_pair01(qi, qp), p23 = tq2_pair23(qi);
        const uint32_t s[4] = {p01 & 0x7fffu, __builtin_amdgcn_ubfe(p01, 16, 15), p23 & 0x7fffu,
                               __builtin_amdgcn_ubfe(p23, 16, 15)};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t a0, a1;
            cb_addr(s[j], a0, a1);
            const uint32_t w0 = lds_word(book, a0), w1 = lds_word(book, a1);
            const XP xs = x + (i * 4 + j) * 4;
            acc0 = fma_lo(w0, xs[0], acc0);
            acc1 = fma_hi(w0, xs[1], acc1);
            acc0 = fma_lo(w1, xs[2], acc0);
            acc1 = fma_hi(w1, xs[3], acc1);
        }
    }
    return acc0 + acc1;
}

// Rotated fp32 activations staged in LDS as 16-byte chunks, chunk c of 128-block bx at
// bx * 32 + (c + bx) % 32: the eight blocks that a wave's lanes read at one chunk index then sit
// in eight different bank groups. x32_stage_index gives the position of chunk c of block bx;
// x32_from_lds copies block b's 128 values into registers (x[i] = activation i of the block).
__device__ __forceinline__ uint32_t x32_stage_index(uint32_t bx, uint32_t c) { return bx * 32u + ((c + bx) & 31u); }
__device__ __forceinline__ void x32_from_lds(const uint4 *xl, uint32_t b, float x[128]) {
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const uint4 v = xl[x32_stage_index(b, (uint32_t)j)];
        x[4 * j] = gd_bits_f32(v.x);
        x[4 * j + 1] = gd_bits_f32(v.y);
        x[4 * j + 2] = gd_bits_f32(v.z);
        x[4 * j + 3] = gd_bits_f32(v.w);
    }
}

// Rotated fp32 activations staged in LDS with one 16-byte chunk of padding per 128-block: chunk c
// of block bx at bx * 33 + c. Block b's 128 values stay contiguous (uint4 33 b ..), so they are
// read at constant offsets from one base, and the eight blocks that a wave's lanes read at one
// chunk index still sit in eight different bank groups.
__device__ __forceinline__ uint32_t x33_stage_index(uint32_t bx, uint32_t c) { return bx * 33u + c; }
// Block's 128 values (starting at xb) into registers: x[i] = activation i of the block.
__device__ __forceinline__ void x33_from_lds(const uint4 *xb, float x[128]) {
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const uint4 v = xb[j];
        x[4 * j] = gd_bits_f32(v.x);
        x[4 * j + 1] = gd_bits_f32(v.y);
        x[4 * j + 2] = gd_bits_f32(v.z);
        x[4 * j + 3] = gd_bits_f32(v.w);
    }
}

// tq2_block_dot of the block whose 128 activations start at xb (LDS, the x33 layout), in two
// halves: the 64 activations of steps 0-15 go into registers, then those of steps 16-31, so the
// dot holds 64 of them at a time (64 VGPRs in all, against 156 for the whole block). The products
// and their order are tq2_block_dot's, so the result is the same bit for bit.
__device__ __forceinline__ float tq2_block_dot_halves(const uint32_t q[8], const uint32_t *book, const uint4 *xb) {
    float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        float x[64];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint4 v = xb[16 * h + j];
            x[4 * j] = gd_bits_f32(v.x);
            x[4 * j + 1] = gd_bits_f32(v.y);
            x[4 * j + 2] = gd_bits_f32(v.z);
            x[4 * j + 3] = gd_bits_f32(v.w);
        }
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            const int i = 4 * h + ii;
            const uint32_t qp = q[(i + 7) & 7];
            const uint32_t p01 = tq2_pair01(q[i], qp), p23 = tq2_pair23(q[i]);
            const uint32_t s[4] = {p01 & 0x7fffu, __builtin_amdgcn_ubfe(p01, 16, 15), p23 & 0x7fffu,
                                   __builtin_amdgcn_ubfe(p23, 16, 15)};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t a0, a1;
                cb_addr(s[j], a0, a1);
                const uint32_t w0 = lds_word(book, a0), w1 = lds_word(book, a1);
                const float *xs = x + (ii * 4 + j) * 4;
                acc0 = fma_lo(w0, xs[0], acc0);
                acc1 = fma_hi(w0, xs[1], acc1);
                acc0 = fma_lo(w1, xs[2], acc0);
                acc1 = fma_hi(w1, xs[3], acc1);
            }
        }
    }
    return acc0 + acc1;
}

// The 9 words from the 4-byte-aligned start of the 34-byte block at byte `off` (even) of `base`.
__device__ __forceinline__ void tq2_load_block(const uint8_t *base, uint64_t off, uint32_t d[9]) {
    gd_guint *w = gd_global(reinterpret_cast<const uint32_t *>(base + (off & ~uint64_t(3))));
#pragma unroll
    for (int j = 0; j < 9; ++j) d[j] = w[j];
}

// Extracts the scale and the 8 aligned stream words of a 34-byte block that starts at byte
// offset `off` (even) inside the 32-bit words d[] (d[0] holds bytes off & ~3 ..).
// Blocks at offsets 0 mod 4 have their stream at 2 mod 4, and vice versa.
__device__ __forceinline__ void tq2_unpack(const uint32_t *d, bool odd_half, float &scale, uint32_t q[8]) {
    if (!odd_half) {  // block starts at a word boundary: scale = d0.lo, stream at byte 2
        scale = gd_half(d[0] & 0xffffu);
#pragma unroll
        for (int j = 0; j < 8; ++j) q[j] = __builtin_amdgcn_alignbyte(d[j + 1], d[j], 2);
    } else {  // block starts at byte 2 of d0: scale = d0.hi, stream word-aligned at d1
        scale = gd_half(d[0] >> 16);
#pragma unroll
        for (int j = 0; j < 8; ++j) q[j] = d[j + 1];
    }
}

// ---- Every Gyro type (src/gyro.zig:32-41) from packed words -------------------------------
// GyroT<ID>: K new bits per step, S steps, BB block bytes (2 scale bytes + S K / 8 stream
// bytes), NW stream words.
template <int ID> struct GyroT;
template <> struct GyroT<144> { static constexpr int K = 8, S = 32, BB = 34; };
template <> struct GyroT<145> { static constexpr int K = 6, S = 32, BB = 26; };
template <> struct GyroT<146> { static constexpr int K = 7, S = 32, BB = 30; };
template <> struct GyroT<147> { static constexpr int K = 5, S = 64, BB = 42; };
template <> struct GyroT<148> { static constexpr int K = 6, S = 64, BB = 50; };
template <> struct GyroT<149> { static constexpr int K = 7, S = 64, BB = 58; };
template <> struct GyroT<150> { static constexpr int K = 5, S = 32, BB = 22; };
template <> struct GyroT<151> { static constexpr int K = 4, S = 32, BB = 18; };
template <int ID> constexpr int gyro_nw() { return (GyroT<ID>::BB - 2) / 4; }

// Scale and stream words of a block that starts at an even byte offset inside the words d[]
// (d[0] holds the block's first bytes when odd_half is false, else they start at byte 2 of
// d[0]); d holds NW + 1 words.
template <int ID>
__device__ __forceinline__ void gyro_unpack(const uint32_t *d, bool odd_half, float &scale,
                                            uint32_t (&w)[gyro_nw<ID>()]) {
    if (!odd_half) {
        scale = gd_half(d[0] & 0xffffu);
#pragma unroll
        for (int j = 0; j < gyro_nw<ID>(); ++j) w[j] = __builtin_amdgcn_alignbyte(d[j + 1], d[j], 2);
    } else {
        scale = gd_half(d[0] >> 16);
#pragma unroll
        for (int j = 0; j < gyro_nw<ID>(); ++j) w[j] = d[j + 1];
    }
}

// 15-bit state of step t (a constant after unrolling) of a k-bit type (src/gyro.zig:107-117):
// the 16-bit window at stream bit (S - 1 - t) K of the circular little-endian stream, masked to
// 15 bits as the hash reads it.
template <int ID>
__device__ __forceinline__ uint32_t gyro_kstate(const uint32_t (&w)[gyro_nw<ID>()], int t) {
    constexpr int NW = gyro_nw<ID>();
    const int off = (GyroT<ID>::S - 1 - t) * GyroT<ID>::K;
    const int i = off >> 5, i1 = (i + 1) % NW;
    return __builtin_amdgcn_alignbit(w[i1], w[i], (uint32_t)(off & 31)) & 0x7fffu;
}

// Unscaled dot of one block with its 128 fp32 activations x (an LDS, register or uniform
// pointer): fp32(codebook value) x fp32 activation, accumulated in fp32 (v_fma_mix_f32).
// 32-step types give two codebook pairs per step (weights 4t .. 4t+3), 64-step types one
// (weights 2t, 2t+1).
template <int ID, typename XP>
__device__ __forceinline__ float gyro_block_dot(const uint32_t (&w)[gyro_nw<ID>()], const uint32_t *book, XP x) {
    if constexpr (ID == 144) {
        return tq2_block_dot(w, book, x);
    } else {
        float acc0 = 0.f, acc1 = 0.f;
        if constexpr (GyroT<ID>::S == 32) {
#pragma unroll
            for (int t = 0; t < 32; ++t) {
                uint32_t a0, a1;
                cb_addr(gyro_kstate<ID>(w, t), a0, a1);
                const uint32_t p0 = lds_word(book, a0), p1 = lds_word(book, a1);
                acc0 = fma_hi(p0, x[4 * t + 1], fma_lo(p0, x[4 * t], acc0));
                acc1 = fma_hi(p1, x[4 * t + 3], fma_lo(p1, x[4 * t + 2], acc1));
            }
        } else {
#pragma unroll
            for (int t = 0; t < 64; t += 2) {
                const uint32_t p0 = lds_word(book, cb_addr0(gyro_kstate<ID>(w, t)));
                const uint32_t p1 = lds_word(book, cb_addr0(gyro_kstate<ID>(w, t + 1)));
                acc0 = fma_hi(p0, x[2 * t + 1], fma_lo(p0, x[2 * t], acc0));
                acc1 = fma_hi(p1, x[2 * t + 3], fma_lo(p1, x[2 * t + 2], acc1));
            }
        }
        return acc0 + acc1;
    }
}

// Half hf of a block against its 64 fp32 activations x[0 .. 63]: trellis steps hf S / 2 ..
// hf S / 2 + S / 2 - 1 (hf per lane). For hf = 1 the circular stream is first rotated left by
// the S K / 2 bits of a half, which puts the states of those steps where steps 0 .. S / 2 - 1
// read theirs; the sums then run as in gyro_block_dot.
template <int ID, typename XP>
__device__ __forceinline__ float gyro_half_dot(const uint32_t (&w)[gyro_nw<ID>()], uint32_t hf, const uint32_t *book,
                                               XP x) {
    if constexpr (ID == 144) {
        return tq2_half_dot(w, hf, book, x);
    } else {
        constexpr int NW = gyro_nw<ID>(), S = GyroT<ID>::S, HB = S / 2 * GyroT<ID>::K, q = HB / 32, r = HB % 32;
        uint32_t v[NW];
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            const uint32_t hi = w[(i - q + NW) % NW], lo = w[(i - q - 1 + 2 * NW) % NW];
            const uint32_t rot = r ? __builtin_amdgcn_alignbit(hi, lo, 32 - r) : hi;
            v[i] = hf ? rot : w[i];
        }
        float acc0 = 0.f, acc1 = 0.f;
        if constexpr (S == 32) {
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                uint32_t a0, a1;
                cb_addr(gyro_kstate<ID>(v, t), a0, a1);
                const uint32_t p0 = lds_word(book, a0), p1 = lds_word(book, a1);
                acc0 = fma_hi(p0, x[4 * t + 1], fma_lo(p0, x[4 * t], acc0));
                acc1 = fma_hi(p1, x[4 * t + 3], fma_lo(p1, x[4 * t + 2], acc1));
            }
        } else {
#pragma unroll
            for (int t = 0; t < 32; t += 2) {
                const uint32_t p0 = lds_word(book, cb_addr0(gyro_kstate<ID>(v, t)));
                const uint32_t p1 = lds_word(book, cb_addr0(gyro_kstate<ID>(v, t + 1)));
                acc0 = fma_hi(p0, x[2 * t + 1], fma_lo(p0, x[2 * t], acc0));
                acc1 = fma_hi(p1, x[2 * t + 3], fma_lo(p1, x[2 * t + 2], acc1));
            }
        }
        return acc0 + acc1;
    }
}

// Expands X(ID) for the (uniform) Gyro type id; unknown ids do nothing.
#define GYRO_TYPE_SWITCH(id, X)       \
    switch (id) {                     \
        case 144: X(144); break;      \
        case 145: X(145); break;      \
        case 146: X(146); break;      \
        case 147: X(147); break;      \
        case 148: X(148); break;      \
        case 149: X(149); break;      \
        case 150: X(150); break;      \
        case 151: X(151); break;      \
        default: break;               \
    }

// Block bytes of a Gyro type id (the host admits only the eight types; other ids read as 34).
__device__ __forceinline__ uint32_t block_bytes_of_type(uint32_t id) {
    GyroType t;
    return gd_type(id, t) ? t.block_bytes : 34u;
}
