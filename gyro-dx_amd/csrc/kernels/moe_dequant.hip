// Dequantises rows of one expert projection with the decoders the fast paths run, so tests can
// compare them bit for bit with the strict decoder (src/gyro.zig:81-105), for every Gyro type:
//   mode 0: the decode path's block decoders (tq2_unpack and the TQ2_T state pairs of
//           tq2_block_dot; gyro_unpack and gyro_kstate of gyro_block_dot), fp32 scale x
//           codebook value;
//   mode 1: the prefill GEMMs' B-operand decoders (gg_gather for TQ2_T; gx_half_stream and
//           gx_gather_piece for the k-bit types), lane half h giving k = 16 s + 8 h .. + 7 of
//           K-step s, fp32 scale x codebook value;
//   mode 2: the B operand itself as the MFMA reads it, binary16(scale x codebook value) from
//           gg_scale, widened to fp32.
// A unit is one 128-weight block (mode 0) or one lane half of it (modes 1, 2); blocks start at
// any even byte offset, so rows of an odd block count exercise both parities.
// Constants: 0 xtab_srv 1 expert 2 proj (0 gate, 1 up, 2 down) 3 row0 4 rows 5 cols
// 6 codebook_srv 7 out_uav 8 out_off 9 mode.
#include "ggemm.h"

#define DQ_MAX_WORDS 16  // the widest block (58 bytes) from its 4-byte-aligned start, plus one word

template <int ID>
__device__ __forceinline__ void dq_decode_path(const uint32_t *d, bool odd, const uint32_t *book, float *out) {
    float sc;
    if constexpr (ID == 144) {
        uint32_t q[8];
        tq2_unpack(d, odd, sc, q);
        for (int i = 0; i < 8; ++i) {
            const uint32_t p01 = tq2_pair01(q[i], q[(i + 7) & 7]), p23 = tq2_pair23(q[i]);
            const uint32_t s[4] = {p01 & 0x7fffu, __builtin_amdgcn_ubfe(p01, 16, 15), p23 & 0x7fffu,
                                   __builtin_amdgcn_ubfe(p23, 16, 15)};
            for (int j = 0; j < 4; ++j) {
                uint32_t a0, a1;
                cb_addr(s[j], a0, a1);
                const uint32_t w0 = lds_word(book, a0), w1 = lds_word(book, a1);
                float *o = out + (i * 4 + j) * 4;
                o[0] = __fmul_rn(sc, gd_half(w0 & 0xffffu));
                o[1] = __fmul_rn(sc, gd_half(w0 >> 16));
                o[2] = __fmul_rn(sc, gd_half(w1 & 0xffffu));
                o[3] = __fmul_rn(sc, gd_half(w1 >> 16));
            }
        }
    } else {
        uint32_t w[gyro_nw<ID>()];
        gyro_unpack<ID>(d, odd, sc, w);
        if constexpr (GyroT<ID>::S == 32) {
            for (int t = 0; t < 32; ++t) {
                uint32_t a0, a1;
                cb_addr(gyro_kstate<ID>(w, t), a0, a1);
                const uint32_t p0 = lds_word(book, a0), p1 = lds_word(book, a1);
                out[4 * t] = __fmul_rn(sc, gd_half(p0 & 0xffffu));
                out[4 * t + 1] = __fmul_rn(sc, gd_half(p0 >> 16));
                out[4 * t + 2] = __fmul_rn(sc, gd_half(p1 & 0xffffu));
                out[4 * t + 3] = __fmul_rn(sc, gd_half(p1 >> 16));
            }
        } else {
            for (int t = 0; t < 64; ++t) {
                const uint32_t p = lds_word(book, cb_addr0(gyro_kstate<ID>(w, t)));
                out[2 * t] = __fmul_rn(sc, gd_half(p & 0xffffu));
                out[2 * t + 1] = __fmul_rn(sc, gd_half(p >> 16));
            }
        }
    }
}

// Lane half h of the prefill decoders: the weights k = 16 s + 8 h + e (e = 0..7) of K-steps
// s = 0..7 into out[k].
template <int ID>
__device__ __forceinline__ void dq_prefill_path(const uint32_t *d, bool odd, uint32_t h, bool b16, const uint32_t *book,
                                                float *out) {
    float sc;
    uint32_t raw[8][4];
    if constexpr (ID == 144) {
        uint32_t q[8];
        tq2_unpack(d, odd, sc, q);
        const uint32_t sel = gg_sel(h);
        for (int s = 0; s < 8; ++s) gg_gather(q, s, sel, book, raw[s]);
    } else {
        uint32_t w[gyro_nw<ID>()];
        gyro_unpack<ID>(d, odd, sc, w);
        gx_half_stream<ID>(w, h);
        for (int s = 0; s < 8; ++s) {
            gx_gather_piece<ID>(w, s, 0, book, raw[s]);
            gx_gather_piece<ID>(w, s, 1, book, raw[s]);
        }
    }
    const half2_t sc2 = {(_Float16)sc, (_Float16)sc};
    for (int s = 0; s < 8; ++s) {
        if (b16) {
            const f16x8 bv = gg_scale(raw[s], sc2);
            for (int e = 0; e < 8; ++e) out[16 * s + 8 * h + e] = (float)bv[e];
        } else {
            for (int j = 0; j < 4; ++j) {
                out[16 * s + 8 * h + 2 * j] = __fmul_rn(sc, gd_half(raw[s][j] & 0xffffu));
                out[16 * s + 8 * h + 2 * j + 1] = __fmul_rn(sc, gd_half(raw[s][j] >> 16));
            }
        }
    }
}

GD_PIPELINE_NAMED(moe_dequant, 256) {
    __shared__ uint32_t book[2048];
    const uint32_t *cb = gd_buf<const uint32_t>(a, a.c[6]);
    for (uint32_t i = threadIdx.x; i < 2048u; i += 256u) book[i] = cb[i];
    __syncthreads();
    const uint32_t cols = a.c[5], nb = cols / 128u, rows = a.c[4], mode = a.c[9];
    const uint32_t halves = mode ? 2u : 1u;
    const uint32_t unit = blockIdx.x * 256u + threadIdx.x;
    if (unit >= rows * nb * halves) return;
    const uint32_t h = unit % halves, rb = unit / halves, r = rb / nb, b = rb - r * nb;
    const ExpertDesc &desc = gd_buf<const ExpertDesc>(a, a.c[0])[a.c[1]];
    const uint32_t proj = a.c[2];
    const uint8_t *base = reinterpret_cast<const uint8_t *>(proj == 0 ? desc.gate : proj == 1 ? desc.up : desc.down);
    const uint32_t type = (desc.types >> (8u * proj)) & 0xffu, bb = block_bytes_of_type(type);
    const uint64_t off = (uint64_t)(a.c[3] + r) * nb * bb + (uint64_t)b * bb;  // even
    const uint32_t *w = reinterpret_cast<const uint32_t *>(base + (off & ~uint64_t(3)));
    const uint32_t nw = (bb + 2u + 3u) / 4u;  // words from the aligned start through the block's end
    uint32_t d[DQ_MAX_WORDS];
    for (uint32_t j = 0; j < DQ_MAX_WORDS; ++j) d[j] = j < nw ? w[j] : 0u;
    const bool odd = (off & 2u) != 0u;
    float *out = gd_buf<float>(a, a.c[7]) + a.c[8] + (size_t)r * cols + b * 128u;
#define DQ_CASE(ID)                                                    \
    if (mode == 0u) dq_decode_path<ID>(d, odd, book, out);             \
    else dq_prefill_path<ID>(d, odd, h, mode == 2u, book, out);
    GYRO_TYPE_SWITCH(type, DQ_CASE)
#undef DQ_CASE
}
