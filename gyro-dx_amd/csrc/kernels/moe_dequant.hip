// Dequantises rows of one expert projection to fp32 with the decoder of the fast paths
// (packed-word trellis states, 24-bit hash addressing, LDS codebook), so tests can compare
// it bit for bit with the strict decoder (src/gyro.zig:81-105). One thread per 128-block.
// Constants: 0 xtab_srv 1 expert 2 proj (0 gate, 1 up, 2 down) 3 row0 4 rows 5 cols
// 6 codebook_srv 7 out_uav 8 out_off. TQ2_T only.
#include "gyro_fast.h"

GD_PIPELINE_NAMED(moe_dequant, 256) {
    __shared__ uint32_t book[2048];
    const uint32_t *cb = gd_buf<const uint32_t>(a, a.c[6]);
    for (uint32_t i = threadIdx.x; i < 2048u; i += 256u) book[i] = cb[i];
    __syncthreads();
    const uint32_t cols = a.c[5], nb = cols / 128u, rows = a.c[4];
    const uint32_t unit = blockIdx.x * 256u + threadIdx.x;
    if (unit >= rows * nb) return;
    const uint32_t r = unit / nb, b = unit - r * nb;
    const ExpertDesc &d = gd_buf<const ExpertDesc>(a, a.c[0])[a.c[1]];
    const uint8_t *proj = reinterpret_cast<const uint8_t *>(a.c[2] == 0 ? d.gate : a.c[2] == 1 ? d.up : d.down);
    const uint64_t off = (uint64_t)(a.c[3] + r) * nb * 34u + b * 34u;
    const uint32_t *w = reinterpret_cast<const uint32_t *>(proj + (off & ~uint64_t(3)));
    uint32_t dw[9];
    for (int j = 0; j < 9; ++j) dw[j] = w[j];
    float scale;
    uint32_t q[8];
    tq2_unpack(dw, (off & 2u) != 0u, scale, q);
    float *out = gd_buf<float>(a, a.c[7]) + a.c[8] + (size_t)r * cols + b * 128u;
    for (int i = 0; i < 8; ++i) {
        const uint32_t p01 = tq2_pair01(q[i], q[(i + 7) & 7]), p23 = tq2_pair23(q[i]);
        const uint32_t s[4] = {p01 & 0x7fffu, __builtin_amdgcn_ubfe(p01, 16, 15), p23 & 0x7fffu,
                               __builtin_amdgcn_ubfe(p23, 16, 15)};
        for (int j = 0; j < 4; ++j) {
            uint32_t a0, a1;
            cb_addr(s[j], a0, a1);
            const uint32_t w0 = lds_word(book, a0), w1 = lds_word(book, a1);
            float *o = out + (i * 4 + j) * 4;
            o[0] = __fmul_rn(scale, gd_half(w0 & 0xffffu));
            o[1] = __fmul_rn(scale, gd_half(w0 >> 16));
            o[2] = __fmul_rn(scale, gd_half(w1 & 0xffffu));
            o[3] = __fmul_rn(scale, gd_half(w1 >> 16));
        }
    }
}
