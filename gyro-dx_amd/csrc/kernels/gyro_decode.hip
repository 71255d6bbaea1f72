// Scalar Gyro conformance decoder: one thread per 128-value block, values written in the
// stored (rotated) basis. Replaces shaders/gyro_decode.hlsl:74-112 behind gd_validate_gyro.
//
// Constants: 0 input byte offset, 1 block count, 2 type id, 3 output byte offset,
// 4/5/6 table slots of input, codebook and output, 7 input bytes, 8 output bytes.
// Invalid ids or spans produce no writes (the host validates before dispatch).
#include "gd_kernel.h"

GD_PIPELINE_NAMED(gyro_decode, 64) {
    const uint32_t in_off = a.c[0], block_count = a.c[1], type_id = a.c[2], out_off = a.c[3];
    const uint8_t *input = gd_buf<const uint8_t>(a, a.c[4]);
    const uint16_t *book = gd_buf<const uint16_t>(a, a.c[5]);
    uint8_t *output = gd_buf<uint8_t>(a, a.c[6]);
    const uint32_t in_bytes = a.c[7], out_bytes = a.c[8];
    const uint32_t block = blockIdx.x * 64u + threadIdx.x;
    if (block >= block_count) return;
    GyroType t;
    if (!gd_type(type_id, t)) return;
    if (in_off > in_bytes || out_off > out_bytes || (out_off & 3u)) return;
    if (block_count > (in_bytes - in_off) / t.block_bytes) return;
    if (block_count > (out_bytes - out_off) / 512u) return;

    const uint8_t *src = input + in_off + (size_t)block * t.block_bytes;
    const float scale = gd_half_exact((uint32_t)src[0] | ((uint32_t)src[1] << 8));
    const uint8_t *stream = src + 2;
    float *dst = reinterpret_cast<float *>(output + out_off + (size_t)block * 512u);
    const uint32_t pairs = t.steps == 64u ? 1u : 2u;
    uint32_t o = 0;
    for (uint32_t step = 0; step < t.steps; ++step) {
        const uint32_t h = gd_hash(gd_state(stream, t, type_id, step));
        for (uint32_t p = 0; p < pairs; ++p) {
            const uint32_t index = p == 0 ? h >> 21 : (h >> 10) & 2047u;
            // One binary32 multiply per value (SPEC section 6).
            dst[o] = __fmul_rn(scale, gd_half_exact(book[index * 2u]));
            dst[o + 1] = __fmul_rn(scale, gd_half_exact(book[index * 2u + 1u]));
            o += 2;
        }
    }
}
