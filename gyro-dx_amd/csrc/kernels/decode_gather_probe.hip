// Measurement pipeline beside the decode path (not on it): the codebook-gather ceiling of the
// decode kernels' block dot. Every lane decodes a register-resident TQ2_T block against 128 fp32
// activations held in registers with tq2_block_dot, the arithmetic of moe_decode_gu, `iters`
// times, the stream words changed on every pass so that no pass repeats another's gathers; the
// loop touches LDS (the codebook pairs) and registers only. Thread 0 of each group records the
// 100 MHz real-time counter (s_memrealtime) and the shader clock (s_memtime) before and after the
// loop, so the host gets the chip's decoded blocks per second and the clock they ran at.
// Grid: groups x 512 threads (one group per compute unit for moe_decode_gu's occupancy).
// Constants: 0 blocks_srv (512 x 9 words: lane l's block at word 9 l) 1 codebook_srv
// 2 x_srv (8 x 128 floats: lane l reads block l % 8, as the lanes of moe_decode_gu hold the
// activations of their own block) 3 out_uav (per group g: words 8 g .. 8 g + 3 = realtime start lo, hi,
// end lo, hi; 8 g + 4 .. + 7 = shader clocks start lo, hi, end lo, hi) 4 sums_uav (one float
// per thread of the grid) 5 iters.
#include "gyro_fast.h"

GD_PIPELINE_NAMED(decode_gather_probe, 512) {
    __shared__ uint4 book4[512];
    const uint32_t tid = threadIdx.x, g = blockIdx.x, iters = a.c[5];
    book4[tid] = gd_buf<const uint4>(a, a.c[1])[tid];
    gd_guint *bw = gd_global(gd_buf<const uint32_t>(a, a.c[0]) + 9u * tid);
    uint32_t d[9];
#pragma unroll
    for (int j = 0; j < 9; ++j) d[j] = bw[j];
    gd_gu32x4 *xv = gd_global4(gd_buf<const uint32_t>(a, a.c[2]) + 128u * (tid & 7u));
    float x[128];
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const gd_u32x4 v = xv[j];
        x[4 * j] = gd_bits_f32(v[0]);
        x[4 * j + 1] = gd_bits_f32(v[1]);
        x[4 * j + 2] = gd_bits_f32(v[2]);
        x[4 * j + 3] = gd_bits_f32(v[3]);
    }
    float sc;
    uint32_t q[8];
    tq2_unpack(d, (tid & 1u) != 0u, sc, q);
    __syncthreads();
    const uint64_t r0 = __builtin_amdgcn_s_memrealtime(), c0 = __builtin_amdgcn_s_memtime();
    float acc = 0.f;
    const uint32_t *book = reinterpret_cast<const uint32_t *>(book4);
    for (uint32_t it = 0; it < iters; ++it) {
        uint32_t qi[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) qi[j] = q[j] ^ (it * 0x9E3779B9u + (uint32_t)j * 0x85EBCA6Bu);
        acc += sc * tq2_block_dot(qi, book, x);
    }
    __syncthreads();
    const uint64_t r1 = __builtin_amdgcn_s_memrealtime(), c1 = __builtin_amdgcn_s_memtime();
    gd_buf<float>(a, a.c[4])[g * 512u + tid] = acc;
    if (tid == 0) {
        uint32_t *o = gd_buf<uint32_t>(a, a.c[3]) + 8u * g;
        o[0] = (uint32_t)r0;
        o[1] = (uint32_t)(r0 >> 32);
        o[2] = (uint32_t)r1;
        o[3] = (uint32_t)(r1 >> 32);
        o[4] = (uint32_t)c0;
        o[5] = (uint32_t)(c0 >> 32);
        o[6] = (uint32_t)c1;
        o[7] = (uint32_t)(c1 >> 32);
    }
}
