// Per slot: a = silu(gate) * up, times the down-projection signs, then the normalised
// 128-block Walsh-Hadamard transform: the input of the down projection. Replaces moe_act of
// shaders/engine/moe.hlsl:213-254 (src/engine.zig:603-607 on the CPU).
// Grid: x = slots; 128 threads (two waves, each transforming whole 128-blocks).
// Constants (ActC): 0 gu_uav 1 gu_off 2 out_uav 3 out_off 4 signs_srv 5 signs_off 6 ff 7 rotate.
// gate/up input layout: [slot][2][ff]; output [slot][ff].
#include "fwht.h"

GD_PIPELINE_NAMED(moe_act, 128) {
    const float *GU = gd_buf<const float>(a, a.c[0]);
    float *O = gd_buf<float>(a, a.c[2]);
    const float *S = gd_buf<const float>(a, a.c[4]);
    const uint32_t ff = a.c[6], rotate = a.c[7], slot = blockIdx.x;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t base = a.c[1] + slot * ff * 2u;
    if (!rotate) {
        for (uint32_t i = threadIdx.x; i < ff; i += 128u)
            O[a.c[3] + slot * ff + i] = gd_silu_accurate(GU[base + i]) * GU[base + ff + i];
        return;
    }
    for (uint32_t blk = wave; blk * 128u < ff; blk += 2u) {
        const uint32_t i = blk * 128u + 2u * lane;
        float x0 = gd_silu_accurate(GU[base + i]) * GU[base + ff + i] * S[a.c[5] + i];
        float x1 = gd_silu_accurate(GU[base + i + 1u]) * GU[base + ff + i + 1u] * S[a.c[5] + i + 1u];
        gd_fwht128_wave(x0, x1);
        O[a.c[3] + slot * ff + i] = x0 * GD_INV_SQRT128;
        O[a.c[3] + slot * ff + i + 1u] = x1 * GD_INV_SQRT128;
    }
}
