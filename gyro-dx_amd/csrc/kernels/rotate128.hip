// y = H_128 (signs * x) per 128-value block, scaled by 1/sqrt(128). Replaces rotate128 of
// shaders/engine/moe.hlsl:256-283. Grid: x = blocks, y = tokens; 64 threads.
// Constants (RotC): 0 x_uav 1 x_off 2 y_uav 3 y_off 4 signs_srv 5 signs_off 6 n 7 stride.
#include "fwht.h"

GD_PIPELINE_NAMED(rotate128, 64) {
    const float *X = gd_buf<const float>(a, a.c[0]);
    float *Y = gd_buf<float>(a, a.c[2]);
    const float *S = gd_buf<const float>(a, a.c[4]);
    const uint32_t lane = threadIdx.x;
    const uint32_t base = blockIdx.y * a.c[7] + blockIdx.x * 128u + 2u * lane;
    const uint32_t sb = a.c[5] + blockIdx.x * 128u + 2u * lane;
    float x0 = X[a.c[1] + base] * S[sb];
    float x1 = X[a.c[1] + base + 1u] * S[sb + 1u];
    gd_fwht128_wave(x0, x1);
    Y[a.c[3] + base] = x0 * GD_INV_SQRT128;
    Y[a.c[3] + base + 1u] = x1 * GD_INV_SQRT128;
}
