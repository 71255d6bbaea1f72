// 128-point Walsh-Hadamard transform held by one wave64, two values per lane: lane l holds
// elements 2l and 2l+1. Stage w pairs element i with i ^ w; the lower element becomes
// lower + upper and the upper becomes lower - upper, the butterfly order of
// src/gyro.zig:152-172, so results match the CPU bit for bit before the final scaling.
#pragma once
#include "gd_kernel.h"

__device__ __forceinline__ void gd_fwht128_wave(float &x0, float &x1) {
    const uint32_t lane = threadIdx.x & 63u;
    {
        const float a = x0, b = x1;
        x0 = a + b;
        x1 = a - b;
    }
#pragma unroll
    for (uint32_t half = 1; half < 64; half <<= 1) {
        const float p0 = __shfl_xor(x0, (int)half, 64);
        const float p1 = __shfl_xor(x1, (int)half, 64);
        if (lane & half) {
            x0 = p0 - x0;
            x1 = p1 - x1;
        } else {
            x0 = x0 + p0;
            x1 = x1 + p1;
        }
    }
}
