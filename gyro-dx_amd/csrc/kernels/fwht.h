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

// One DPP move of a float (bound_ctrl: lanes without a source read 0; every use below has a
// source).
template <int CTRL>
__device__ __forceinline__ float gd_dpp_f(float v) {
    return gd_bits_f32((uint32_t)__builtin_amdgcn_update_dpp(0, (int)gd_f32_bits(v), CTRL, 0xf, 0xf, true));
}

// The same 128-point transform held by an 8-lane group, 16 consecutive values per lane: lane
// l8 (0..7 within the group, the group at lanes 8g .. 8g + 7 of a wave) holds elements
// 16 l8 .. 16 l8 + 15 in v. Widths 1..8 pair register indices, widths 16, 32, 64 pair lanes
// l8 ^ 1, ^ 2, ^ 4 through DPP, in the same stage order as gd_fwht128_wave.
__device__ __forceinline__ void gd_fwht128_x16(float (&v)[16], uint32_t l8) {
#pragma unroll
    for (int w = 1; w < 16; w <<= 1)
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if (!(j & w)) {
                const float lo = v[j], hi = v[j + w];
                v[j] = lo + hi;
                v[j + w] = lo - hi;
            }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const float p1 = gd_dpp_f<0xB1>(v[j]);  // quad_perm [1,0,3,2]: lane ^ 1
        v[j] = (l8 & 1u) ? p1 - v[j] : v[j] + p1;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const float p2 = gd_dpp_f<0x4E>(v[j]);  // quad_perm [2,3,0,1]: lane ^ 2
        v[j] = (l8 & 2u) ? p2 - v[j] : v[j] + p2;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const float up4 = gd_dpp_f<0x104>(v[j]);  // row_shl:4, lane + 4
        const float dn4 = gd_dpp_f<0x114>(v[j]);  // row_shr:4, lane - 4
        v[j] = (l8 & 4u) ? dn4 - v[j] : v[j] + up4;
    }
}
