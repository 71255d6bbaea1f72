// Fused Gyro decode and matrix-vector product of the routed experts for layers whose experts
// and projections mix Gyro types (src/engine.zig:567-633 with dotRow per matrix,
// src/kernels.zig:201-210). The reference GPU path needs one type per layer
// (src/gpu_engine.zig:408-409); this kernel finds each selected expert's projection and its
// type in the layer's expert descriptor table instead of the uniform slot table.
// One (slot, projection) per grid row as moe_gyro: grid x = 32-row groups, y = slot
// (token * n_used + k), z = projection pass (proj 0: gate, z = 1 adds up; proj 2: down).
// Output: gate/up [slot][2][rows], down [slot][rows].
// Constants: 0 ids_uav 1 ids_off 2 xtab_srv (32-byte ExpertDesc per expert) 3 codebook_srv
// 4 x_uav 5 x_off 6 x_stride 7 y_uav 8 y_off 9 rows 10 cols 11 proj 12 n_used 13 x_per_slot
// 14 n_expert.
#include "gyro_fast.h"

#define GYRO_MAX_COLS 8192

GD_PIPELINE_NAMED(moe_gyro_x, 256) {
    __shared__ uint32_t book[2048];
    __shared__ float xs[GYRO_MAX_COLS];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t slot = blockIdx.y, proj = a.c[11] + blockIdx.z;
    const uint32_t rows = a.c[9], cols = a.c[10] < GYRO_MAX_COLS ? a.c[10] : GYRO_MAX_COLS;
    const uint32_t n_used = a.c[12], NE = a.c[14];
    const uint32_t *cb = gd_buf<const uint32_t>(a, a.c[3]);
    for (uint32_t i = tid; i < 2048u; i += 256u) book[i] = cb[i];
    const float *X = gd_buf<const float>(a, a.c[4]);
    const uint32_t xbase = a.c[5] + (a.c[13] ? slot : slot / n_used) * a.c[6];
    for (uint32_t i = tid; i < cols; i += 256u) xs[i] = X[xbase + i];
    __syncthreads();
    uint32_t e = gd_buf<const uint32_t>(a, a.c[0])[a.c[1] + slot];
    e = e < NE ? e : NE - 1u;
    const ExpertDesc d = gd_buf<const ExpertDesc>(a, a.c[2])[e];
    const uint32_t type_id = (d.types >> (8u * proj)) & 0xffu;
    GyroType t;
    if (!gd_type(type_id, t)) return;
    const uint8_t *W = reinterpret_cast<const uint8_t *>(proj == 0u ? d.gate : proj == 1u ? d.up : d.down);
    const uint32_t blocks = cols / 128u, row_bytes = blocks * t.block_bytes;
    const uint32_t pairs = t.steps == 64u ? 1u : 2u, per_step = 2u * pairs;
    const uint32_t step_shift = t.steps == 64u ? 6u : 5u;
    float *Y = gd_buf<float>(a, a.c[7]);
    const uint32_t out_base = a.c[11] == 2u ? a.c[8] + slot * rows : a.c[8] + (slot * 2u + blockIdx.z) * rows;
    for (uint32_t r = 0; r < 8u; ++r) {
        const uint32_t row = blockIdx.x * 32u + wave * 8u + r;
        if (row >= rows) break;
        const uint8_t *wr = W + (size_t)row * row_bytes;
        float acc = 0.f;
        for (uint32_t g = lane; g < (blocks << step_shift); g += 64u) {
            const uint32_t b = g >> step_shift, step = g & (t.steps - 1u);
            const uint8_t *blk = wr + b * t.block_bytes;
            const uint32_t h = gd_hash(gd_state(blk + 2, t, type_id, step));
            const float *xv = xs + b * 128u + step * per_step;
            const uint32_t pa = book[h >> 21];
            float part = gd_half(pa & 0xffffu) * xv[0] + gd_half(pa >> 16) * xv[1];
            if (pairs == 2u) {
                const uint32_t pb = book[(h >> 10) & 2047u];
                part += gd_half(pb & 0xffffu) * xv[2] + gd_half(pb >> 16) * xv[3];
            }
            acc += gd_half((uint32_t)blk[0] | ((uint32_t)blk[1] << 8)) * part;
        }
        acc = gd_wave_sum(acc);
        if (lane == 0) Y[out_base + row] = acc;
    }
}
