// Fused Gyro decode and matrix-vector product for the routed experts, one (slot, projection)
// per grid row. Replaces moe_gyro of shaders/engine/moe.hlsl:106-211 with its grid and
// constants: grid x = 32-row groups, y = slot (token * n_used + k), z = projection pass
// (g_proj 0: gate with z adding up as 1; g_proj 2: down). Output: gate/up [slot][2][rows],
// down [slot][rows]. Constants (GyroC): 0 table_uav 1 codebook_srv 2 x_uav 3 x_off 4 x_stride
// 5 y_uav 6 y_off 7 rows 8 cols 9 type 10 block_bytes 11 proj 12 n_used 13 x_per_slot.
// The slot table entry (6 words per slot) gives the buffer index and byte offset of each
// projection (moe_resolve). Works for every Gyro type; the per-type fast paths of the
// MI355X decode and prefill kernels are moe_decode_* and moe_ggemm_*.
#include "gd_kernel.h"

#define GYRO_MAX_COLS 8192

GD_PIPELINE_NAMED(moe_gyro, 256) {
    __shared__ uint32_t book[2048];
    __shared__ float xs[GYRO_MAX_COLS];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t slot = blockIdx.y, proj = a.c[11] + blockIdx.z;
    const uint32_t rows = a.c[7], cols = a.c[8] < GYRO_MAX_COLS ? a.c[8] : GYRO_MAX_COLS;
    const uint32_t type_id = a.c[9], n_used = a.c[12];
    const uint32_t *cb = gd_buf<const uint32_t>(a, a.c[1]);
    for (uint32_t i = tid; i < 2048u; i += 256u) book[i] = cb[i];
    const float *X = gd_buf<const float>(a, a.c[2]);
    const uint32_t xbase = a.c[3] + (a.c[13] ? slot : slot / n_used) * a.c[4];
    for (uint32_t i = tid; i < cols; i += 256u) xs[i] = X[xbase + i];
    __syncthreads();
    GyroType t;
    if (!gd_type(type_id, t)) return;
    const uint32_t *entry = gd_buf<const uint32_t>(a, a.c[0]) + slot * 6u + proj * 2u;
    const uint8_t *W = gd_buf<const uint8_t>(a, entry[0]) + entry[1];
    const uint32_t blocks = cols / 128u, row_bytes = blocks * t.block_bytes;
    const uint32_t pairs = t.steps == 64u ? 1u : 2u, per_step = 2u * pairs;
    const uint32_t step_shift = t.steps == 64u ? 6u : 5u;
    float *Y = gd_buf<float>(a, a.c[5]);
    const uint32_t out_base = a.c[11] == 2u ? a.c[6] + slot * rows : a.c[6] + (slot * 2u + blockIdx.z) * rows;
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
