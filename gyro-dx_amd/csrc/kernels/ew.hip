// Elementwise ops over rows with strides, replacing shaders/engine/ops.hlsl:95-128.
// y[r][i] = op(a[r][i], b[r][i]); op 0 silu(a)*b, 1 a*sigmoid(b), 2 a+b, 3 copy a,
// 4 a*sigmoid(b[r]) (row scalar), 5 bit-exact 32-bit copy.
// Constants (EwC): a_uav a_off a_stride b_uav b_off b_stride y_uav y_off y_stride n rows op.
#include "gd_kernel.h"

GD_PIPELINE_NAMED(ew, 256) {
    const uint32_t n = a.c[9], rows = a.c[10], op = a.c[11];
    const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    if (idx >= n * rows) return;
    const uint32_t r = idx / n, i = idx % n;
    const uint32_t *A = gd_buf<const uint32_t>(a, a.c[0]);
    uint32_t *Y = gd_buf<uint32_t>(a, a.c[6]);
    const uint32_t ai = a.c[1] + r * a.c[2] + i, yi = a.c[7] + r * a.c[8] + i;
    if (op == 5u) {
        Y[yi] = A[ai];
        return;
    }
    const float x = gd_bits_f32(A[ai]);
    float v;
    if (op == 3u) {
        v = x;
    } else {
        const uint32_t *Bm = gd_buf<const uint32_t>(a, a.c[3]);
        const float b = gd_bits_f32(op == 4u ? Bm[a.c[4] + r * a.c[5]] : Bm[a.c[4] + r * a.c[5] + i]);
        if (op == 0u) v = gd_silu_accurate(x) * b;
        else if (op == 1u || op == 4u) v = x * gd_sigmoid_accurate(b);
        else v = x + b;
    }
    Y[yi] = gd_f32_bits(v);
}
