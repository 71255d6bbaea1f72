// out[t][i] = sum_k w[t][k] * down[t*U + k][i] + sigmoid(shared_gate[t]) * shared[t][i], summed
// in k order. Replaces moe_combine of shaders/engine/moe.hlsl:285-305.
// Grid: x = ceil(dim / 256), y = tokens; 256 threads.
// Constants (CombineC): 0 down_uav 1 down_off 2 w_uav 3 w_off 4 out_uav 5 out_off 6 n_used
// 7 dim 8 sh_uav 9 sh_off 10 shg_uav 11 shg_off.
#include "gd_kernel.h"

GD_PIPELINE_NAMED(moe_combine, 256) {
    const uint32_t t = blockIdx.y, i = blockIdx.x * 256u + threadIdx.x, U = a.c[6], dim = a.c[7];
    if (i >= dim) return;
    const float *D = gd_buf<const float>(a, a.c[0]);
    const float *W = gd_buf<const float>(a, a.c[2]);
    float acc = 0.f;
    for (uint32_t k = 0; k < U; ++k)
        acc += W[a.c[3] + t * U + k] * D[a.c[1] + (t * U + k) * dim + i];
    const float gate = gd_sigmoid_accurate(gd_buf<const float>(a, a.c[10])[a.c[11] + t]);
    acc += gate * gd_buf<const float>(a, a.c[8])[a.c[9] + t * dim + i];
    gd_buf<float>(a, a.c[4])[a.c[5] + t * dim + i] = acc;
}
