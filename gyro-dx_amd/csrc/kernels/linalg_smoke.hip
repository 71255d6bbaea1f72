// One 16x16x16 fp16 product on the matrix cores with fp32 accumulation, checked exactly by
// gd_validate_linalg. Replaces shaders/linalg_smoke.hlsl:13-22 (a LinAlg wave matrix).
// Constants: table slots of A (16x16 fp16 row-major), B (16x16 fp16 row-major), C (16x16 fp32).
#include "gd_kernel.h"

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));

GD_PIPELINE_NAMED(linalg_smoke, 64) {
    const _Float16 *A = gd_buf<const _Float16>(a, a.c[0]);
    const _Float16 *B = gd_buf<const _Float16>(a, a.c[1]);
    float *Cm = gd_buf<float>(a, a.c[2]);
    const uint32_t lane = threadIdx.x;
    // v_mfma_f32_16x16x16_f16: lane l holds A[row = l % 16][k = 4 (l / 16) .. +4] and
    // B[k = 4 (l / 16) .. +4][col = l % 16]; the result D[row = 4 (l / 16) + i][col = l % 16].
    const uint32_t rc = lane & 15u, kq = (lane >> 4) * 4u;
    half4 av, bv;
    for (int i = 0; i < 4; ++i) {
        av[i] = A[rc * 16u + kq + i];
        bv[i] = B[(kq + i) * 16u + rc];
    }
    float4v acc = {0.f, 0.f, 0.f, 0.f};
    acc = __builtin_amdgcn_mfma_f32_16x16x16f16(av, bv, acc, 0, 0, 0);
    for (int i = 0; i < 4; ++i) Cm[(kq + i) * 16u + rc] = acc[i];
}
