// GGUF Q8_0 rows (34-byte blocks: binary16 scale, 32 int8 quants) into the layout mv_q8 reads:
// per row the cols quants, then the cols / 32 scales (shaders/engine/mv.hlsl:94-119). One thread
// per block; block index = x + y * 65535 * 256 over rows * cols / 32 blocks.
// Constants as mv_q8: 0 src srv, 1 src offset (bytes), 2 rows, 3 cols, 8 dst uav, 9 dst offset
// (bytes), 14 dst row bytes (cols + cols / 16). Requires cols a multiple of 64 and both offsets
// multiples of 4.
#include "gd_kernel.h"

GD_PIPELINE_NAMED(q8_repack, 256) {
    const uint32_t rows = a.c[2], cols = a.c[3], row_bytes = a.c[14], bpr = cols / 32u;
    const uint32_t index = blockIdx.x * 256u + threadIdx.x + blockIdx.y * 65535u * 256u;
    if (index >= rows * bpr) return;
    const uint32_t row = index / bpr, b = index - row * bpr;
    // The source block starts on a 2-byte boundary: read it as 17 halfwords.
    const uint16_t *src = reinterpret_cast<const uint16_t *>(gd_buf<const uint8_t>(a, a.c[0]) + a.c[1] +
                                                             ((size_t)row * bpr + b) * 34u);
    uint32_t *dst = reinterpret_cast<uint32_t *>(gd_buf<uint8_t>(a, a.c[8]) + a.c[9] + (size_t)row * row_bytes);
    uint16_t h[17];
#pragma unroll
    for (int j = 0; j < 17; ++j) h[j] = src[j];
    uint4 *q = reinterpret_cast<uint4 *>(dst + b * 8u);
#pragma unroll
    for (int j = 0; j < 2; ++j)
        q[j] = make_uint4(h[1 + 8 * j] | (uint32_t)h[2 + 8 * j] << 16, h[3 + 8 * j] | (uint32_t)h[4 + 8 * j] << 16,
                          h[5 + 8 * j] | (uint32_t)h[6 + 8 * j] << 16, h[7 + 8 * j] | (uint32_t)h[8 + 8 * j] << 16);
    // Two scales share a word; the even block writes both (cols / 32 is even).
    if ((b & 1u) == 0u) dst[cols / 4u + b / 2u] = h[0] | (uint32_t)src[17] << 16;
}
