// moe_decode_gu_x for batches of 2 to 8 tokens: the same routing, loads and products, with the
// block dot reading each lane's 128 activations from LDS step by step, so the kernel needs far
// fewer VGPRs and several groups share a compute unit (256 groups per token). Constants, grid
// and requirements: those of moe_decode_gu_x.
#define GX_PIPELINE moe_decode_gu_xb
#define GX_STEPWISE 1
#include "moe_decode_gu_x.hip"
