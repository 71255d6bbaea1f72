// moe_decode_gu for batches of 2 to 8 tokens: the same routing, loads and products, with each
// lane's 128 activations read from LDS into registers one half block at a time
// (tq2_block_dot_halves), so the kernel needs 64 VGPRs and up to four groups share a compute
// unit (256 groups per token). Constants, grid and requirements: those of moe_decode_gu.
#define GU_PIPELINE moe_decode_gu_b
#define GU_HALVES 1
#include "moe_decode_gu.hip"
