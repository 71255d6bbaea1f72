// moe_decode_down_g for layers whose n_used F / 128 rotated input blocks exceed 64 (up to 128:
// top-16 at F 1024), at 67.6 KB of LDS per group.
#define DG_MAX_ABLK 128
#define DG_PIPELINE moe_decode_down_gl
#include "moe_decode_down_g.hip"
