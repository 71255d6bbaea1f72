// moe_decode_down_x built for 2 to 8 tokens: 16 output rows per group, one block per lane (see
// moe_decode_down_x.hip).
#define DX_PIPELINE moe_decode_down_xb
#define DN_ROWS 16
#include "moe_decode_down_x.hip"
