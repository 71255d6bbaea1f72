// moe_decode_gu_g for layers of any Gyro types (src/engine.zig:567-606 with the types of
// src/gyro.zig:32-41): a run's experts are found through the layer's expert table (gate and up
// pointers, one type per projection), the whole table staged in LDS with the other independent
// loads. A block is loaded as the widest type's 15 words from its first byte rounded down to a
// word, and each projection's block is decoded in its own type (gyro_block_dot, fp32 activations).
// Constants: as moe_decode_gu_g, with 11-14 unused and 22 xtab_srv. Requires n_expert <= 256 and
// the host checks of moe_decode_gu_g.
#define GG_PIPELINE moe_decode_gu_xg
#define GG_GENERIC 1
#include "moe_decode_gu_g.hip"
