// moe_decode_down_g for layers of any Gyro types (src/engine.zig:603-641 with the types of
// src/gyro.zig:32-41): each expert's down rows are found through the layer's expert table (its
// down pointer and down type), the table staged in LDS while the ids load. A block is loaded as
// the widest type's 15 words from its first byte rounded down to a word, and an item decodes
// its half of both rows' blocks in its expert's type (gyro_half_dot).
// Constants: as moe_decode_down_g, with 6-9 unused and 24 xtab_srv. Requires n_expert <= 256,
// n_used F / 128 <= 128 and the host checks of moe_decode_down_g; 67.6 KB of rotated inputs.
#define DG_MAX_ABLK 128
#define DG_GENERIC 1
#define DG_PIPELINE moe_decode_down_xg
#include "moe_decode_down_g.hip"
