// Prefill path, steps 4 and 5 in one launch with the small-tile units: moe_prefill_gemm (the
// persistent grouped gate/up and down GEMMs, src/engine.zig:567-633; its description, grid and
// constants) whose tiles of at most constant-22 rows take the units of gemm_small.h (the tile's
// activation rows resident in LDS, weight blocks streamed from HBM into registers, no barrier in
// the K loop). Outputs are bit-identical to moe_prefill_gemm's. The engine takes it when the
// average expert segment is at most 8 slots (n n_used <= 8 n_expert), where most tiles are small.
#include "gemm_persistent.h"

GD_PIPELINE_NAMED_OCC(moe_prefill_gemm_s, 512, 4) { prefill_gemm_body<true>(a); }
