// Prefill path, steps 4 and 5 in one launch for layers whose experts and projections mix Gyro
// types (src/engine.zig:567-633 with the types of src/gyro.zig:32-41): the units of
// moe_prefill_gu_x and moe_prefill_down_x (gemm_units_x.h) from the two queues of
// moe_prefill_gemm, with its hand-off: gate/up units (tile, fb) for fb < F / 128 write their
// act16 rows with device-scope stores and count their tile's finished units; the unit that
// completes a tile appends it to the ready list; down units (tile, eb) for eb < E / 256 take the
// tiles in the order they became ready, with bounded waits that set the give-up word (the
// caller must then discard the call's outputs). Every wait ends: gate/up units never wait, and
// every tile is completed by units taken before any down unit.
//
// Grid: any number of groups (one per CU fills the GPU: 152.5 KB of LDS); 512 threads. Requires
// the sort to have zeroed sched words 0 .. 63 + 2 tiles in the same stream (its constant 8),
// Gyro types 144..151, E % 256 == 0 and F % 128 == 0 with F >= 256.
// Constants: 0 meta_uav 1 order_uav 2 order_off 3 xh16_uav 4 xh16_off (words) 5 xtab_srv
// 6 codebook_srv 7 signs_srv (0xffffffff: none) 8 signs_off 9 act16_uav 10 act16_off (words)
// 11 E 12 F 13 n_used 14 range flag (as moe_prefill_gu_x) 15 down32_uav 16 down32_off (words)
// 17 sched_uav (as moe_prefill_gemm) 18 spin limit (polls of a ready slot).
#include "gemm_persistent.h"

GD_PIPELINE_NAMED_OCC(moe_prefill_gemm_x, 512, 2) { prefill_gemm_x_body(a); }
