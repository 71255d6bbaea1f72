// Prefill path, steps 4 and 5 in one launch: the grouped gate/up and down GEMMs of the sorted
// slots (src/engine.zig:567-633), TQ2_T experts, as a persistent kernel over two work queues.
//
// The units are those of moe_prefill_gu and moe_prefill_down (gemm_units.h): gate/up unit
// (tile, fb) for fb < F / 128, down unit (tile, eb) for eb < E / 256. Every unit decodes its
// 256 weight rows once whatever the tile's row count, so all gate/up units cost about the same,
// and a down unit about a quarter of that. With one launch per kind, the tile count rarely fills
// the last round of two groups per CU: the last gate/up groups ran nearly alone, and the down
// kernel could not start before them. Here two groups per CU take all gate/up units (tile by
// tile, the sort's longest-first order; group g takes unit g first, the later ones come from the
// queue) and then down units, so the down units fill the CUs the gate/up tail leaves idle.
//
// A down unit needs its tile's act16 rows from all F / 128 gate/up units of the tile. A gate/up
// unit writes its rows with device-scope stores, waits for them, and adds 1 to its tile's
// counter; the unit that completes the tile appends it to the ready list (device-scope store of
// tile + 1). Down units go through the ready list in order: unit v waits (device-scope loads,
// bounded by the spin limit) until slot v / neb is filled, so tiles are taken in the order they
// finished and a down unit waits only while no further tile is ready. The rows are never read
// before they are written in a launch, so no cache holds an older copy. A wait that reaches the
// limit sets the give-up word (sched[1]) and skips its unit; the caller must then discard the
// call's outputs. Gate/up units never wait, and every tile is completed by units taken before
// any down unit, so every wait ends; every group leaves once both queues are empty.
//
// Grid: any number of groups (two per CU fill the GPU); 512 threads, 80 KB of LDS, at most 128
// VGPRs. Requires the sort to have zeroed sched words 0 .. 63 + 2 tiles in the same stream (its
// constant 8), TQ2_T experts, E % 256 == 0 and F % 128 == 0 with F >= 256.
// Constants: 0 meta_uav 1 order_uav 2 order_off 3 xh16_uav 4 xh16_off (words) 5 base_lo
// 6 base_hi 7 slot_stride 8 proj_bytes 9 codebook_srv 10 signs_srv (0xffffffff: none) 11 signs_off
// 12 act16_uav 13 act16_off (words) 14 E 15 F 16 n_used 17 range flag (as moe_prefill_gu)
// 18 down32_uav 19 down32_off (words) 20 sched_uav (u32: [0] gate/up queue (units from gridDim.x
// on), [1] give-up, [2] down queue, [3] ready count, [64 + t] tile t's finished gate/up units,
// [64 + tiles + s] ready slot s: tile + 1, 0 while empty) 21 spin limit (polls of a ready slot) 22 small-tile rows SR (read by
// moe_prefill_gemm_s only: 16 or 8, tiles of at most SR rows take the small units of
// gemm_small.h; 0: none).
#include "gemm_persistent.h"

GD_PIPELINE_NAMED_OCC(moe_prefill_gemm, 512, 4) { prefill_gemm_body<false>(a); }
