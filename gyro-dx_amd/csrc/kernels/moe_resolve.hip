// Slot table for resident experts: each selected (layer * n_expert + expert) maps through the
// lookup to a slot, then to an arena and a byte offset. Entry (6 words): gate srv, gate
// offset, up srv, up offset, down srv, down offset. Replaces moe_resolve of
// shaders/engine/moe.hlsl:82-104. Grid: ceil(count / 64); 64 threads.
// Constants (ResolveC): 0 ids_uav 1 ids_off 2 count 3 table_uav 4 lookup_uav 5 lookup_off
// 6 per_arena 7 slot_stride 8 gate_bytes 9 n_arenas 10-11 pad 12-19 arena srv indices.
#include "gd_kernel.h"

GD_PIPELINE_NAMED(moe_resolve, 64) {
    const uint32_t k = blockIdx.x * 64u + threadIdx.x;
    if (k >= a.c[2]) return;
    const uint32_t e = gd_buf<const uint32_t>(a, a.c[0])[a.c[1] + k];
    const uint32_t slot = gd_buf<const uint32_t>(a, a.c[4])[a.c[5] + e];
    const uint32_t arena_i = slot / a.c[6];
    const uint32_t arena = a.c[12 + (arena_i < 8u ? arena_i : 7u)];
    const uint32_t o = (slot % a.c[6]) * a.c[7];
    uint32_t *T = gd_buf<uint32_t>(a, a.c[3]) + k * 6u;
    T[0] = arena; T[1] = o;
    T[2] = arena; T[3] = o + a.c[8];
    T[4] = arena; T[5] = o + 2u * a.c[8];
}
