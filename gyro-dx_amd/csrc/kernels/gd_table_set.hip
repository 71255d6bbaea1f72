// Points entries of the context's table of base pointers at addresses carried in the dispatch's
// constants, so that work queued on a stream can name memory known only when it is queued (the
// caller's input and output of the MoE engine's no-allocation entry point) without a host copy
// into the table. Vector stores only; the next dispatch sees the entries.
// Constants: 0 count (at most 19), then for entry i: 1 + 3 i table index, 2 + 3 i address bits
// 0..31, 3 + 3 i address bits 32..63. Indices at or past the table's 65,536 entries are skipped.
#include "gd_kernel.h"

#define GD_TABLE_ENTRIES 65536u
#define GD_TABLE_SET_MAX 19u

GD_PIPELINE_NAMED(gd_table_set, 64) {
    const uint32_t i = threadIdx.x;
    if (i >= a.c[0] || i >= GD_TABLE_SET_MAX) return;
    const uint32_t index = a.c[1u + 3u * i];
    if (index >= GD_TABLE_ENTRIES) return;
    uint64_t *table = const_cast<uint64_t *>(a.table);
    table[index] = (uint64_t)a.c[2u + 3u * i] | ((uint64_t)a.c[3u + 3u * i] << 32);
}
