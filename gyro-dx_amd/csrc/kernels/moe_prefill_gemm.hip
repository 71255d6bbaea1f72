// Prefill path, steps 4 and 5 in one launch: the grouped gate/up and down GEMMs of the sorted
// slots (src/engine.zig:567-633), TQ2_T experts, as a persistent kernel over two work queues.
//
// The units are those of moe_prefill_gu and moe_prefill_down (gemm_units.h): gate/up unit
// (tile, fb) for fb < F / 128, down unit (tile, eb) for eb < E / 256. Every unit decodes its
// 256 weight rows once whatever the tile's row count, so all gate/up units cost about the same,
// and a down unit about a quarter of that. With one launch per kind, the tile count rarely fills
// the last round of two groups per CU: the last gate/up groups ran nearly alone, and the down
// kernel could not start before them. Here two groups per CU take all gate/up units (tile by
// tile, the sort's longest-first order) and then down units, so the down units fill the CUs the
// gate/up tail leaves idle.
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
// 18 down32_uav 19 down32_off (words) 20 sched_uav (u32: [0] gate/up queue, [1] give-up, [2] down
// queue, [3] ready count, [64 + t] tile t's finished gate/up units, [64 + tiles + s] ready slot s:
// tile + 1, 0 while empty) 21 spin limit (polls of a ready slot) 22 small-tile rows SR (16 or 8:
// tiles of at most SR rows take the small units of gemm_small.h; 0: none; the host passes
// gs_rows_for(E) when E and F are multiples of 512).
#include "gemm_small.h"

__device__ __forceinline__ GuUnitArgs gemm_gu_args(const GdArgs &a) {
    const uint32_t *meta = gd_buf<const uint32_t>(a, a.c[0]);
    GuUnitArgs g;
    g.order = gd_buf<const uint32_t>(a, a.c[1]) + a.c[2];
    g.xh16 = gd_buf<const uint32_t>(a, a.c[3]) + a.c[4];
    g.base = ((uint64_t)a.c[6] << 32) | a.c[5];
    g.slot_stride = a.c[7];
    g.proj_bytes = a.c[8];
    g.codebook = gd_buf<const uint4>(a, a.c[9]);
    g.signs = a.c[10] != 0xffffffffu ? gd_buf<const uint32_t>(a, a.c[10]) + a.c[11] : nullptr;
    g.act16 = gd_buf<uint32_t>(a, a.c[12]) + a.c[13];
    g.flag = a.c[17] ? const_cast<uint32_t *>(meta) + 1022u : nullptr;
    g.E = a.c[14];
    g.F = a.c[15];
    g.U = a.c[16];
    return g;
}
__device__ __forceinline__ DnUnitArgs gemm_dn_args(const GdArgs &a) {
    DnUnitArgs d;
    d.order = gd_buf<const uint32_t>(a, a.c[1]) + a.c[2];
    d.act16 = gd_buf<const uint32_t>(a, a.c[12]) + a.c[13];
    d.base = ((uint64_t)a.c[6] << 32) | a.c[5];
    d.slot_stride = a.c[7];
    d.down_off = 2u * a.c[8];
    d.codebook = gd_buf<const uint4>(a, a.c[9]);
    d.down32 = gd_buf<float>(a, a.c[18]) + a.c[19];
    d.E = a.c[14];
    d.F = a.c[15];
    return d;
}

GD_PIPELINE_NAMED_OCC(moe_prefill_gemm, 512, 4) {
    __shared__ GhLds sm;
    const uint32_t tid = threadIdx.x;
    const uint32_t *meta = gd_buf<const uint32_t>(a, a.c[0]);
    const uint32_t tiles = __builtin_amdgcn_readfirstlane(meta[1023]);
    const uint32_t E = a.c[14], F = a.c[15], nfb = F / 128u, neb = E / 256u;
    const uint32_t n_gu = tiles * nfb, n_units = n_gu + tiles * neb, limit = a.c[21], small = a.c[22];
    // Global (not flat) accesses: a flat atomic still in flight would make the compiler wait for
    // all LDS traffic at every counted LDS wait of the next unit's K loop.
    __attribute__((address_space(1))) uint32_t *sched =
        (__attribute__((address_space(1))) uint32_t *)(uintptr_t)gd_buf<uint32_t>(a, a.c[20]);
    const uint4 *tile_list = reinterpret_cast<const uint4 *>(meta + 1024u);
    // Tile counters at kSchedCount, the ready list (tile + 1 per finished tile, 0: not yet) after them.
    constexpr uint32_t kSchedCount = 64u;
    __attribute__((address_space(1))) uint32_t *ready = sched + kSchedCount + tiles;

    // Queue numbers go through one LDS word; the LDS is free between units.
    uint32_t *unit_word = reinterpret_cast<uint32_t *>(&sm.a[2][0]);
    auto take = [&](uint32_t q) {
        __syncthreads();  // the previous unit is done with the LDS
        if (tid == 0) *unit_word = __hip_atomic_fetch_add(sched + q, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        const uint32_t u = __builtin_amdgcn_readfirstlane(*unit_word);
        __syncthreads();  // every wave has read the word
        return u;
    };
    // Gate/up units (queue word 0). The unit that completes a tile appends the tile to the
    // ready list.
    for (;;) {
        const uint32_t u = take(0);
        if (u >= n_gu) break;  // uniform
        const uint32_t tile = u / nfb, fb = u - tile * nfb;
        const uint4 td = tile_list[tile];
        const uint32_t trows = __builtin_amdgcn_readfirstlane(td.z);
        if (small == 16u && trows <= 16u) gs_gu_unit<16, true>(sm, gemm_gu_args(a), td, fb);
        else if (small == 8u && trows <= 8u) gs_gu_unit<8, true>(sm, gemm_gu_args(a), td, fb);
        else gu_unit<true>(sm, gemm_gu_args(a), td, fb);
        __builtin_amdgcn_s_waitcnt(0);  // this thread's act16 stores acknowledged
        __syncthreads();
        if (tid == 0) {
            const uint32_t done =
                __hip_atomic_fetch_add(sched + kSchedCount + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (done + 1u == nfb) {  // every gate/up unit of the tile has stored its rows
                const uint32_t pos = __hip_atomic_fetch_add(sched + 3, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(ready + pos, tile + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    // Down units (queue word 2), tiles in the order they became ready: unit v takes column block
    // v % neb of the tile in ready slot v / neb.
    const uint32_t n_dn = tiles * neb;
    for (;;) {
        const uint32_t v = take(2);
        if (v >= n_dn) break;  // uniform
        const uint32_t slot = v / neb, eb = v - slot * neb;
        if (tid == 0) {
            uint32_t r = 0;
            for (uint32_t spins = 0;; ++spins) {
                r = __hip_atomic_load(ready + slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (r) break;
                if (spins >= limit) {
                    __hip_atomic_store(sched + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            *unit_word = r;
        }
        __syncthreads();
        const uint32_t r = __builtin_amdgcn_readfirstlane(*unit_word);
        __syncthreads();  // every wave has read the word
        if (r == 0u || r > tiles) continue;  // gave up (the call is marked invalid): skip the unit
        const uint4 td = tile_list[r - 1u];
        const uint32_t trows = __builtin_amdgcn_readfirstlane(td.z);
        if (small == 16u && trows <= 16u) gs_dn_unit<16>(sm, gemm_dn_args(a), td, eb);
        else if (small == 8u && trows <= 8u) gs_dn_unit<8>(sm, gemm_dn_args(a), td, eb);
        else dn_unit(sm, gemm_dn_args(a), td, eb);
    }
}
