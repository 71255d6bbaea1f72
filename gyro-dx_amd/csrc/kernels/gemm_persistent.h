// The persistent grouped-GEMM kernels of the prefill path: the queue and hand-off shared by the
// TQ2_T kernels moe_prefill_gemm (the staged units only) and moe_prefill_gemm_s (also the
// small-tile units of gemm_small.h), and by the type-generic moe_prefill_gemm_x (the units of
// gemm_units_x.h). The queue, hand-off and constants are described in moe_prefill_gemm.hip.
#pragma once
#include "gemm_small.h"
#include "gemm_units_x.h"

// Tile counters at kSchedCount, the ready list (tile + 1 per finished tile, 0: not yet) after them.
constexpr uint32_t kSchedCount = 64u;

// Both queues of one launch. nfb gate/up units and neb down units per tile; sched: the queue
// words, give-up word, tile counters and ready list; limit: the polls of a ready slot before a
// down unit gives up. gu(td, fb) and dn(td, eb) run one unit of tile descriptor td; the group's
// LDS is free when they start (they are inlined: as calls, their captures would pass through
// scratch memory). unit_word: one LDS word that is free between units.
template <class GU, class DN>
__device__ __forceinline__ void prefill_gemm_queue(const uint32_t *meta, uint32_t *sched_ptr, uint32_t nfb,
                                                   uint32_t neb, uint32_t limit, uint32_t *unit_word, GU &&gu,
                                                   DN &&dn) {
    const uint32_t tid = threadIdx.x;
    const uint32_t tiles = __builtin_amdgcn_readfirstlane(meta[1023]);
    const uint32_t n_gu = tiles * nfb;
    // Global (not flat) accesses: a flat atomic still in flight would make the compiler wait for
    // all LDS traffic at every counted LDS wait of the next unit's K loop.
    __attribute__((address_space(1))) uint32_t *sched = (__attribute__((address_space(1))) uint32_t *)(uintptr_t)sched_ptr;
    const uint4 *tile_list = reinterpret_cast<const uint4 *>(meta + 1024u);
    __attribute__((address_space(1))) uint32_t *ready = sched + kSchedCount + tiles;

    // Queue numbers go through one LDS word.
    auto take = [&](uint32_t q) {
        __syncthreads();  // the previous unit is done with the LDS
        if (tid == 0) *unit_word = __hip_atomic_fetch_add(sched + q, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        const uint32_t u = __builtin_amdgcn_readfirstlane(*unit_word);
        __syncthreads();  // every wave has read the word
        return u;
    };
    // Gate/up units. The first round is static (group g takes unit g), the rest come from queue
    // word 0 (unit = groups + the word's count): a device-scope atomic on one word that every
    // group of the GPU polls costs about 2 us a take under that contention, and a first round
    // taken without it measured the launch 6-8% faster. The unit that completes a tile appends
    // the tile to the ready list.
    bool first = true;
    for (;;) {
        uint32_t u;
        if (first) {
            u = blockIdx.x;
            first = false;
        } else {
            u = gridDim.x + take(0);
        }
        if (u >= n_gu) break;  // uniform
        const uint32_t tile = u / nfb, fb = u - tile * nfb;
        gu(tile_list[tile], fb);
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
        dn(tile_list[r - 1u], eb);
    }
}

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

// The TQ2_T kernel body; SMALL adds the small-tile units (tiles of at most constant-22 rows take
// gs_gu_unit / gs_dn_unit). The instantiation without them keeps the other units' register
// allocation: the branches alone cost them 3-5% (more spills at unit boundaries).
template <bool SMALL>
__device__ __forceinline__ void prefill_gemm_body(const GdArgs &a) {
    __shared__ GhLds sm;
    const uint32_t *meta = gd_buf<const uint32_t>(a, a.c[0]);
    const uint32_t E = a.c[14], F = a.c[15];
    prefill_gemm_queue(
        meta, gd_buf<uint32_t>(a, a.c[20]), F / 128u, E / 256u, a.c[21], reinterpret_cast<uint32_t *>(&sm.a[2][0]),
        [&](uint4 td, uint32_t fb) __attribute__((always_inline)) {
            if constexpr (SMALL) {
                const uint32_t trows = __builtin_amdgcn_readfirstlane(td.z), small = a.c[22];
                if (small == 16u && trows <= 16u) gs_gu_unit<16, true>(sm, gemm_gu_args(a), td, fb);
                else if (small == 8u && trows <= 8u) gs_gu_unit<8, true>(sm, gemm_gu_args(a), td, fb);
                else gu_unit<true>(sm, gemm_gu_args(a), td, fb);
            } else {
                gu_unit<true>(sm, gemm_gu_args(a), td, fb);
            }
        },
        [&](uint4 td, uint32_t eb) __attribute__((always_inline)) {
            if constexpr (SMALL) {
                const uint32_t trows = __builtin_amdgcn_readfirstlane(td.z), small = a.c[22];
                if (small == 16u && trows <= 16u) gs_dn_unit<16>(sm, gemm_dn_args(a), td, eb);
                else if (small == 8u && trows <= 8u) gs_dn_unit<8>(sm, gemm_dn_args(a), td, eb);
                else dn_unit(sm, gemm_dn_args(a), td, eb);
            } else {
                dn_unit(sm, gemm_dn_args(a), td, eb);
            }
        });
}

// The type-generic kernel body (moe_prefill_gemm_x's constants).
__device__ __forceinline__ void prefill_gemm_x_body(const GdArgs &a) {
    __shared__ GxLds sm;
    const uint32_t *meta = gd_buf<const uint32_t>(a, a.c[0]);
    const uint32_t E = a.c[11], F = a.c[12];
    prefill_gemm_queue(
        meta, gd_buf<uint32_t>(a, a.c[17]), F / 128u, E / 256u, a.c[18], reinterpret_cast<uint32_t *>(&sm.a[2][0]),
        [&](uint4 td, uint32_t fb) __attribute__((always_inline)) {
            GuxArgs p;
            p.order = gd_buf<const uint32_t>(a, a.c[1]) + a.c[2];
            p.xh16 = gd_buf<const uint32_t>(a, a.c[3]) + a.c[4];
            p.xtab = gd_buf<const ExpertDesc>(a, a.c[5]);
            p.codebook = gd_buf<const uint4>(a, a.c[6]);
            p.signs = a.c[7] != 0xffffffffu ? gd_buf<const float>(a, a.c[7]) + a.c[8] : nullptr;
            p.act16 = gd_buf<uint32_t>(a, a.c[9]) + a.c[10];
            p.flag = a.c[14] ? const_cast<uint32_t *>(meta) + 1022u : nullptr;
            p.E = E;
            p.F = F;
            p.U = a.c[13];
            gux_unit<true>(sm, p, td, fb);
        },
        [&](uint4 td, uint32_t eb) __attribute__((always_inline)) {
            DnxArgs p;
            p.order = gd_buf<const uint32_t>(a, a.c[1]) + a.c[2];
            p.act16 = gd_buf<const uint32_t>(a, a.c[9]) + a.c[10];
            p.xtab = gd_buf<const ExpertDesc>(a, a.c[5]);
            p.codebook = gd_buf<const uint4>(a, a.c[6]);
            p.down32 = gd_buf<float>(a, a.c[15]) + a.c[16];
            p.E = E;
            p.F = F;
            dnx_unit(sm, p, td, eb);
        });
}
