// Prefill path, step 3: counting-sort dispatch of the token slots into per-expert segments
// (src/engine.zig:553-564) and the tile list of the grouped GEMMs.
//
// Slot s = t * n_used + k routes token t to expert ids[s]. The result is the reference's
// stable order: order_start[e] is the exclusive prefix of the expert counts and
// route_order[order_start[e] + i] is the i-th slot, in increasing slot order, that chose e.
// One group of 16 waves: wave w owns a contiguous run of slots. Pass 1 counts per (wave,
// expert) with LDS atomics; the counts become per-wave write cursors by a prefix over waves
// then over experts; pass 2 walks each run again in slot order and places every slot at its
// cursor plus its rank among the lanes of the same round that chose the same expert (found
// with ten ballots over the expert id bits); the highest such lane advances the cursor.
// Tiles: each expert's segment is cut into tiles of at most tile_rows sorted rows. The list
// holds the full tiles first (expert by expert), then the partial tiles by decreasing row count
// (ties by expert), so that the grouped GEMMs, whose groups start in list order, begin with the
// longest tiles and end with the shortest.
// Output meta (u32 words): [0, n_expert] order_start, [1023] tile count,
// [1024 + 4 i ..] tile i = {expert, first sorted row, rows, 0}.
// Grid: 1; 1024 threads. Requires n_expert <= 512.
// Constants: 0 ids_uav 1 ids_off 2 n_slots 3 n_expert 4 order_uav 5 order_off 6 meta_uav
// 7 tile_rows.
#include "gd_kernel.h"

#define SORT_MAX_E 512
#define SORT_WAVES 16

GD_PIPELINE_NAMED(moe_prefill_sort, 1024) {
    __shared__ uint32_t cur[SORT_WAVES][SORT_MAX_E];
    __shared__ uint32_t start[SORT_MAX_E + 1], tstart[SORT_MAX_E + 1], fstart[SORT_MAX_E + 1];
    __shared__ uint32_t psz[SORT_MAX_E];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t n_slots = a.c[2], NE = a.c[3], TM = a.c[7];
    const uint32_t *ids = gd_buf<const uint32_t>(a, a.c[0]) + a.c[1];
    uint32_t *order = gd_buf<uint32_t>(a, a.c[4]) + a.c[5];
    uint32_t *meta = gd_buf<uint32_t>(a, a.c[6]);

    for (uint32_t i = tid; i < SORT_WAVES * SORT_MAX_E; i += 1024u) (&cur[0][0])[i] = 0u;
    __syncthreads();
    // Runs of whole rounds of 64 slots per wave.
    const uint32_t per_wave = ((n_slots + SORT_WAVES * 64u - 1u) / (SORT_WAVES * 64u)) * 64u;
    const uint32_t s0 = wave * per_wave, s1 = min(s0 + per_wave, n_slots);
    for (uint32_t s = s0 + lane; s < s1; s += 64u) atomicAdd(&cur[wave][min(ids[s], NE - 1u)], 1u);
    __syncthreads();
    // Column prefix over waves: cur[w][e] becomes the count of e in runs before w.
    uint32_t total = 0;
    if (tid < NE) {
        for (uint32_t w = 0; w < SORT_WAVES; ++w) {
            const uint32_t c = cur[w][tid];
            cur[w][tid] = total;
            total += c;
        }
    }
    // Exclusive prefix over experts of the counts and of the tile counts (wave 0..7 hold
    // experts 0..511; each wave scans its 64, then the 8 wave totals are added).
    __shared__ uint32_t wsum[8][3];
    uint32_t cnt = tid < NE ? total : 0u, tiles = (cnt + TM - 1u) / TM, full = cnt / TM;
    uint32_t ic = cnt, it = tiles, iff = full;
    if (tid < NE) psz[tid] = cnt - full * TM;
    if (wave < 8u) {
#pragma unroll
        for (uint32_t o = 1; o < 64; o <<= 1) {
            const uint32_t pc = __shfl_up(ic, o, 64), pt = __shfl_up(it, o, 64), pf = __shfl_up(iff, o, 64);
            if (lane >= o) {
                ic += pc;
                it += pt;
                iff += pf;
            }
        }
        if (lane == 63u) {
            wsum[wave][0] = ic;
            wsum[wave][1] = it;
            wsum[wave][2] = iff;
        }
    }
    __syncthreads();
    if (wave < 8u) {
        uint32_t bc = 0, bt = 0, bf = 0;
        for (uint32_t w = 0; w < wave; ++w) {
            bc += wsum[w][0];
            bt += wsum[w][1];
            bf += wsum[w][2];
        }
        if (tid <= NE) {  // tid == NE (< 512) receives the grand totals
            start[tid] = bc + ic - cnt;
            tstart[tid] = bt + it - tiles;
            fstart[tid] = bf + iff - full;
        }
    }
    __syncthreads();
    if (tid <= NE) meta[tid] = start[tid];
    if (tid == 0) meta[1023] = tstart[NE];
    // Cursors: segment start plus the counts of earlier runs.
    if (tid < NE)
        for (uint32_t w = 0; w < SORT_WAVES; ++w) cur[w][tid] += start[tid];
    __syncthreads();
    // Stable placement, one round of 64 slots at a time.
    for (uint32_t base = s0; base < s1; base += 64u) {
        const uint32_t s = base + lane;
        const bool valid = s < s1;
        const uint32_t e = valid ? min(ids[s], NE - 1u) : 1023u;  // 1023: matches no expert
        uint64_t peers = ~0ull;
#pragma unroll
        for (int b = 0; b < 10; ++b) {
            const uint64_t bb = __builtin_amdgcn_ballot_w64(((e >> b) & 1u) != 0u);
            peers &= ((e >> b) & 1u) ? bb : ~bb;
        }
        const uint32_t rank = (uint32_t)__builtin_popcountll(peers & ((1ull << lane) - 1ull));
        if (valid) {
            const uint32_t pos = cur[wave][e] + rank;
            order[pos] = s;
            if (lane == 63u - (uint32_t)__builtin_clzll(peers)) cur[wave][e] += (uint32_t)__builtin_popcountll(peers);
        }
    }
    // Tile list: full tiles at the exclusive prefix of the full-tile counts, then the partial
    // tile of each expert at the full-tile total plus its rank by decreasing size.
    if (tid < NE) {
        uint4 *list = reinterpret_cast<uint4 *>(meta + 1024u);
        const uint32_t c = start[tid + 1] - start[tid], nf = c / TM, p = c - nf * TM;
        for (uint32_t j = 0; j < nf; ++j) list[fstart[tid] + j] = make_uint4(tid, start[tid] + j * TM, TM, 0u);
        if (p) {
            uint32_t rank = 0;
            for (uint32_t e2 = 0; e2 < NE; ++e2) {
                const uint32_t q = psz[e2];
                rank += (q > p || (q == p && e2 < tid)) ? 1u : 0u;
            }
            list[fstart[NE] + rank] = make_uint4(tid, start[tid] + nf * TM, p, 0u);
        }
    }
}
