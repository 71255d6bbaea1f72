// Prefill path, step 3: counting-sort dispatch of the token slots into per-expert segments
// (src/engine.zig:553-564) and the tile list of the grouped GEMMs.
//
// Slot s = t * n_used + k routes token t to expert ids[s]. The result is the reference's
// stable order: order_start[e] is the exclusive prefix of the expert counts and
// route_order[order_start[e] + i] is the i-th slot, in increasing slot order, that chose e.
// One group of 16 waves. The expert ids are first copied into LDS as 16-bit values (every
// load issued up front). Wave w >= 1 owns a contiguous run of slots (wave 0 none: it ranks
// the partial tiles meanwhile). Pass 1 counts per (wave,
// expert) with LDS atomics; the counts become per-wave write cursors by a prefix over waves
// then over experts; pass 2 walks each run again in slot order and places every slot at its
// cursor plus its rank among the lanes of the same round that chose the same expert; the lanes
// of an expert find each other through a per-wave LDS table of 64-bit lane masks (ds_or), or
// with one ballot per expert-id bit beyond 256 experts; the highest such lane advances the
// cursor.
// Tiles: each expert's segment is cut into tiles of at most tile_rows sorted rows. The list
// holds the full tiles first (expert by expert), then the partial tiles by decreasing row count
// (ties by expert), so that the grouped GEMMs, whose groups start in list order, begin with the
// longest tiles and end with the shortest; wave 0 ranks the partial tiles by a histogram of their
// sizes and stable ranks within each size.
// Output meta (u32 words): [0, n_expert] order_start, [1023] tile count,
// [1024 + 4 i ..] tile i = {expert, first sorted row, rows, 0}.
// Grid: 1; 1024 threads. Requires n_expert <= 512, n_slots <= 32768, tile_rows <= 256.
// Constants: 0 ids_uav 1 ids_off 2 n_slots 3 n_expert 4 order_uav 5 order_off 6 meta_uav
// 7 tile_rows 8 sched_uav (0: none; else words 0 .. 63 + 2 x tile count are zeroed for
// moe_prefill_gemm: its queue words, give-up word, one counter and one ready slot per tile).
#include "gd_kernel.h"

#define SORT_MAX_E 512
#define SORT_WAVES 16
#define SORT_MAX_SLOTS 32768
#define SORT_MASK_E 256  // experts covered by the lane-mask table
#define SORT_MAX_TM 256

GD_PIPELINE_NAMED(moe_prefill_sort, 1024) {
    __shared__ uint32_t cur[SORT_WAVES][SORT_MAX_E];
    __shared__ uint32_t start[SORT_MAX_E + 1], tstart[SORT_MAX_E + 1], fstart[SORT_MAX_E + 1];
    __shared__ uint32_t psz[SORT_MAX_E], rnk[SORT_MAX_E];
    __shared__ uint32_t hsz[SORT_MAX_TM], seen[SORT_MAX_TM];
    __shared__ uint16_t id16[SORT_MAX_SLOTS];
    __shared__ uint64_t pmask[SORT_WAVES][SORT_MASK_E];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t n_slots = a.c[2], NE = a.c[3], TM = a.c[7];
    const uint32_t *ids = gd_buf<const uint32_t>(a, a.c[0]) + a.c[1];
    uint32_t *order = gd_buf<uint32_t>(a, a.c[4]) + a.c[5];
    uint32_t *meta = gd_buf<uint32_t>(a, a.c[6]);

    for (uint32_t i = tid; i < SORT_WAVES * SORT_MAX_E; i += 1024u) (&cur[0][0])[i] = 0u;
    for (uint32_t i = tid; i < SORT_WAVES * SORT_MASK_E; i += 1024u) (&pmask[0][0])[i] = 0ull;
    if (tid < SORT_MAX_TM) {
        hsz[tid] = 0u;
        seen[tid] = 0u;
    }
#pragma unroll 8
    for (uint32_t i = tid; i < n_slots; i += 1024u) id16[i] = (uint16_t)min(ids[i], NE - 1u);
    __syncthreads();
    // Runs of whole rounds of 64 slots per wave. Wave 0 ranks the partial tiles while waves
    // 1 .. 15 place the slots, so the placement runs have no slots for wave 0.
    const uint32_t per_wave = ((n_slots + (SORT_WAVES - 1u) * 64u - 1u) / ((SORT_WAVES - 1u) * 64u)) * 64u;
    const uint32_t s0 = wave == 0u ? n_slots : (wave - 1u) * per_wave, s1 = min(s0 + per_wave, n_slots);
    for (uint32_t s = s0 + lane; s < s1; s += 64u) atomicAdd(&cur[wave][id16[s]], 1u);
    __syncthreads();
    // Column prefix over waves, in registers: colp[w] is the count of e in runs before w.
    uint32_t total = 0, colp[SORT_WAVES];
    if (tid < NE) {
#pragma unroll
        for (uint32_t w = 0; w < SORT_WAVES; ++w) colp[w] = cur[w][tid];
#pragma unroll
        for (uint32_t w = 0; w < SORT_WAVES; ++w) {
            const uint32_t c = colp[w];
            colp[w] = total;
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
    if (tid < NE && psz[tid]) atomicAdd(&hsz[psz[tid]], 1u);
    __syncthreads();
    if (tid <= NE) meta[tid] = start[tid];
    if (tid == 0) meta[1023] = tstart[NE];
    if (a.c[8]) {
        // The persistent GEMM's queue words and per-tile counters. Word 1, its give-up word, is
        // sticky: only the host clears it, after reading it, so a give-up in any call of a run or
        // layer of a stack stays visible until then.
        uint32_t *sched = gd_buf<uint32_t>(a, a.c[8]);
        for (uint32_t i = tid; i < 64u + 2u * tstart[NE]; i += 1024u)
            if (i != 1u) sched[i] = 0u;
    }
    // Cursors: segment start plus the counts of earlier runs.
    if (tid < NE) {
        const uint32_t st = start[tid];
#pragma unroll
        for (uint32_t w = 0; w < SORT_WAVES; ++w) cur[w][tid] = colp[w] + st;
    }
    __syncthreads();
    // Rank of each partial tile by decreasing size, ties by expert (wave 0, before its share of
    // the placement): rank = (partial tiles larger than p) + (earlier experts of size p).
    if (wave == 0u) {
        // above[p] = sum of hsz[q] over q > p, p = 4 lane .. 4 lane + 3 (a scan over lanes from
        // the top).
        uint32_t h[4], hs = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            h[j] = 4u * lane + j < SORT_MAX_TM ? hsz[4u * lane + j] : 0u;
            hs += h[j];
        }
        uint32_t suf = hs;  // inclusive suffix over lanes >= lane
#pragma unroll
        for (uint32_t o = 1; o < 64; o <<= 1) {
            const uint32_t v = __shfl_down(suf, o, 64);
            if (lane + o < 64u) suf += v;
        }
        uint32_t ab = suf - hs;  // sizes above this lane's four
#pragma unroll
        for (int j = 3; j >= 0; --j) {
            seen[4u * lane + j] = ab;  // reused below as "above" until the rounds start
            ab += h[j];
        }
        // Stable ranks within a size: one round of 64 experts at a time.
        const uint32_t nbs = 32u - (uint32_t)__builtin_clz(SORT_MAX_TM - 1u);
        uint32_t above_p[SORT_MAX_E / 64];
#pragma unroll
        for (uint32_t r = 0; r < SORT_MAX_E / 64u; ++r) {
            const uint32_t e = r * 64u + lane;
            const uint32_t p = e < NE ? psz[e] : 0u;
            above_p[r] = seen[p];
        }
        for (uint32_t i = lane; i < SORT_MAX_TM; i += 64u) seen[i] = 0u;
#pragma unroll
        for (uint32_t r = 0; r < SORT_MAX_E / 64u; ++r) {
            if (r * 64u >= NE) break;  // uniform
            const uint32_t e = r * 64u + lane;
            const uint32_t p = e < NE ? psz[e] : 0u;
            uint64_t peers = __builtin_amdgcn_ballot_w64(p != 0u);
#pragma unroll
            for (uint32_t b = 0; b < nbs; ++b) {
                const uint64_t bb = __builtin_amdgcn_ballot_w64(((p >> b) & 1u) != 0u);
                peers &= ((p >> b) & 1u) ? bb : ~bb;
            }
            if (p) {
                rnk[e] = above_p[r] + seen[p] + (uint32_t)__builtin_popcountll(peers & ((1ull << lane) - 1ull));
                if (lane == 63u - (uint32_t)__builtin_clzll(peers)) seen[p] += (uint32_t)__builtin_popcountll(peers);
            }
        }
    }
    // Stable placement, one round of 64 slots at a time.
    const bool use_mask = NE <= SORT_MASK_E;
    const uint32_t nb = NE > 1u ? 32u - (uint32_t)__builtin_clz(NE - 1u) : 1u;
    for (uint32_t base = s0; base < s1; base += 64u) {
        const uint32_t s = base + lane;
        const bool valid = s < s1;
        const uint32_t e = valid ? (uint32_t)id16[s] : 0u;
        uint64_t peers;
        if (use_mask) {  // uniform
            if (valid) atomicOr(reinterpret_cast<unsigned long long *>(&pmask[wave][e]), 1ull << lane);
            peers = valid ? pmask[wave][e] : 0ull;
        } else {
            peers = __builtin_amdgcn_ballot_w64(valid);
#pragma unroll
            for (uint32_t b = 0; b < 9u; ++b) {
                if (b >= nb) break;  // uniform
                const uint64_t bb = __builtin_amdgcn_ballot_w64(((e >> b) & 1u) != 0u);
                peers &= ((e >> b) & 1u) ? bb : ~bb;
            }
        }
        const uint32_t rank = (uint32_t)__builtin_popcountll(peers & ((1ull << lane) - 1ull));
        if (valid) {
            const uint32_t pos = cur[wave][e] + rank;
            order[pos] = s;
            if (lane == 63u - (uint32_t)__builtin_clzll(peers)) {
                cur[wave][e] += (uint32_t)__builtin_popcountll(peers);
                if (use_mask) pmask[wave][e] = 0ull;
            }
        }
    }
    __syncthreads();
    // Tile list: full tiles at the exclusive prefix of the full-tile counts, then the partial
    // tile of each expert at the full-tile total plus its rank.
    if (tid < NE) {
        uint4 *list = reinterpret_cast<uint4 *>(meta + 1024u);
        const uint32_t c = start[tid + 1] - start[tid], nf = c / TM, p = c - nf * TM;
        for (uint32_t j = 0; j < nf; ++j) list[fstart[tid] + j] = make_uint4(tid, start[tid] + j * TM, TM, 0u);
        if (p) list[fstart[NE] + rnk[tid]] = make_uint4(tid, start[tid] + nf * TM, p, 0u);
    }
}
