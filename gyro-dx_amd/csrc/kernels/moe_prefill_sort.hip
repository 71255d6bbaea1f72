// Prefill path, step 3: counting-sort dispatch of the token slots into per-expert segments
// (src/engine.zig:553-564) and the tile list of the grouped GEMMs.
//
// Slot s = t * n_used + k routes token t to expert ids[s]. The result is the reference's
// stable order: order_start[e] is the exclusive prefix of the expert counts and
// route_order[order_start[e] + i] is the i-th slot, in increasing slot order, that chose e.
// The slots form chunks of 256, and moe_prefill_topk has counted hist[c][e], the slots of chunk c
// that chose expert e (device-scope atomics into a histogram the router zeroed; a chunk's counts
// are contiguous, so a popular expert's atomics spread over one cache line per chunk). Group c
// places chunk c:
//  - thread e sums column e of the histogram: the expert's total, and its count in the chunks
//    before c;
//  - the group scans the totals over experts into order_start, so each expert's cursor for the
//    chunk is order_start[e] plus its count in the earlier chunks;
//  - wave 0 walks the chunk's slots in slot order, 64 per round, and places each slot at its
//    expert's cursor plus its rank among the round's lanes of the same expert (one ballot per
//    expert-id bit); the highest such lane advances the cursor.
// Tiles (group 0): each expert's segment is cut into tiles of at most tile_rows sorted rows. The
// list holds the full tiles first (expert by expert), then the partial tiles by decreasing row
// count (ties by expert), so that the grouped GEMMs, whose groups start in list order, begin with
// the longest tiles and end with the shortest; wave 1 ranks the partial tiles by a histogram of
// their sizes and stable ranks within each size.
// Output meta (u32 words): [0, n_expert] order_start, [1023] tile count,
// [1024 + 4 i ..] tile i = {expert, first sorted row, rows, 0}.
// Grid: ceil(n_slots / 256); 256 threads. Requires n_expert <= 256, n_slots <= 32768,
// tile_rows <= 256.
// Constants: 0 ids_uav 1 ids_off 2 n_slots 3 n_expert 4 order_uav 5 order_off 6 meta_uav
// 7 tile_rows 8 sched_uav (0: none; else group 0 zeroes words 0 and 2 .. 63 + 2 x tile count for
// moe_prefill_gemm: its queue words, one counter and one ready slot per tile; word 1, the
// persistent GEMM's give-up word, is left for the host) 9 hist_uav 10 hist_off (words;
// [ceil(n_slots / 256)][n_expert] counts).
#include "gd_kernel.h"

#define SORT_CHUNK 256
#define SORT_MAX_E 256
#define SORT_MAX_TM 256

GD_PIPELINE_NAMED(moe_prefill_sort, 256) {
    __shared__ uint32_t start[SORT_MAX_E + 1], tstart[SORT_MAX_E + 1], fstart[SORT_MAX_E + 1];
    __shared__ uint32_t cur[SORT_MAX_E], psz[SORT_MAX_E], rnk[SORT_MAX_E];
    __shared__ uint32_t hsz[SORT_MAX_TM], seen[SORT_MAX_TM];
    __shared__ uint32_t idc[SORT_CHUNK];
    __shared__ uint32_t wsum[4][3];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t n_slots = a.c[2], NE = a.c[3], TM = a.c[7];
    const uint32_t c = blockIdx.x, nch = (n_slots + SORT_CHUNK - 1u) / SORT_CHUNK;
    const bool lead = c == 0u;  // uniform per group
    uint32_t *order = gd_buf<uint32_t>(a, a.c[4]) + a.c[5];
    uint32_t *meta = gd_buf<uint32_t>(a, a.c[6]);
    // The chunk's expert ids and the histogram column, every load issued before the sums.
    const uint32_t s_mine = c * SORT_CHUNK + tid;
    const uint32_t id_mine = s_mine < n_slots ? gd_global(gd_buf<const uint32_t>(a, a.c[0]) + a.c[1])[s_mine] : 0u;
    uint32_t total = 0, colp = 0;
    if (tid < NE) {
        gd_guint *col = gd_global(gd_buf<const uint32_t>(a, a.c[9]) + a.c[10] + tid);
#pragma unroll 8
        for (uint32_t q = 0; q < nch; ++q) {
            const uint32_t h = col[q * NE];
            total += h;
            colp += q < c ? h : 0u;
        }
    }
    idc[tid] = min(id_mine, NE - 1u);
    if (lead) {
        hsz[tid] = 0u;
        seen[tid] = 0u;
    }
    // Exclusive prefix over experts of the counts, the tile counts and the full-tile counts:
    // each wave scans its 64 experts, then the wave totals are added.
    const uint32_t tiles = (total + TM - 1u) / TM, full = total / TM;
    uint32_t ic = total, it = tiles, iff = full;
    if (tid < NE) psz[tid] = total - full * TM;
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
    __syncthreads();
    uint32_t bc = 0, bt = 0, bf = 0;
    for (uint32_t w = 0; w < wave; ++w) {
        bc += wsum[w][0];
        bt += wsum[w][1];
        bf += wsum[w][2];
    }
    if (tid < NE) {
        start[tid] = bc + ic - total;
        tstart[tid] = bt + it - tiles;
        fstart[tid] = bf + iff - full;
        cur[tid] = bc + ic - total + colp;
    }
    if (tid == 0) {  // the grand totals
        start[NE] = (wsum[0][0] + wsum[1][0]) + (wsum[2][0] + wsum[3][0]);
        tstart[NE] = (wsum[0][1] + wsum[1][1]) + (wsum[2][1] + wsum[3][1]);
        fstart[NE] = (wsum[0][2] + wsum[1][2]) + (wsum[2][2] + wsum[3][2]);
    }
    if (lead && tid < NE && psz[tid]) atomicAdd(&hsz[psz[tid]], 1u);
    __syncthreads();

    // Stable placement of the chunk, one round of 64 slots at a time (wave 0).
    if (wave == 0u) {
        const uint32_t nb = NE > 1u ? 32u - (uint32_t)__builtin_clz(NE - 1u) : 1u;
#pragma unroll
        for (uint32_t r = 0; r < SORT_CHUNK / 64u; ++r) {
            const uint32_t s = c * SORT_CHUNK + r * 64u + lane;
            const bool valid = s < n_slots;
            const uint32_t e = idc[r * 64u + lane];
            uint64_t peers = __builtin_amdgcn_ballot_w64(valid);
#pragma unroll
            for (uint32_t b = 0; b < 8u; ++b) {
                if (b >= nb) break;  // uniform
                const uint64_t bb = __builtin_amdgcn_ballot_w64(((e >> b) & 1u) != 0u);
                peers &= ((e >> b) & 1u) ? bb : ~bb;
            }
            const uint32_t rank = (uint32_t)__builtin_popcountll(peers & ((1ull << lane) - 1ull));
            if (valid) {
                const uint32_t pos = cur[e] + rank;
                if (pos < n_slots) order[pos] = s;  // always, for a histogram of these ids
                if (lane == 63u - (uint32_t)__builtin_clzll(peers)) cur[e] += (uint32_t)__builtin_popcountll(peers);
            }
        }
    }
    if (!lead) return;  // uniform: the rest is group 0's

    // The counts of a histogram of these ids add up to n_slots; otherwise (a histogram not
    // zeroed before its call) no tile is listed, rather than a list past the buffers.
    const bool consistent = start[NE] == n_slots;
    const uint32_t n_tiles = consistent ? tstart[NE] : 0u;
    if (tid < NE) meta[tid] = start[tid];
    if (tid == 0) {
        meta[NE] = start[NE];
        meta[1023] = n_tiles;
    }
    if (a.c[8]) {
        uint32_t *sched = gd_buf<uint32_t>(a, a.c[8]);
        for (uint32_t i = tid; i < 64u + 2u * n_tiles; i += 256u)
            if (i != 1u) sched[i] = 0u;
    }
    // Rank of each partial tile by decreasing size, ties by expert (wave 1):
    // rank = (partial tiles larger than p) + (earlier experts of size p).
    if (wave == 1u) {
        // above[p] = sum of hsz[q] over q > p, p = 4 lane .. 4 lane + 3 (a scan over lanes from
        // the top).
        uint32_t h[4], hs = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            h[j] = hsz[4u * lane + j];
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
            seen[4u * lane + j] = ab;  // "above" until the rounds start
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
    __syncthreads();
    // Tile list: full tiles at the exclusive prefix of the full-tile counts, then the partial
    // tile of each expert at the full-tile total plus its rank.
    if (consistent && tid < NE) {
        uint4 *list = reinterpret_cast<uint4 *>(meta + 1024u);
        const uint32_t cnt = start[tid + 1] - start[tid], nf = cnt / TM, p = cnt - nf * TM;
        for (uint32_t j = 0; j < nf; ++j) list[fstart[tid] + j] = make_uint4(tid, start[tid] + j * TM, TM, 0u);
        if (p) list[fstart[NE] + rnk[tid]] = make_uint4(tid, start[tid] + nf * TM, p, 0u);
    }
}
