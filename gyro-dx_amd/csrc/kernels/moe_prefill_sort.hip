// Prefill path, step 3: counting-sort dispatch of the token slots into per-expert segments
// (src/engine.zig:553-564) and the tile list of the grouped GEMMs.
//
// Slot s = t * n_used + k routes token t to expert ids[s]. The result is the reference's
// stable order: order_start[e] is the exclusive prefix of the expert counts and
// route_order[order_start[e] + i] is the i-th slot, in increasing slot order, that chose e.
// The slots form chunks of 256, and moe_prefill_topk has counted hist[c][e], the slots of chunk c
// that chose expert e (device-scope atomics into a histogram the router zeroed; a chunk's counts
// are contiguous, so a popular expert's atomics spread over one cache line per chunk). Group c
// places chunk c, its four waves side by side at every step:
//  - the expert's total and its count in the chunks before c: thread e reads its histogram
//    column itself when there are at most 8 chunks; otherwise wave w sums chunks w, w + 4, ... for
//    experts 4 lane .. 4 lane + 3 (16-byte loads when rows are whole 16-byte words; every load
//    issued before the sums) and thread e adds the four waves' partial sums;
//  - wave scans (DPP) of the totals, the tile counts and the full-tile counts give order_start
//    and each expert's cursor for the chunk: order_start[e] plus its count in the earlier chunks;
//  - thread i holds slot 256 c + i; its rank among the wave's lanes of the same expert (one
//    ballot per expert-id bit) plus the counts of that expert in the chunk's earlier waves puts
//    it at its expert's cursor plus the slots of that expert before it in the chunk.
// Tiles (group 0): each expert's segment is cut into tiles of at most tile_rows sorted rows. The
// list holds the full tiles first (expert by expert), then the partial tiles by decreasing row
// count (ties by expert), so that the grouped GEMMs, whose groups start in list order, begin with
// the longest tiles and end with the shortest. A partial tile's rank is the number of larger
// partial tiles (a scan over sizes of the size histogram) plus the number of earlier experts
// whose partial tile has its size (its rank among its wave's lanes of that size plus the counts
// of earlier waves).
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
#define SORT_WAVES 4

// Rank of this lane among the wave's valid lanes whose key has the same low `bits` bits (bits <=
// 8, uniform), the number of such lanes, and whether this lane is the highest of them.
__device__ __forceinline__ uint32_t sort_match(uint32_t key, uint32_t bits, bool valid, uint32_t &count,
                                               bool &highest) {
    const uint32_t lane = threadIdx.x & 63u;
    uint64_t peers = __builtin_amdgcn_ballot_w64(valid);
#pragma unroll
    for (uint32_t b = 0; b < 8u; ++b) {
        if (b >= bits) break;  // uniform
        const uint64_t bb = __builtin_amdgcn_ballot_w64(((key >> b) & 1u) != 0u);
        peers &= ((key >> b) & 1u) ? bb : ~bb;
    }
    const uint64_t own = valid ? peers : 1ull;  // a valid lane is among its own peers
    count = (uint32_t)__builtin_popcountll(peers);
    highest = valid && lane == 63u - (uint32_t)__builtin_clzll(own);
    return (uint32_t)__builtin_popcountll(peers & ((1ull << lane) - 1ull));
}

// Exclusive prefixes over the group's 256 threads of N values per thread, from the DPP wave
// scans and the wave totals (one barrier for all N); total[i]: the sum of value i over all
// threads. part: N x 4 words of LDS. Every thread of the group must call it.
template <int N>
__device__ __forceinline__ void sort_group_scan(const uint32_t (&v)[N], uint32_t (*part)[SORT_WAVES],
                                                uint32_t (&excl)[N], uint32_t (&total)[N]) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    uint32_t incl[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        incl[i] = gd_wave_scan_u32(v[i]);
        if (lane == 63u) part[i][wave] = incl[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < N; ++i) {
        uint32_t before = 0;
        for (uint32_t w = 0; w < wave; ++w) before += part[i][w];
        total[i] = (part[i][0] + part[i][1]) + (part[i][2] + part[i][3]);
        excl[i] = before + incl[i] - v[i];
    }
}

GD_PIPELINE_NAMED(moe_prefill_sort, 256) {
    __shared__ uint32_t start[SORT_MAX_E + 1], tstart[SORT_MAX_E + 1], fstart[SORT_MAX_E + 1];
    __shared__ uint32_t cur[SORT_MAX_E], above[SORT_MAX_TM];
    __shared__ uint32_t wtot[SORT_WAVES][SORT_MAX_E], wcol[SORT_WAVES][SORT_MAX_E];
    __shared__ uint32_t wcnt[SORT_WAVES][SORT_MAX_E], wsz[SORT_WAVES][SORT_MAX_TM];
    __shared__ uint32_t part[3][SORT_WAVES];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t n_slots = a.c[2], NE = a.c[3], TM = a.c[7];
    const uint32_t c = blockIdx.x, nch = (n_slots + SORT_CHUNK - 1u) / SORT_CHUNK;
    const bool lead = c == 0u;  // uniform per group
    uint32_t *order = gd_buf<uint32_t>(a, a.c[4]) + a.c[5];
    uint32_t *meta = gd_buf<uint32_t>(a, a.c[6]);

    // The slot's expert id and the histogram partials, every load issued before the sums.
    const uint32_t s_mine = c * SORT_CHUNK + tid;
    const bool valid = s_mine < n_slots;
    const uint32_t id_mine = valid ? gd_global(gd_buf<const uint32_t>(a, a.c[0]) + a.c[1])[s_mine] : 0u;
    const uint32_t *hist = gd_buf<const uint32_t>(a, a.c[9]) + a.c[10];
#pragma unroll
    for (int w = 0; w < SORT_WAVES; ++w) {
        wcnt[w][tid] = 0u;
        wsz[w][tid] = 0u;
    }
    // Thread e: the expert's total and its count in the chunks before c. Up to 8 chunks, thread e
    // reads its column itself; more, wave w sums chunks w, w + 4, ... for experts 4 lane ..
    // 4 lane + 3 and thread e adds the four waves' partial sums.
    uint32_t total = 0, colp = 0;
    if (nch <= 8u) {  // uniform
        if (tid < NE) {
            gd_guint *h1 = gd_global(hist) + tid;
            uint32_t h[8];
#pragma unroll
            for (uint32_t q = 0; q < 8u; ++q) h[q] = q < nch ? h1[q * NE] : 0u;
#pragma unroll
            for (uint32_t q = 0; q < 8u; ++q) {
                total += h[q];
                colp += q < c ? h[q] : 0u;
            }
        }
    } else {
        uint32_t tot[4] = {0u, 0u, 0u, 0u}, col[4] = {0u, 0u, 0u, 0u};
        if ((NE & 3u) == 0u && (a.c[10] & 3u) == 0u) {  // uniform: rows of whole 16-byte words
            // Lane l reads experts 4 l .. 4 l + 3 of a row as one 16-byte load: a wave covers the
            // row's contiguous words.
            gd_gu32x4 *h4 = gd_global4(hist);
            const uint32_t l4 = min(lane, NE / 4u - 1u);
#pragma unroll 8
            for (uint32_t q = wave; q < nch; q += SORT_WAVES) {
                const gd_u32x4 h = h4[q * (NE / 4u) + l4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t hv = 4u * lane < NE ? h[j] : 0u;
                    tot[j] += hv;
                    col[j] += q < c ? hv : 0u;
                }
            }
        } else {
            gd_guint *h1 = gd_global(hist);
#pragma unroll 8
            for (uint32_t q = wave; q < nch; q += SORT_WAVES) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t e = 4u * lane + (uint32_t)j;
                    const uint32_t h = h1[q * NE + min(e, NE - 1u)];
                    const uint32_t hv = e < NE ? h : 0u;
                    tot[j] += hv;
                    col[j] += q < c ? hv : 0u;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            wtot[wave][4u * lane + j] = tot[j];
            wcol[wave][4u * lane + j] = col[j];
        }
        __syncthreads();
        if (tid < NE) {
#pragma unroll
            for (int w = 0; w < SORT_WAVES; ++w) {
                total += wtot[w][tid];
                colp += wcol[w][tid];
            }
        }
    }

    // Order_start, the tile starts and the full-tile starts as exclusive prefixes over experts.
    const uint32_t tiles = (total + TM - 1u) / TM, full = total / TM;
    const uint32_t scan_in[3] = {total, tiles, full};
    uint32_t ex[3], all[3];
    sort_group_scan<3>(scan_in, part, ex, all);
    if (tid < NE) {
        start[tid] = ex[0];
        tstart[tid] = ex[1];
        fstart[tid] = ex[2];
        cur[tid] = ex[0] + colp;
    }
    if (tid == 0) {  // the grand totals
        start[NE] = all[0];
        tstart[NE] = all[1];
        fstart[NE] = all[2];
    }

    // Stable placement of the chunk: each wave's lanes of one expert in lane order, after the
    // chunk's earlier waves.
    const uint32_t e_mine = min(id_mine, NE - 1u);
    const uint32_t nb = NE > 1u ? 32u - (uint32_t)__builtin_clz(NE - 1u) : 1u;
    uint32_t cnt;
    bool highest;
    const uint32_t rank = sort_match(e_mine, nb, valid, cnt, highest);
    if (highest) wcnt[wave][e_mine] = cnt;
    // Group 0 also ranks the partial tiles by decreasing size, ties by expert:
    // rank = (partial tiles larger than p) + (earlier experts of size p). Here each wave's lanes
    // of one size in expert order.
    const uint32_t p_mine = tid < NE ? total - full * TM : 0u;
    uint32_t srank = 0;
    if (lead) {
        const uint32_t nbs = 32u - (uint32_t)__builtin_clz(SORT_MAX_TM - 1u);
        uint32_t scnt;
        bool shighest;
        srank = sort_match(p_mine, nbs, p_mine != 0u, scnt, shighest);
        if (shighest) wsz[wave][p_mine] = scnt;
    }
    __syncthreads();  // cur, wcnt and wsz
    if (valid) {
        uint32_t pos = cur[e_mine] + rank;
        for (uint32_t w = 0; w < wave; ++w) pos += wcnt[w][e_mine];
        if (pos < n_slots) order[pos] = s_mine;  // always, for a histogram of these ids
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
    // Partial tiles larger than each size p (wave 0, lane l for sizes 4 l .. 4 l + 3: the size
    // histogram from the four waves' counts, then a DPP scan over sizes).
    if (wave == 0u) {
        uint32_t hq[4], sum = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t p = 4u * lane + (uint32_t)j;
            hq[j] = (wsz[0][p] + wsz[1][p]) + (wsz[2][p] + wsz[3][p]);
            sum += hq[j];
        }
        const uint32_t incl = gd_wave_scan_u32(sum);
        const uint32_t n_partial = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
        uint32_t run = incl - sum;  // partial tiles of sizes below 4 lane
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            run += hq[j];
            above[4u * lane + j] = n_partial - run;
        }
    }
    __syncthreads();
    // Tile list: full tiles at the exclusive prefix of the full-tile counts, then the partial
    // tile of each expert at the full-tile total plus its rank.
    if (consistent && tid < NE) {
        uint4 *list = reinterpret_cast<uint4 *>(meta + 1024u);
        const uint32_t cnt_e = start[tid + 1] - start[tid], nf = cnt_e / TM, p = cnt_e - nf * TM;
        for (uint32_t j = 0; j < nf; ++j) list[fstart[tid] + j] = make_uint4(tid, start[tid] + j * TM, TM, 0u);
        if (p) {
            uint32_t r = above[p] + srank;
            for (uint32_t w = 0; w < wave; ++w) r += wsz[w][p];
            if (fstart[NE] + r < n_tiles) list[fstart[NE] + r] = make_uint4(tid, start[tid] + nf * TM, p, 0u);
        }
    }
}
