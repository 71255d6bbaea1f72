// Decode path in one launch for uniform TQ2_T layers at batch 1: (optional stack RMSNorm,
// src/kernels.zig:281-291) router and input rotation, routing, the routed gate/up dequant-GEMV
// with SwiGLU, the down rotation and dequant-GEMV, and the route-weighted combine
// (src/engine.zig:520-642). The steps that depend on one another run in different workgroups of
// one grid and hand their results over through device memory, so a token costs one launch
// instead of three.
//
// The G workgroups (all resident together: the host launches at most one per CU) exchange with
// device-scope loads and stores, which the L2s keep coherent; no fence (an L2 writeback) is
// issued. A store that another group must see before a counter update is acknowledged first
// (s_waitcnt), and every exchanged value is read with a device-scope load.
//  (0) every group reads the call's epoch e = EP + 1 (EP, the last call's, is in the exchange
//      area; 0 is skipped), so consecutive calls tag their words differently;
//  (1) group g computes router rows g, g + G, ... and stores each logit as one 64-bit word
//      (e << 32 | bits), one word per 128-byte line; groups without a router row store an
//      arrival word in slot g the same way, after their last read of the input; every group
//      rotates the input into LDS itself;
//  (2) group 0 polls slots 0 .. max(NE, G) - 1 until all carry e (every group has read the input
//      and EP), stores EP = e, routes the token (top-U by logit, ties to the lower index,
//      renormalised weights; one wave, unrolled rounds) and stores the U id words tagged e, then
//      the U weight words; every group polls the ids (and, with its flags, the weights);
//  (3) gate/up unit (k, j): rows FB j .. FB j + FB - 1 of slot k's gate and up matrices, one
//      (row, block) per thread, summed per row in block order through LDS; the SwiGLU times the
//      down sign goes to ACT[k][f]; once the group's stores are acknowledged it adds 1 to slot
//      k's counter; the arrival that completes the count (F / FB) resets it and stores the slot's
//      flag e;
//  (4) down unit rb: rows RB rb .. RB rb + RB - 1 of every slot's down matrix, requested right
//      after routing with the gate/up rows; once every slot's flag carries e the group reads
//      ACT, rotates it (H_128 per block in 16-lane DPP rows), decodes half blocks (one per
//      thread) against it, sums each (slot, row) in (block, half) order, and writes the output
//      row sum_k w_k d_k[r] in slot order (then adds the residual, when the call has one).
// Per-group LDS sums read all their operands at once (clamped indices, zero terms past the end),
// so each is one LDS round trip.
// Counters are zero between calls. Every wait is bounded by a spin limit; a group that gives up
// stores e to the error tag (acknowledged before its next counter update or route store) and 1
// to the sticky error word, and goes on, so the grid always drains; a group that gave up, or
// that reads the error tag equal to e after its flag wait, writes NaN rows, and the host
// refuses the call's output.
//
// Grid: G <= 512 groups; 512 threads.
// Constants: 0 x_uav 1 x_off 2 router_srv 3 bias_srv (0xffffffff: none) 4 signs_srv (gate signs
// [E], then down signs [F]) 5 rotations (bit 0: the input, bit 1: the down input) 6 xch_uav (the
// exchange area) 7 log_off 8 route_off 9 act_off 10 cnt_off 11 flag_off (word offsets in the
// exchange area; logits, counters and flags 32 words apart) 12 out_uav 13 out_off 14 base_lo
// 15 base_hi 16 slot_stride 17 gate_bytes 18 codebook_srv 19 E 20 F 21 n_expert 22 n_used
// 23 scale (fp32 bits) 24 ctl_off (EP at ctl_off, the error tag at + 32, the sticky error word at
// + 64) 25 ids_uav 26 ids_off 27 weights_uav 28 weights_off 29 residual (0: none, 1: add)
// 30 res_uav 31 res_off 32 range flag (table index, 0: none) 33 spin limit 34 norm (0: none,
// 1: RMSNorm without weight, 2: with weight) 35 FB 36 RB 37 norm_w_srv 38 eps (fp32 bits).
// Requires E a multiple of 256 up to 4096, F a multiple of 128 up to 1024, F % FB == 0,
// E % RB == 0, 1 <= n_used <= 16, n_used F / 128 <= FU_MAX_ABLK, n_expert <= 512, and per group
// at most FU_MAX_GUNITS gate/up and FU_MAX_DUNITS down units whose items fit FU_ITEMS per thread
// (the host checks).
#include "gyro_fast.h"
#include "fwht.h"
#include "route_fast.h"

#define FU_ITEMS 4                 // gate/up (row, block) and down (slot, row, block, half) items per thread
#define FU_MAX_U 16
#define FU_MAX_DUNITS 4            // down units per group
#define FU_MAX_GUNITS 4            // gate/up units per group
#define FU_MAX_FB 16
#define FU_MAX_ABLK 128            // rotated down-input blocks (slots x F / 128) in LDS
#define FU_BLOCK_STRIDE 132        // floats per 128-block of a down input in LDS (bank spread)

typedef unsigned long long fu_u64;

__device__ __forceinline__ fu_u64 fu_ld64(const fu_u64 *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void fu_st64(fu_u64 *p, fu_u64 v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ uint32_t fu_ld32(const uint32_t *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void fu_st32(uint32_t *p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void fu_stf(float *p, float v) {
    __hip_atomic_store(reinterpret_cast<uint32_t *>(p), gd_f32_bits(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float fu_ldf(const float *p) {
    return gd_bits_f32(__hip_atomic_load(reinterpret_cast<const uint32_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// A wait that reached the spin limit: the call's error tag and the sticky error word.
__device__ __forceinline__ void fu_give_up(uint32_t *ctl, uint32_t epoch) {
    fu_st32(ctl + 32, epoch);
    fu_st32(ctl + 64, 1u);
}

// The 9 words from the 4-byte-aligned start of the 34-byte block at byte `off` of `base`.
__device__ __forceinline__ void fu_load_block(const uint8_t *base, uint64_t off, uint32_t d[9]) {
    gd_guint *w = gd_global(reinterpret_cast<const uint32_t *>(base + (off & ~uint64_t(3))));
#pragma unroll
    for (int j = 0; j < 9; ++j) d[j] = w[j];
}

// Top-U of the token by one wave from the lane's logits lv[j] (expert lane + 64 j, PER per
// lane) in unrolled rounds (route_fast.h); UU bounds U at compile time. Returns the id of rank
// lane % 16; top[k] holds the k-th logit (0 past U).
template <int PER, int UU>
__device__ __forceinline__ uint32_t fu_top(const float lv[8], uint32_t NE, uint32_t U, float top[FU_MAX_U]) {
    float v[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) v[j] = lv[j];
    uint64_t key[PER];
    rf_init<PER>(v, NE, key);
    uint32_t ids[UU];
#pragma unroll
    for (int k = 0; k < FU_MAX_U; ++k) top[k] = 0.f;
#pragma unroll
    for (int k = 0; k < UU; ++k) {
        ids[k] = 0u;
        if (UU < FU_MAX_U || (uint32_t)k < U) ids[k] = rf_next<PER>(key, top[k]);  // uniform
    }
    const uint32_t me = threadIdx.x & 15u;
    uint32_t id = ids[0];
#pragma unroll
    for (int k = 1; k < UU; ++k) id = me == (uint32_t)k ? ids[k] : id;
    return id;
}

// Weight of rank lane % 16: w_k = exp(l_k - l_0) / sum_j exp(l_j - l_0) over the U selected
// logits, times the layer's scale unless it is 0 or 1 (rf_weights).
__device__ __forceinline__ float fu_weight(const float top[FU_MAX_U], uint32_t U, float scale) {
    float wts[FU_MAX_U], total = 0.f;
#pragma unroll
    for (int k = 0; k < FU_MAX_U; ++k) {
        wts[k] = 0.f;
        if ((uint32_t)k < U) {
            wts[k] = expf(top[k] - top[0]);
            total += wts[k];
        }
    }
    const float inv = 1.0f / total;
    const uint32_t me = threadIdx.x & 15u;
    float w = wts[0];
#pragma unroll
    for (int k = 1; k < FU_MAX_U; ++k) w = me == (uint32_t)k ? wts[k] : w;
    w *= inv;
    if (scale != 0.f && scale != 1.f) w *= scale;
    return w;
}

// 16-lane H_128 of the values v[0..7] of lanes 8 l16 .. + 7 of one block, times 1 / sqrt(128)
// (widths 1, 2, 4 in registers, then 8 .. 64 across the 16-lane row: src/gyro.zig:152-172).
__device__ __forceinline__ void fu_fwht16(float v[8], uint32_t l16) {
#pragma unroll
    for (int w = 1; w < 8; w <<= 1)
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (!(j & w)) {
                const float lo = v[j], hi = v[j + w];
                v[j] = lo + hi;
                v[j + w] = lo - hi;
            }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float p1 = gd_dpp_f<0xB1>(v[j]);  // quad_perm [1,0,3,2]
        v[j] = (l16 & 1u) ? p1 - v[j] : v[j] + p1;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float p2 = gd_dpp_f<0x4E>(v[j]);  // quad_perm [2,3,0,1]
        v[j] = (l16 & 2u) ? p2 - v[j] : v[j] + p2;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float up4 = gd_dpp_f<0x104>(v[j]), dn4 = gd_dpp_f<0x114>(v[j]);  // row_shl:4, row_shr:4
        v[j] = (l16 & 4u) ? dn4 - v[j] : v[j] + up4;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float up8 = gd_dpp_f<0x108>(v[j]), dn8 = gd_dpp_f<0x118>(v[j]);  // row_shl:8, row_shr:8
        v[j] = (l16 & 8u) ? dn8 - v[j] : v[j] + up8;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] *= GD_INV_SQRT128;
}

GD_PIPELINE_NAMED(moe_decode_fused, 512) {
    __shared__ gd_u32x4 book4[512];
    __shared__ uint4 xh4[4096 / 8];  // rotated input as binary16, block b's chunk c at b * 16 + (c + b) % 16
    __shared__ float gred[FU_ITEMS * 512];
    __shared__ float gsum[FU_MAX_GUNITS * 2 * FU_MAX_FB];
    __shared__ float dred[FU_ITEMS * 512];
    __shared__ float actr[FU_MAX_ABLK * FU_BLOCK_STRIDE];  // rotated down input, (slot, block) rows
    __shared__ float rsum[8][2];
    __shared__ uint32_t rid[FU_MAX_U];
    __shared__ float rw[FU_MAX_U];
    __shared__ uint32_t bad;  // this group gave up a wait, or another group did before its flags

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t g = blockIdx.x, G = gridDim.x;
    const uint32_t E = a.c[19], F = a.c[20], NE = a.c[21], U = a.c[22];
    const uint32_t nb = E / 128u, nbF = F / 128u, FB = a.c[35], RB = a.c[36];
    const uint32_t limit = a.c[33], norm = a.c[34];
    const bool has_signs = (a.c[5] & 1u) != 0u, has_dsigns = (a.c[5] & 2u) != 0u;
    uint32_t *X = gd_buf<uint32_t>(a, a.c[6]);  // the exchange area
    fu_u64 *LOG = reinterpret_cast<fu_u64 *>(X + a.c[7]);
    fu_u64 *ROUTE = reinterpret_cast<fu_u64 *>(X + a.c[8]);
    float *ACT = reinterpret_cast<float *>(X + a.c[9]);
    uint32_t *CNT = X + a.c[10];   // slot counters, 32 words apart
    uint32_t *FLAG = X + a.c[11];  // slot flags, 32 words apart
    uint32_t *CTL = X + a.c[24];   // EP, error tag (+ 32), sticky error word (+ 64)
    if (tid == 0) bad = 0u;

    // ---- (0) the call's epoch, (1) router rows, rotated input -------------------------------
    uint32_t epoch = fu_ld32(CTL) + 1u;
    epoch = epoch ? epoch : 1u;
    const float *Xin = gd_buf<const float>(a, a.c[0]) + a.c[1];
    const bool xt = tid < E / 8u;  // thread t holds x[8 t .. 8 t + 7]
    float xv[8], sv[8], nwv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) { xv[j] = 0.f; sv[j] = 1.f; nwv[j] = 1.f; }
    if (xt) {
        gd_gu32x4 *xp = gd_global4(reinterpret_cast<const uint32_t *>(Xin) + 8u * tid);
        const gd_u32x4 x0 = xp[0], x1 = xp[1];
#pragma unroll
        for (int j = 0; j < 4; ++j) { xv[j] = gd_bits_f32(x0[j]); xv[4 + j] = gd_bits_f32(x1[j]); }
        if (norm == 2u) {
            gd_gu32x4 *np = gd_global4(gd_buf<const uint32_t>(a, a.c[37]) + 8u * tid);
            const gd_u32x4 n0 = np[0], n1 = np[1];
#pragma unroll
            for (int j = 0; j < 4; ++j) { nwv[j] = gd_bits_f32(n0[j]); nwv[4 + j] = gd_bits_f32(n1[j]); }
        }
    }
    // RMSNorm scale 1 / sqrt(mean(x^2) + eps), summed per wave, then over the 8 waves.
    float scn = 1.f;
    if (norm) {
        const float ss = ((xv[0] * xv[0] + xv[1] * xv[1]) + (xv[2] * xv[2] + xv[3] * xv[3])) +
                         ((xv[4] * xv[4] + xv[5] * xv[5]) + (xv[6] * xv[6] + xv[7] * xv[7]));
        const float q = gd_wave_sum_dpp(ss);
        if (lane == 0) rsum[wave][1] = q;
        __syncthreads();
        const float t = ((rsum[0][1] + rsum[1][1]) + (rsum[2][1] + rsum[3][1])) +
                        ((rsum[4][1] + rsum[5][1]) + (rsum[6][1] + rsum[7][1]));
        scn = 1.0f / sqrtf(t / (float)E + gd_bits_f32(a.c[38]));
    }
    float xw[8];  // the router's input: x times the norm weight
#pragma unroll
    for (int j = 0; j < 8; ++j) xw[j] = xv[j] * nwv[j];
    const uint32_t *W = gd_buf<const uint32_t>(a, a.c[2]);
    for (uint32_t r = g; r < NE; r += G) {  // uniform per group
        float acc = 0.f;
        if (xt) {
            gd_gu32x4 *wp = gd_global4(W + (size_t)r * E + 8u * tid);
            const gd_u32x4 w0 = wp[0], w1 = wp[1];
            acc = ((xw[0] * gd_bits_f32(w0[0]) + xw[1] * gd_bits_f32(w0[1])) +
                   (xw[2] * gd_bits_f32(w0[2]) + xw[3] * gd_bits_f32(w0[3]))) +
                  ((xw[4] * gd_bits_f32(w1[0]) + xw[5] * gd_bits_f32(w1[1])) +
                   (xw[6] * gd_bits_f32(w1[2]) + xw[7] * gd_bits_f32(w1[3])));
        }
        const float s = gd_wave_sum_dpp(acc);
        if (lane == 0) rsum[wave][0] = s;
        __syncthreads();
        if (tid == 0) {
            float v = ((rsum[0][0] + rsum[1][0]) + (rsum[2][0] + rsum[3][0])) +
                      ((rsum[4][0] + rsum[5][0]) + (rsum[6][0] + rsum[7][0]));
            if (norm) v *= scn;
            if (a.c[3] != 0xffffffffu) v += gd_buf<const float>(a, a.c[3])[r];
            fu_st64(LOG + (size_t)r * 16u, ((fu_u64)epoch << 32) | gd_f32_bits(v));
        }
        __syncthreads();
    }
    // The codebook and sign vector after the router rows, off their critical path.
    book4[tid] = gd_global4(gd_buf<const uint32_t>(a, a.c[18]))[tid];
    if (xt && has_signs) {
        gd_gu32x4 *sp = gd_global4(gd_buf<const uint32_t>(a, a.c[4]) + 8u * tid);
        const gd_u32x4 s0 = sp[0], s1 = sp[1];
#pragma unroll
        for (int j = 0; j < 4; ++j) { sv[j] = gd_bits_f32(s0[j]); sv[4 + j] = gd_bits_f32(s1[j]); }
    }
    // Rotated input: 16 lanes per 128-block, 8 values per lane (the butterfly of moe_router).
    if (xt) {
        const uint32_t l16 = lane & 15u, blk = tid >> 4;
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = norm ? (xv[j] * scn) * (sv[j] * nwv[j]) : xv[j] * sv[j];
        if (has_signs) fu_fwht16(v, l16);
        uint4 o;
        bool out_of_range = false;
        uint32_t h[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            out_of_range |= !gd_half_ok(v[j]);
            h[j] = __builtin_bit_cast(uint16_t, (_Float16)v[j]);
        }
        o.x = h[0] | (h[1] << 16); o.y = h[2] | (h[3] << 16); o.z = h[4] | (h[5] << 16); o.w = h[6] | (h[7] << 16);
        xh4[blk * 16u + ((l16 + blk) & 15u)] = o;
        if (g == 0u) gd_range_flag(a.table, a.c[32], out_of_range);
    }
    if (g >= NE) {  // uniform: the arrival word, after every thread's last use of the input
        __syncthreads();
        if (tid == 0) fu_st64(LOG + (size_t)g * 16u, (fu_u64)epoch << 32);
    }

    // ---- (2) routing --------------------------------------------------------------------
    if (g == 0u && wave == 0u) {
        const uint32_t slots = NE > G ? NE : G;
        float lv[8];
        for (uint32_t spins = 0;; ++spins) {  // uniform per wave
            bool ok = true;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t i = lane + 64u * (uint32_t)j;
                lv[j] = 0.f;
                if (i < slots) {
                    const fu_u64 v = fu_ld64(LOG + (size_t)i * 16u);
                    lv[j] = gd_bits_f32((uint32_t)v);
                    ok &= (uint32_t)(v >> 32) == epoch;
                }
            }
            if (__all(ok)) break;
            if (spins >= limit) {
                if (lane == 0) {
                    fu_give_up(CTL, epoch);
                    bad = 1u;
                }
                __builtin_amdgcn_s_waitcnt(0);  // the error tag before the route words
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        if (lane == 0) fu_st32(CTL, epoch);  // every group has read EP
        // The ids first (the gate/up rows wait for them), then the weights (needed at the end).
        float top[FU_MAX_U];
        uint32_t id;
        if (NE <= 256u && U == 8u) id = fu_top<4, 8>(lv, NE, U, top);
        else if (NE <= 256u && U == 10u) id = fu_top<4, 10>(lv, NE, U, top);
        else if (NE <= 256u) id = fu_top<4, FU_MAX_U>(lv, NE, U, top);
        else id = fu_top<8, FU_MAX_U>(lv, NE, U, top);
        if (lane < U) fu_st64(ROUTE + lane, ((fu_u64)epoch << 32) | id);
        const float wv = fu_weight(top, U, gd_bits_f32(a.c[23]));
        if (lane < 32u && (lane & 15u) < U) {
            const uint32_t k = lane & 15u;
            if (lane >= 16u) fu_st64(ROUTE + lane, ((fu_u64)epoch << 32) | gd_f32_bits(wv));
            if (lane < 16u) gd_buf<uint32_t>(a, a.c[25])[a.c[26] + k] = id;
            else gd_buf<float>(a, a.c[27])[a.c[28] + k] = wv;
        }
    }
    if (wave == 0u) {  // the ids; the weights are read with the flags
        const bool mine = lane < U;
        uint32_t val = 0;
        for (uint32_t spins = 0;; ++spins) {
            bool ok = true;
            if (mine) {
                const fu_u64 v = fu_ld64(ROUTE + lane);
                val = (uint32_t)v;
                ok = (uint32_t)(v >> 32) == epoch;
            }
            if (__all(ok)) break;
            if (spins >= limit) {
                if (lane == 0) {
                    fu_give_up(CTL, epoch);
                    bad = 1u;
                }
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        if (mine) rid[lane] = val < NE ? val : NE - 1u;
    }
    __syncthreads();

    // ---- (3) loads of this group's gate/up and down rows ---------------------------------
    const uint64_t layer_base = (uint64_t)a.c[14] | ((uint64_t)a.c[15] << 32);
    const uint8_t *LB = reinterpret_cast<const uint8_t *>(layer_base);
    const uint32_t stride = a.c[16], gate_bytes = a.c[17];
    const uint32_t gu_units = U * (F / FB), PU = 2u * FB * nb;  // items per gate/up unit
    const uint32_t dn_units = E / RB, SP = RB * nbF * 2u, PD = U * SP;  // items per down slot and unit
    const uint32_t row_bytes = nb * 34u, drow_bytes = nbF * 34u;
    uint32_t gdw[FU_ITEMS][9], ddw[FU_ITEMS][9];
    bool godd[FU_ITEMS], dodd[FU_ITEMS];
#pragma unroll
    for (int s = 0; s < FU_ITEMS; ++s) {
        const uint32_t j = tid + 512u * (uint32_t)s, i = j / PU, u = g + G * i;
        godd[s] = false;
        if (i < FU_MAX_GUNITS && u < gu_units) {
            const uint32_t idx = j - i * PU, k = u / (F / FB), jj = u - k * (F / FB);
            const uint32_t row = idx / nb, b = idx - row * nb, proj = row / FB, f = FB * jj + (row - proj * FB);
            const uint64_t off = (uint64_t)rid[k] * stride + (proj ? gate_bytes : 0u) + (uint64_t)f * row_bytes + b * 34u;
            fu_load_block(LB, off, gdw[s]);
            godd[s] = (off & 2u) != 0u;
        }
    }
#pragma unroll
    for (int s = 0; s < FU_ITEMS; ++s) {
        const uint32_t j = tid + 512u * (uint32_t)s, i = j / PD, u = g + G * i;
        dodd[s] = false;
        if (i < FU_MAX_DUNITS && u < dn_units) {
            const uint32_t idx = j - i * PD, k = idx / SP, rem = idx - k * SP;
            const uint32_t row = rem / (2u * nbF), blk = (rem - row * 2u * nbF) >> 1;
            const uint64_t off = (uint64_t)rid[k] * stride + 2u * (uint64_t)gate_bytes +
                                 (uint64_t)(RB * u + row) * drow_bytes + blk * 34u;
            fu_load_block(LB, off, ddw[s]);
            dodd[s] = (off & 2u) != 0u;
        }
    }

    // ---- (3) gate/up: block dots, row sums, SwiGLU, ACT ------------------------------------
    const uint32_t *book = reinterpret_cast<const uint32_t *>(book4);
#pragma unroll
    for (int s = 0; s < FU_ITEMS; ++s) {
        const uint32_t j = tid + 512u * (uint32_t)s, i = j / PU, u = g + G * i;
        if (i < FU_MAX_GUNITS && u < gu_units) {
            const uint32_t b = (j - i * PU) % nb;
            uint32_t xs[64];
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                const uint4 v = xh4[b * 16u + (((uint32_t)c + b) & 15u)];
                xs[4 * c] = v.x; xs[4 * c + 1] = v.y; xs[4 * c + 2] = v.z; xs[4 * c + 3] = v.w;
            }
            float sc;
            uint32_t q[8];
            tq2_unpack(gdw[s], godd[s], sc, q);
            gred[j] = sc * tq2_block_dot_h(q, book, xs);
        }
    }
    __syncthreads();
    const uint32_t n_gu = g < gu_units ? (gu_units - g + G - 1u) / G : 0u;  // this group's gate/up units
    const uint32_t ng = n_gu < FU_MAX_GUNITS ? n_gu : FU_MAX_GUNITS;
    if (tid < ng * 2u * FB) {  // row sums in block order, every load issued at once (nb <= 32)
        const uint32_t i = tid / (2u * FB), row = tid - i * 2u * FB;
        const float *src = gred + i * PU + row * nb;
        float acc = 0.f;
#pragma unroll
        for (uint32_t b = 0; b < 32u; ++b) {
            const float v = src[b < nb ? b : nb - 1u];
            acc += b < nb ? v : 0.f;
        }
        gsum[tid] = acc;
    }
    __syncthreads();
    if (tid < ng * FB) {
        const uint32_t i = tid / FB, fr = tid - i * FB, u = g + G * i;
        const uint32_t k = u / (F / FB), f = FB * (u - k * (F / FB)) + fr;
        const float gv = gsum[i * 2u * FB + fr], uv = gsum[i * 2u * FB + FB + fr];
        float v = gd_silu_rcp(gv) * uv;
        if (has_dsigns) v *= gd_buf<const float>(a, a.c[4])[E + f];
        fu_stf(ACT + (size_t)k * F + f, v);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores acknowledged (and its row loads landed)
    __syncthreads();
    if (tid == 0) {
        for (uint32_t i = 0; i < ng; ++i) {
            const uint32_t u = g + G * i, k = u / (F / FB);
            const uint32_t old = __hip_atomic_fetch_add(CNT + 32u * k, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (old + 1u == F / FB) {
                fu_st32(CNT + 32u * k, 0u);
                fu_st32(FLAG + 32u * k, epoch);
            }
        }
    }

    // ---- (4) down: wait for every slot's input, rotate, block dots, output rows ------------
    const uint32_t n_dn = g < dn_units ? (dn_units - g + G - 1u) / G : 0u;
    const uint32_t nd = n_dn < FU_MAX_DUNITS ? n_dn : FU_MAX_DUNITS;
    if (nd == 0u) return;  // uniform: no down unit (the group's counter updates are issued)
    uint32_t tag = 0u;  // wave 0 lane 0: the error tag, read after the flags
    if (wave == 0u) {  // lanes 0 .. U - 1: the slots' flags; lanes 16 .. 16 + U - 1: the route weights
        const bool wl = lane >= 16u && lane < 16u + U;
        uint32_t wbits = 0u;
        for (uint32_t spins = 0;; ++spins) {
            bool ok = true;
            if (lane < U) ok = fu_ld32(FLAG + 32u * lane) == epoch;
            if (wl) {
                const fu_u64 v = fu_ld64(ROUTE + lane);
                wbits = (uint32_t)v;
                ok = (uint32_t)(v >> 32) == epoch;
            }
            if (__all(ok)) break;
            if (spins >= limit) {
                if (lane == 0) {
                    fu_give_up(CTL, epoch);
                    bad = 1u;
                }
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        if (wl) rw[lane - 16u] = gd_bits_f32(wbits);
        if (lane == 0) tag = fu_ld32(CTL + 32u);
    }
    __syncthreads();  // every wave reads ACT after wave 0 saw the flags
    // Slot k, block bb, 16 lanes of 8 values: a = H_128(s_down * silu(g) * u) / sqrt(128).
    for (uint32_t qb = tid >> 4; qb < U * nbF; qb += 32u) {  // whole 16-lane rows
        const uint32_t l16 = lane & 15u, k = qb / nbF, bb = qb - k * nbF;
        const float *src = ACT + (size_t)k * F + bb * 128u + l16 * 8u;
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = fu_ldf(src + j);
        if (has_dsigns) fu_fwht16(v, l16);
        float4 *dst = reinterpret_cast<float4 *>(actr + qb * FU_BLOCK_STRIDE + l16 * 8u);
        dst[0] = make_float4(v[0], v[1], v[2], v[3]);
        dst[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
    if (tid == 0 && tag == epoch) bad = 1u;
    __syncthreads();
#pragma unroll
    for (int s = 0; s < FU_ITEMS; ++s) {
        const uint32_t j = tid + 512u * (uint32_t)s, i = j / PD, u = g + G * i;
        if (i < FU_MAX_DUNITS && u < dn_units) {
            const uint32_t idx = j - i * PD, k = idx / SP, bh = (idx - k * SP) % (2u * nbF);
            const uint32_t blk = bh >> 1, hf = bh & 1u;
            float sc;
            uint32_t q[8];
            tq2_unpack(ddw[s], dodd[s], sc, q);
            dred[j] = sc * tq2_half_dot(q, hf, book, actr + (k * nbF + blk) * FU_BLOCK_STRIDE + 64u * hf);
        }
    }
    __syncthreads();
    // (unit, row, slot): w_k times the sum of the row's half-block dots in (block, half) order,
    // into gred[(i RB + row) U + k] (the host keeps nd RB U <= 2048; 2 F / 128 <= 16 loads at once).
    const uint32_t nbh = 2u * nbF;
    for (uint32_t p = tid; p < nd * RB * U; p += 512u) {
        const uint32_t i = p / (RB * U), rem = p - i * RB * U, row = rem / U, k = rem - row * U;
        const float *d = dred + i * PD + k * SP + row * nbh;
        float dk = 0.f;
#pragma unroll
        for (uint32_t bh = 0; bh < 16u; ++bh) {
            const float v = d[bh < nbh ? bh : nbh - 1u];
            dk += bh < nbh ? v : 0.f;
        }
        gred[p] = rw[k] * dk;
    }
    __syncthreads();
    if (tid < nd * RB) {  // the output row: the slots' terms in slot order, then the residual
        const uint32_t i = tid / RB, row = tid - i * RB, r = RB * (g + G * i) + row;
        const float *pk = gred + (i * RB + row) * U;
        float acc = 0.f;
#pragma unroll
        for (uint32_t k = 0; k < FU_MAX_U; ++k) {
            const float v = pk[k < U ? k : U - 1u];
            acc += k < U ? v : 0.f;
        }
        if (a.c[29]) acc = gd_buf<const float>(a, a.c[30])[a.c[31] + r] + acc;
        gd_buf<float>(a, a.c[12])[a.c[13] + r] = bad ? __builtin_nanf("") : acc;
    }
}
