// Device-side conventions shared by every gyro_native pipeline (gfx950, wave64).
//
// A pipeline is one code object exporting one kernel that takes GdArgs, the `gd_entry` string
// naming that kernel and `gd_workgroup[3]` (GD_PIPELINE_NAMED below). GdArgs
// carries the device table of buffer base pointers and up to 60 32-bit constants, the same
// constant layouts the reference's HLSL kernels read from root constants
// (shaders/engine/common.hlsli:9-14): buffers are named by table index; element offsets count
// 4-byte words unless a kernel says bytes.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

struct GdArgs {
    const uint64_t *table;
    uint32_t c[60];
};

// Defines the pipeline's kernel `NAME`, its workgroup size and the `gd_entry` string through
// which gd_create_pipeline finds the kernel (so profilers show each pipeline by name).
#define GD_PIPELINE_NAMED(NAME, WG)                                        \
    extern "C" __constant__ uint32_t gd_workgroup[3] = {WG, 1, 1};        \
    extern "C" __constant__ char gd_entry[32] = #NAME;                     \
    extern "C" __global__ __launch_bounds__(WG) void NAME(const GdArgs a)
#define GD_PIPELINE(WG) GD_PIPELINE_NAMED(gd_main, WG)
// As GD_PIPELINE_NAMED, asking the compiler to fit WAVES waves per SIMD (registers included).
#define GD_PIPELINE_NAMED_OCC(NAME, WG, WAVES)                             \
    extern "C" __constant__ uint32_t gd_workgroup[3] = {WG, 1, 1};        \
    extern "C" __constant__ char gd_entry[32] = #NAME;                     \
    extern "C" __global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(WAVES, WAVES))) void NAME(const GdArgs a)

template <typename T>
__device__ __forceinline__ T *gd_buf(const GdArgs &a, uint32_t index) {
    return reinterpret_cast<T *>(a.table[index]);
}

__device__ __forceinline__ float gd_bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ uint32_t gd_f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }

// binary16 -> binary32 through the hardware conversion (exact for every finite value; the
// fp16 denormal mode is IEEE on gfx950).
__device__ __forceinline__ float gd_half(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// binary16 -> binary32 in integer arithmetic, the normative conversion of src/gyro.zig:127-141.
__device__ __forceinline__ float gd_half_exact(uint32_t h) {
    uint32_t sign = (h & 0x8000u) << 16;
    uint32_t exponent = (h >> 10) & 31u;
    uint32_t mantissa = h & 1023u;
    if (exponent == 31u) return gd_bits_f32(sign | 0x7f800000u | (mantissa << 13));
    if (exponent != 0u) return gd_bits_f32(sign | ((exponent + 112u) << 23) | (mantissa << 13));
    if (mantissa == 0u) return gd_bits_f32(sign);
    // Subnormal: shift the leading one into bit 10 (clz of a value below 1024).
    uint32_t shift = __builtin_clz(mantissa) - 21u;
    mantissa <<= shift;
    return gd_bits_f32(sign | ((113u - shift) << 23) | ((mantissa & 1023u) << 13));
}

__device__ __forceinline__ float gd_silu(float x) { return x / (1.0f + __expf(-x)); }
__device__ __forceinline__ float gd_sigmoid(float x) { return 1.0f / (1.0f + __expf(-x)); }
__device__ __forceinline__ float gd_silu_accurate(float x) { return x / (1.0f + expf(-x)); }
// silu through the hardware reciprocal (v_rcp_f32, about 1 ulp) instead of an IEEE division;
// for results rounded to binary16 afterwards.
__device__ __forceinline__ float gd_silu_rcp(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
__device__ __forceinline__ float gd_sigmoid_accurate(float x) { return 1.0f / (1.0f + expf(-x)); }

// Gyro type table, src/gyro.zig:32-41: k (new bits per step), steps, block bytes.
struct GyroType {
    uint32_t k, steps, block_bytes;
};
__device__ __forceinline__ bool gd_type(uint32_t id, GyroType &t) {
    switch (id) {
        case 144: t = {8, 32, 34}; return true;
        case 145: t = {6, 32, 26}; return true;
        case 146: t = {7, 32, 30}; return true;
        case 147: t = {5, 64, 42}; return true;
        case 148: t = {6, 64, 50}; return true;
        case 149: t = {7, 64, 58}; return true;
        case 150: t = {5, 32, 22}; return true;
        case 151: t = {4, 32, 18}; return true;
        default: t = {0, 0, 0}; return false;
    }
}

// 16-bit trellis state of a step (src/gyro.zig:107-117) read from a byte stream.
__device__ __forceinline__ uint32_t gd_state(const uint8_t *stream, const GyroType &t, uint32_t id,
                                             uint32_t step) {
    if (id == 144u) return ((uint32_t)stream[(step + 31u) & 31u] << 8) | stream[step];
    uint32_t len = t.steps * t.k / 8u;
    uint32_t off = (t.steps - 1u - step) * t.k;
    uint32_t byte = off >> 3;
    uint32_t b1 = byte + 1u >= len ? byte + 1u - len : byte + 1u;
    uint32_t b2 = byte + 2u >= len ? byte + 2u - len : byte + 2u;
    uint32_t word = (uint32_t)stream[byte] | ((uint32_t)stream[b1] << 8) | ((uint32_t)stream[b2] << 16);
    return (word >> (off & 7u)) & 0xffffu;
}

// Multiplicative hash of SPEC section 5: one product serves both codebook indices.
__device__ __forceinline__ uint32_t gd_hash(uint32_t state) { return (state & 0x7fffu) * 0x9e3779b1u; }

// Wave64 reductions.
__device__ __forceinline__ float gd_wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float gd_wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
// Wave64 sum with DPP (no LDS traffic, so no wait on outstanding loads): row prefix sums by
// row_shr 1, 2, 4, 8, then row_bcast 15 and 31 carry rows 0..2 into lane 63, which every lane
// reads (a scalar). A fixed order: the same inputs give the same sum.
template <int CTRL, int ROWS>
__device__ __forceinline__ float gd_dpp_add_step(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xf, false));
}
__device__ __forceinline__ float gd_wave_sum_dpp(float v) {
    v = gd_dpp_add_step<0x111, 0xf>(v);  // row_shr:1
    v = gd_dpp_add_step<0x112, 0xf>(v);  // row_shr:2
    v = gd_dpp_add_step<0x114, 0xf>(v);  // row_shr:4
    v = gd_dpp_add_step<0x118, 0xf>(v);  // row_shr:8
    v = gd_dpp_add_step<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    v = gd_dpp_add_step<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Inclusive prefix sum of 32-bit integers over the wave's 64 lanes (lane i gets the sum of lanes
// 0 .. i), by the DPP steps of gd_wave_sum_dpp: no LDS traffic.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t gd_dpp_add_step_u32(uint32_t v) {
    return v + (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xf, false);
}
__device__ __forceinline__ uint32_t gd_wave_scan_u32(uint32_t v) {
    v = gd_dpp_add_step_u32<0x111, 0xf>(v);  // row_shr:1
    v = gd_dpp_add_step_u32<0x112, 0xf>(v);  // row_shr:2
    v = gd_dpp_add_step_u32<0x114, 0xf>(v);  // row_shr:4
    v = gd_dpp_add_step_u32<0x118, 0xf>(v);  // row_shr:8: prefix sums within rows of 16
    v = gd_dpp_add_step_u32<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    v = gd_dpp_add_step_u32<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}

// Global-address-space views of table buffers. Loads through them are global_load, counted by
// vmcnt only (a flat load also counts against lgkmcnt), so an LDS-only wait leaves them in flight.
typedef uint32_t gd_u32x4 __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) uint32_t gd_guint;
typedef const __attribute__((address_space(1))) gd_u32x4 gd_gu32x4;
__device__ __forceinline__ gd_guint *gd_global(const uint32_t *p) { return (gd_guint *)(uintptr_t)p; }
__device__ __forceinline__ gd_gu32x4 *gd_global4(const uint32_t *p) { return (gd_gu32x4 *)(uintptr_t)p; }

// Workgroup barrier that waits for this wave's LDS (and scalar) traffic only, so global loads
// issued before it stay in flight; the memory clobber keeps the compiler from moving LDS
// accesses across it.
__device__ __forceinline__ void gd_lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// v as rounded to fp32, opaque to the compiler: a product passed through it is not fused with a
// later add. (Under fp-contract=fast the compiler may turn `v = a * b; v + w` into fma(a, b, w)
// in one build of a kernel and not in another, which changes the last bits of the sum.)
__device__ __forceinline__ float gd_rounded(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

// Activation range guard: an activation rounded to binary16 must be finite and at most 65504 in
// magnitude (false for NaN and infinities). A kernel that rounds one outside stores 1 to the
// flag word at table index `flag` (0: no flag); the host reads it and recomputes on the fp32 path.
__device__ __forceinline__ bool gd_half_ok(float v) { return __builtin_fabsf(v) <= 65504.0f; }
__device__ __forceinline__ void gd_range_flag(const uint64_t *table, uint32_t flag, bool bad) {
    if (flag && bad) reinterpret_cast<uint32_t *>(table[flag])[0] = 1u;
}

// XCD-aware order of the x groups of a grid: the dispatcher hands workgroup i (linear id) to
// XCD i % 8, so logical index (i % 8) (G / 8) + i / 8 gives each XCD a contiguous run of G / 8
// groups and neighbouring groups, which share the cache lines at their edges, one L2. A grid
// whose x size G is a multiple of 8 keeps the property for every row y (linear id x + y G).
// Identity when G % 8 != 0.
__device__ __forceinline__ uint32_t gd_xcd_group(uint32_t x, uint32_t G) {
    return (G & 7u) ? x : (x & 7u) * (G >> 3) + (x >> 3);
}

// 1 / sqrt(128) rounded to binary32, the normalisation of a 128-point Walsh-Hadamard block.
#define GD_INV_SQRT128 0.0883883461356163f
