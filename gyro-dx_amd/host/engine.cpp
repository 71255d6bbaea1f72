// MoE layer engine above the gyro_native ABI: resident experts in slot arenas, the reference
// dispatch sequence of src/gpu_engine.zig:1052-1119, and the MI355X decode and grouped-GEMM
// paths. C entry points are declared in include/gyro_moe.h.
//
// This file is compiled as HIP source for one reason: it defines the device array `scratch`
// that the no-allocation decode entry point (gm_forward_decode_noalloc) uses for its
// intermediate buffers. Every kernel still comes from the pipelines in the kernel directory.
#include <dirent.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <initializer_list>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "device.h"
#include "gyro_moe.h"

// Intermediate buffers of gm_forward_decode_noalloc: router logits, routes, the rotated input,
// the gate/up partials and the shared expert's rows. One copy per GPU, alive until the process
// ends; every no-allocation call on a GPU shares it, so calls that overlap on one GPU race.
static __device__ __align__(256) uint8_t scratch[GM_NOALLOC_SCRATCH_BYTES];

namespace gyro {
namespace {

// src/gyro.zig:32-41.
uint32_t block_bytes_of(uint32_t type_id) {
    switch (type_id) {
        case 144: return 34;
        case 145: return 26;
        case 146: return 30;
        case 147: return 42;
        case 148: return 50;
        case 149: return 58;
        case 150: return 22;
        case 151: return 18;
        default: return 0;
    }
}

uint32_t bits(float v) {
    uint32_t u;
    std::memcpy(&u, &v, 4);
    return u;
}

constexpr uint32_t kNone = 0xffffffffu;
constexpr uint64_t kArenaLimit = 2ull << 30;  // src/gpu_engine.zig:601
constexpr uint32_t kMaxArenas = 8;            // src/gpu_engine.zig:617
constexpr uint32_t kStagingBytes = 32u << 20;

struct ExpertDesc {
    uint64_t gate, up, down;
    uint32_t types;
    uint32_t pad;
};
static_assert(sizeof(ExpertDesc) == 32, "expert descriptor layout");

struct Layer {
    Buffer router, bias, signs, xtab;
    Buffer router16;  // the router rows split into binary16 pairs for moe_prefill_router
    bool has_bias = false, has_gate_signs = false, has_down_signs = false;
    float scale = 0;
    uint32_t type_id = 0;     // uniform Gyro type, 0 when projections mix types
    uint32_t gate_bytes = 0;  // per projection, uniform types only
    uint64_t base = 0;        // device address of expert 0's bundle; expert e at base + e * stride
    float max_scale = 0;      // largest |block scale| over the layer's experts
    uint32_t SF = 0;          // shared expert width (0: none)
    uint32_t sh_kind = GM_SHARED_BF16;  // row format of the shared matrices on the device
    uint32_t sh_row_e = 0, sh_row_f = 0;  // device row bytes of the gate/up rows (E columns), down rows (SF)
    Buffer sh_gu, sh_down, sh_gate;  // [2 SF] rows (gate, then up), [E] rows, in the mv kernels' format; fp32 [E]
    Buffer sh_gu16, sh_down16;       // binary16 copies x 2^k per matrix (prefill path)
    float sh_unscale[3] = {1, 1, 1}; // 2^-k of the gate, up and down copies
    Buffer norm;                     // fp32 [E] RMSNorm weight of the layer's input in a stack
    bool has_norm = false;
    float norm_eps = 0;
};

// binary16 -> float for host-side range checks.
float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 31u, man = h & 1023u;
    uint32_t u;
    if (exp == 31u) u = sign | 0x7f800000u | (man << 13);
    else if (exp) u = sign | ((exp + 112u) << 23) | (man << 13);
    else {
        float f = std::ldexp((float)man, -24);
        return sign ? -f : f;
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// Largest |scale| of the Gyro blocks (bb bytes each, the scale in the first two) in `bytes`
// bytes of packed rows; a NaN scale reads as infinite.
float max_block_scale(const uint8_t *p, uint64_t bytes, uint32_t bb) {
    float m = 0;
    for (uint64_t off = 0; off + bb <= bytes; off += bb) {
        uint16_t h;
        std::memcpy(&h, p + off, 2);
        const float v = std::fabs(half_to_float(h));
        if (v != v) return INFINITY;
        m = std::max(m, v);
    }
    return m;
}

float bf16_to_float(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// float -> binary16, round to nearest even (subnormals included; overflow to infinity).
uint16_t float_to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    x &= 0x7fffffffu;
    if (x >= 0x7f800000u) return sign | 0x7c00u | (x > 0x7f800000u ? 0x200u : 0u);
    const int e = (int)(x >> 23) - 127;
    if (e < -14) {  // subnormal binary16: units of 2^-24
        const double q = std::nearbyint((double)std::fabs(f) * 16777216.0);  // ties to even
        return sign | (uint16_t)q;  // q == 1024 is the smallest normal, same bits
    }
    uint32_t m = (x & 0x7fffffu) | 0x800000u, r = m >> 13;
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    int eb = e + 15;
    if (r == 0x800u) {
        r = 0x400u;
        ++eb;
    }
    if (eb >= 31) return sign | 0x7c00u;
    return sign | (uint16_t)(eb << 10) | (uint16_t)(r & 0x3ffu);
}

// Binary16 copy of n fp32 values times 2^k, k chosen so that the largest finite |value| lands in
// [2^14, 2^15): every bf16 value whose scaled magnitude is a normal binary16 converts exactly (bf16
// carries 8 significant bits, binary16 11); Q8_0 and fp32 weights round to nearest even.
// Returns 2^-k.
float floats_to_scaled_half(const float *src, size_t n, std::vector<uint16_t> &dst) {
    float mx = 0;
    for (size_t i = 0; i < n; ++i) {
        const float v = std::fabs(src[i]);
        if (v == v && v != INFINITY) mx = std::max(mx, v);
    }
    int ex = 0;
    if (mx > 0) std::frexp(mx, &ex);  // mx < 2^ex
    const int k = mx > 0 ? 15 - ex : 0;
    dst.resize(n);
    for (size_t i = 0; i < n; ++i) dst[i] = float_to_half(std::ldexp(src[i], k));
    return std::ldexp(1.0f, -k);
}

// The router rows as moe_prefill_router takes them: row r scaled by 2^k_r, k_r chosen so that its
// largest finite |weight| lands in [2^14, 2^15), and each scaled value v carried as hi = f16(v)
// and lo = f16((v - hi) 2^11) (round to nearest even; v - hi is exact). Row r, chunk c (k = 16 c
// .. 16 c + 15) takes words 16 (r E / 16 + c) ..: the 16 hi values, then the 16 lo values; after
// the NE x E words come the NE factors 2^-k_r.
std::vector<uint32_t> split_router_rows(const float *w, uint32_t NE, uint32_t E) {
    std::vector<uint32_t> out((size_t)NE * E + NE);
    uint16_t *h = reinterpret_cast<uint16_t *>(out.data());
    for (uint32_t r = 0; r < NE; ++r) {
        const float *row = w + (size_t)r * E;
        float mx = 0;
        for (uint32_t k = 0; k < E; ++k) {
            const float v = std::fabs(row[k]);
            if (v == v && v != INFINITY) mx = std::max(mx, v);
        }
        int ex = 0;
        if (mx > 0) std::frexp(mx, &ex);  // mx < 2^ex
        const int kr = mx > 0 ? 15 - ex : 0;
        for (uint32_t k = 0; k < E; ++k) {
            const float v = std::ldexp(row[k], kr);
            const uint16_t hi = float_to_half(v);
            const uint16_t lo = float_to_half((v - half_to_float(hi)) * 2048.0f);
            const size_t at = ((size_t)r * E + (k & ~15u)) * 2 + (k & 15u);
            h[at] = hi;
            h[at + 16] = lo;
        }
        const float unscale = std::ldexp(1.0f, -kr);
        std::memcpy(&out[(size_t)NE * E + r], &unscale, 4);
    }
    return out;
}

// Shared-expert row formats: bytes of a source row of `cols` values (as gm_layer_desc gives it)
// and of a device row (what mv_bf16 / mv_q8 / mv_f32 read; Q8_0 repacked by q8_repack).
uint64_t shared_src_row(uint32_t kind, uint64_t cols) {
    return kind == GM_SHARED_Q8_0 ? cols / 32 * 34 : kind == GM_SHARED_F32 ? cols * 4 : cols * 2;
}
uint64_t shared_dev_row(uint32_t kind, uint64_t cols) {
    return kind == GM_SHARED_Q8_0 ? cols + cols / 16 : kind == GM_SHARED_F32 ? cols * 4 : cols * 2;
}
// fp32 values of rows x cols source rows of a shared matrix (Q8_0: d * q, exact in fp32).
void shared_to_floats(uint32_t kind, const void *src, uint64_t rows, uint64_t cols, std::vector<float> &out) {
    out.resize(rows * cols);
    const uint8_t *p = static_cast<const uint8_t *>(src);
    for (uint64_t r = 0; r < rows; ++r) {
        const uint8_t *row = p + r * shared_src_row(kind, cols);
        float *o = out.data() + r * cols;
        if (kind == GM_SHARED_F32) {
            std::memcpy(o, row, cols * 4);
        } else if (kind == GM_SHARED_BF16) {
            for (uint64_t i = 0; i < cols; ++i) {
                uint16_t b;
                std::memcpy(&b, row + 2 * i, 2);
                o[i] = bf16_to_float(b);
            }
        } else {
            for (uint64_t blk = 0; blk < cols / 32; ++blk) {
                uint16_t h;
                std::memcpy(&h, row + blk * 34, 2);
                const float dscale = half_to_float(h);
                for (uint64_t j = 0; j < 32; ++j) o[blk * 32 + j] = dscale * (float)(int8_t)row[blk * 34 + 2 + j];
            }
        }
    }
}

std::vector<uint8_t> read_file(const std::string &path) {
    std::ifstream f(path, std::ios::binary);
    return std::vector<uint8_t>((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
}

// Device address of `scratch` on each GPU, looked up once per device with that device current.
// In host code the array's name is only a stand-in for the symbol; kernels get this address.
constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
void *scratch_ptr[kMaxDevices] = {};

void *scratch_address(uint32_t device) {
    if (device >= (uint32_t)kMaxDevices) throw NativeError(-1, "device ordinal out of range for the scratch table");
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (!scratch_ptr[device]) {
        hipError_t rc = hipSetDevice((int)device);
        if (rc != hipSuccess) throw NativeError(-1, std::string("hipSetDevice: ") + hipGetErrorString(rc));
        void *p = nullptr;
        rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (rc != hipSuccess || !p)
            throw NativeError(-1, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(rc));
        scratch_ptr[device] = p;
    }
    return scratch_ptr[device];
}

// Fixed regions of the scratch array: the shared expert's rows (n <= 8 tokens x 2 SF <= 2048
// floats) and gate dots come first, at their own table entries (moe_router takes them without
// an offset); the per-call buffers follow from kNoallocBase.
constexpr uint64_t kNoallocShH = 0, kNoallocShHBytes = 64u << 10;
constexpr uint64_t kNoallocShG = kNoallocShHBytes, kNoallocShGBytes = 256;

constexpr uint64_t kNoallocBase = 128u << 10;
static_assert(kNoallocShG + kNoallocShGBytes <= kNoallocBase, "scratch regions overlap");

}  // namespace

// Table indices and word offsets of the shared expert's intermediate buffers: the gate and up
// rows h [n][2 SF], the SwiGLU a [n][SF], the output o [n][E], the gate dots g [n] and, on the
// decode path, the gated output s [n][E].
struct SharedBufs {
    uint32_t h, h_off, a, a_off, o, o_off, g, g_off, s, s_off;
};

// Table indices (and word offsets) of the intermediate buffers of the decode path.
struct DecodeBufs {
    uint32_t logits, logits_off, ids, ids_off, weights, weights_off, xh, xh_off, gu, gu_off;
    uint32_t sh_h, sh_g;  // the fused shared expert's rows and gate dots (offset 0)
    SharedBufs shared;    // the shared expert outside the fused kernels
};

// Residual stream of a stack step: the layer input is normalised by the layer's RMSNorm inside
// the path's first kernel, and the path's last kernel adds res to its output.
struct StackStep {
    bool on = false;
    uint32_t res_uav = kNone, res_off = 0;
};

// The next layer's RMSNorm, computed by the prefill combine of a stack (moe_prefill_combine_norm):
// its weight (kNone: none) and eps; the normalised rows go to the engine's `hn`.
struct NormNext {
    uint32_t w_srv = kNone, eps_bits = 0;
};

class Engine {
  public:
    Device dev;
    std::map<std::string, gd_pipeline *, std::less<>> pipes;
    // Direct launches (no recording) on a caller's stream, for gm_forward_decode_noalloc.
    bool direct = false;
    void *direct_stream = nullptr;
    Buffer na_base, na_shh, na_shg, na_x, na_out;  // table entries into `scratch` and for the caller's x, out
    // Compute units of the device (the persistent GEMM's two groups per unit, the decode
    // kernels' target group count).
    uint32_t cus = 0;
    // Prefill GEMMs: one persistent launch over both (moe_prefill_gemm for uniform TQ2_T layers,
    // moe_prefill_gemm_x for the others) unless the environment sets GYRO_PREFILL_FUSED=0 (then
    // moe_prefill_gu and moe_prefill_down, or moe_prefill_gu_x and moe_prefill_down_x);
    // the polls a down unit makes for a ready tile before it gives up (GYRO_PREFILL_SPIN_LIMIT,
    // default 2^20); its queue words, give-up word, tile counters and ready list.
    bool prefill_fused = true;
    uint32_t prefill_spin_limit = 1u << 20;
    // The persistent GEMM with the small-tile units (moe_prefill_gemm_s: tiles of at most 16 rows,
    // 8 past hidden 2048; hidden and F multiples of 512) for calls whose expert segments average at
    // most 8 slots (n n_used <= 8 n_expert), where most tiles are small; the small units' code costs
    // the other units 3-5% (register allocation), so larger calls take moe_prefill_gemm. The
    // environment's GYRO_PREFILL_SMALL: 0 never, 2 always (where the shape allows), else that rule.
    uint32_t prefill_small = 1;
    // Stack prefill: the combine also computes the next layer's RMSNorm (environment's
    // GYRO_STACK_NORM_FUSED=0: moe_stack_norm before every layer instead).
    bool stack_norm_fused = true;
    // The prefill router's K split doubles while its groups stay within this count (the
    // environment's GYRO_ROUTER_GROUPS overrides it). One group per CU (96 KB of LDS each)
    // measured best: splits that give 512 or 1024 groups were slower at 256 and 1024 tokens.
    uint32_t router_groups = 256;
    // Calls of at least this many tokens take the wide router build (moe_prefill_router_w: 32
    // tokens x 256 experts per group, each wave two 32-expert tiles over its group's whole K
    // range), which stages a quarter fewer bytes per logit and needs a quarter of the groups; the
    // environment's GYRO_ROUTER_WIDE_MIN overrides it (0: never).
    uint32_t router_wide_min = 2048;
    uint32_t small_rows() const {
        if (E % 512 || F % 512) return 0;
        return E <= 2048 ? 16u : (E <= 4096 ? 8u : 0u);
    }
    bool use_small(uint32_t n) const {
        if (!prefill_small || !small_rows()) return false;
        return prefill_small == 2 || n * U <= 8 * NE;
    }
    Buffer gemm_sched;
    static constexpr uint32_t kSchedWords = 64;  // words before the tile counters and the ready list
    std::string error;
    uint32_t max_tok = 0;
    uint32_t E = 0, F = 0, NE = 0, U = 0;
    std::vector<Layer> layers;
    // Expert arenas (src/gpu_engine.zig:593-650).
    std::vector<Buffer> arenas;
    uint32_t slot_stride = 0, per_arena = 0, used_slots = 0;
    Buffer lookup;
    // Shared buffers.
    Buffer staging, codebook, zeros;
    Buffer x_in, router_out, ids, weights, table, xh, gu, gu_part, act, down, out;
    Buffer order, meta;  // prefill: sorted slots; segment starts, tile count and tile list
    // Prefill: per chunk of 256 slots, the slots that chose each expert ([chunk][n_expert]; the
    // router zeroes it, the top-k counts into it, the sort places each chunk from it).
    Buffer hist;
    static constexpr uint32_t kSortChunk = 256;
    uint32_t hist_words(uint32_t n) const { return (n * U + kSortChunk - 1) / kSortChunk * NE; }
    // Activation range guard: word 0 of range_flag (set by moe_prefill_router and
    // moe_prefill_shared) and word kMetaRangeFlag of meta (set by the prefill gate/up GEMMs) become
    // 1 when an activation rounded to binary16 is outside its range.
    Buffer range_flag;
    static constexpr uint32_t kMetaRangeFlag = 1022;
    Buffer sh_h, sh_a, sh_o, sh_g;  // shared expert: [T][2 SF], [T][SF], [T][E], [T]
    Buffer sh_s;                    // decode path: sigmoid(g . x) * shared output (+ stream) [T][E]
    Buffer x16;                     // prefill shared expert: the unrotated input [T][E] binary16
    uint32_t sh_width = 0;          // SF the shared buffers are sized for
    Buffer tokens, outputs;
    Buffer hn;  // stack: the normalised input of the current layer [T][E]
    uint32_t n_tokens = 0;
    uint32_t parts = 0;
    float max_codebook = 0;  // largest |codebook value|
    static constexpr uint32_t kTileRows = 128;

    gd_pipeline *pipe(const char *name) {
        auto it = pipes.find(name);
        if (it == pipes.end()) throw NativeError(-1, std::string("pipeline missing: ") + name);
        return it->second;
    }

    void dispatch_words(const char *name, const uint32_t *c, uint32_t count, uint32_t x, uint32_t y, uint32_t z) {
        if (direct)
            check(gd_dispatch_on(dev.ctx, pipe(name), c, count, x, y, z, direct_stream), "gd_dispatch_on");
        else
            dev.dispatch(pipe(name), c, count, x, y, z);
    }
    void dispatch(const char *name, const std::vector<uint32_t> &c, uint32_t x, uint32_t y = 1, uint32_t z = 1) {
        dispatch_words(name, c.data(), (uint32_t)c.size(), x, y, z);
    }
    void dispatch(const char *name, std::initializer_list<uint32_t> c, uint32_t x, uint32_t y = 1, uint32_t z = 1) {
        dispatch_words(name, c.begin(), (uint32_t)c.size(), x, y, z);
    }

    // Dispatch that records its own start and end timestamps when `timed` is set (their
    // indices are appended to marks).
    void dispatch_maybe_timed(bool timed, std::vector<uint32_t> *marks, const char *name,
                              std::initializer_list<uint32_t> c, uint32_t x, uint32_t y = 1, uint32_t z = 1) {
        if (timed && marks) {
            const uint32_t first = dev.dispatch_timed(pipe(name), c.begin(), (uint32_t)c.size(), x, y, z);
            marks->push_back(first);
            marks->push_back(first + 1);
        } else {
            dispatch(name, c, x, y, z);
        }
    }

    void load_kernels(const std::string &dir) {
        DIR *d = opendir(dir.c_str());
        if (!d) throw NativeError(-1, "kernel directory not found: " + dir);
        while (dirent *ent = readdir(d)) {
            std::string name = ent->d_name;
            if (name.size() > 3 && name.compare(name.size() - 3, 3, ".co") == 0) {
                std::vector<uint8_t> code = read_file(dir + "/" + name);
                pipes[name.substr(0, name.size() - 3)] = dev.pipeline(code);
            }
        }
        closedir(d);
    }

    // Copies host bytes into a device buffer through the mapped staging buffer and the
    // bit-exact copy of the elementwise pipeline (as src/gpu_engine.zig:447-461 uploads the
    // codebook).
    void upload(const Buffer &dst, uint64_t dst_off, const void *src, uint64_t bytes) {
        if (bytes % 4 || dst_off % 4) throw NativeError(-1, "upload must be word aligned");
        const uint8_t *s = static_cast<const uint8_t *>(src);
        while (bytes) {
            const uint64_t chunk = std::min<uint64_t>(bytes, kStagingBytes);
            std::memcpy(staging.mapped, s, chunk);
            const uint32_t words = (uint32_t)(chunk / 4);
            dev.begin();
            dispatch("ew", {staging.uav, 0, 0, staging.uav, 0, 0, dst.uav, (uint32_t)(dst_off / 4), 0, words, 1, 5},
                     (words + 255) / 256);
            dev.wait(dev.submit());
            s += chunk;
            dst_off += chunk;
            bytes -= chunk;
        }
    }

    void fill_zero(const Buffer &dst) {
        const uint32_t words = (uint32_t)(dst.bytes / 4);
        uint32_t done = 0;
        dev.begin();
        while (done < words) {
            const uint32_t n = std::min<uint32_t>(words - done, 1u << 16);
            // y = a + b over a zero host row: the zero-filled staging buffer head.
            dispatch("ew", {zeros.uav, 0, 0, zeros.uav, 0, 0, dst.uav, done, 0, n, 1, 5}, (n + 255) / 256);
            done += n;
        }
        dev.wait(dev.submit());
    }

    void create(const std::string &kernel_dir, uint32_t adapter, uint32_t tokens_per_call) {
        max_tok = tokens_per_call;
        dev.init(adapter);
        load_kernels(kernel_dir);
        staging = dev.buffer(kStagingBytes, Kind::host);
        zeros = dev.buffer(1u << 18, Kind::host);  // stays zero: the source of fills
        codebook = dev.buffer(8192, Kind::device);
        std::vector<uint8_t> book = read_file(kernel_dir + "/../../data/gyro_codebook.f16");
        if (book.size() != 8192) throw NativeError(-1, "codebook must hold 8192 bytes");
        upload(codebook, 0, book.data(), 8192);
        for (uint32_t i = 0; i < 4096; ++i) {
            uint16_t h;
            std::memcpy(&h, book.data() + 2 * i, 2);
            max_codebook = std::max(max_codebook, std::fabs(half_to_float(h)));
        }
        range_flag = dev.buffer(256, Kind::device);
        fill_zero(range_flag);
        // Table entries of the no-allocation entry point: into this GPU's scratch array, and two
        // whose addresses each call sets (the caller's input and output).
        uint8_t *sp = static_cast<uint8_t *>(scratch_address(adapter));
        na_base = dev.wrap(sp, GM_NOALLOC_SCRATCH_BYTES);
        na_shh = dev.wrap(sp + kNoallocShH, kNoallocShHBytes);
        na_shg = dev.wrap(sp + kNoallocShG, kNoallocShGBytes);
        na_x = dev.wrap(nullptr, 0);
        na_out = dev.wrap(nullptr, 0);
        int cu = 0;
        if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, (int)adapter) != hipSuccess) cu = 0;
        cus = (uint32_t)std::max(cu, 0);
        const char *pf = std::getenv("GYRO_PREFILL_FUSED");
        prefill_fused = !(pf && pf[0] == '0');
        const char *psm = std::getenv("GYRO_PREFILL_SMALL");
        prefill_small = psm && psm[0] == '0' ? 0u : (psm && psm[0] == '2' ? 2u : 1u);
        const char *snf = std::getenv("GYRO_STACK_NORM_FUSED");
        stack_norm_fused = !(snf && snf[0] == '0');
        if (const char *ps = std::getenv("GYRO_PREFILL_SPIN_LIMIT"))
            prefill_spin_limit = (uint32_t)std::strtoul(ps, nullptr, 10);
        if (const char *rg = std::getenv("GYRO_ROUTER_GROUPS"))
            router_groups = std::max(1u, (uint32_t)std::strtoul(rg, nullptr, 10));
        if (const char *rw = std::getenv("GYRO_ROUTER_WIDE_MIN"))
            router_wide_min = (uint32_t)std::strtoul(rw, nullptr, 10);
    }

    // The decode path's own intermediate buffers.
    DecodeBufs engine_bufs() const {
        return {router_out.uav, 0, ids.uav, 0, weights.uav, 0, xh.uav, 0, gu_part.uav, 0, sh_h.uav, sh_g.uav,
                engine_shared()};
    }

    void allocate_activations() {
        const uint64_t T = max_tok, f = 4;
        x_in = dev.buffer(T * E * f, Kind::device);
        router_out = dev.buffer(2 * T * NE * f, Kind::device);  // two logit planes of max_tok rows
        ids = dev.buffer(T * U * 4, Kind::device);
        weights = dev.buffer(T * U * f, Kind::device);
        table = dev.buffer(T * U * 24, Kind::device);
        xh = dev.buffer(T * E * f, Kind::device);
        gu = dev.buffer(T * U * 2 * F * f, Kind::device);
        parts = (E + 1023) / 1024;  // K-parts of up to 8 blocks of the decode gate/up kernels
        gu_part = dev.buffer(parts * T * U * 2 * F * f, Kind::device);
        act = dev.buffer(T * U * F * f, Kind::device);
        down = dev.buffer(T * U * E * f, Kind::device);
        out = dev.buffer(T * E * f, Kind::device);
        hn = dev.buffer(T * E * f, Kind::device);
        order = dev.buffer(T * U * 4, Kind::device);
        hist = dev.buffer((uint64_t)hist_words(std::min<uint32_t>(max_tok, 32768u / U + 1u)) * 4, Kind::device);
        fill_zero(hist);
        meta = dev.buffer((1024 + 4ull * max_tiles(max_tok)) * 4, Kind::device);
        fill_zero(meta);
        gemm_sched = dev.buffer((kSchedWords + 2ull * max_tiles(max_tok)) * 4ull, Kind::device);
        fill_zero(gemm_sched);
        // The shared-expert inputs of moe_combine: zero output and gate (sigmoid(0) * 0 = 0).
        Buffer z = dev.buffer(T * E * f, Kind::device);
        fill_zero(z);
        sh_zero = z;
    }
    Buffer sh_zero;

    // Upper bound of the sort's tile count for n tokens: every non-empty expert segment
    // adds at most one partial tile.
    uint32_t max_tiles(uint32_t n) const {
        return (n * U + kTileRows - 1) / kTileRows + std::min(NE, n * U);
    }

    // q8_repack of rows x cols GGUF Q8_0 rows at the start of src into dst (row_bytes per row).
    void repack_q8(const Buffer &src, uint64_t rows, uint64_t cols, const Buffer &dst, uint32_t row_bytes) {
        const uint64_t blocks = rows * (cols / 32);
        const uint32_t groups = (uint32_t)((blocks + 255) / 256);
        dev.begin();
        dispatch("q8_repack", {src.srv, 0, (uint32_t)rows, (uint32_t)cols, 0, 0, 0, 0, dst.uav, 0, 0, 0, 0, 0, row_bytes, 0},
                 std::min(groups, 65535u), (groups + 65534) / 65535);
        dev.wait(dev.submit());
    }

    uint32_t add_layer(const gm_layer_desc &d) {
        if (layers.empty()) {
            E = d.E; F = d.F; NE = d.n_expert; U = d.n_used;
            if (!E || !F || E % 128 || F % 128 || NE == 0 || NE > 512 || U == 0 || U > 16 || U > NE)
                throw NativeError(-1, "unsupported layer shape");
            allocate_activations();
        } else if (d.E != E || d.F != F || d.n_expert != NE || d.n_used != U) {
            throw NativeError(-1, "layers of one engine must share their shape");
        }
        const uint32_t il = (uint32_t)layers.size();
        Layer L;
        L.scale = d.expert_weights_scale;
        // Per-expert projection sizes and the slot stride (256-byte aligned bundles).
        std::vector<uint64_t> gb(NE), ub(NE), db(NE);
        uint64_t max_bundle = 0;
        bool uniform = true;
        for (uint32_t e = 0; e < NE; ++e) {
            const uint32_t tg = d.types[e * 3], tu = d.types[e * 3 + 1], td = d.types[e * 3 + 2];
            if (!block_bytes_of(tg) || !block_bytes_of(tu) || !block_bytes_of(td))
                throw NativeError(-1, "unsupported Gyro type");
            gb[e] = (uint64_t)F * (E / 128) * block_bytes_of(tg);
            ub[e] = (uint64_t)F * (E / 128) * block_bytes_of(tu);
            db[e] = (uint64_t)E * (F / 128) * block_bytes_of(td);
            max_bundle = std::max(max_bundle, gb[e] + ub[e] + db[e]);
            if (tg != d.types[0] || tu != d.types[0] || td != d.types[0]) uniform = false;
        }
        L.type_id = uniform ? d.types[0] : 0;
        L.gate_bytes = uniform ? (uint32_t)gb[0] : 0;
        if (!slot_stride) {
            // A first layer that mixes Gyro types reserves the bundle of the largest type, so
            // that later mixed layers fit the same slots; a uniform first layer fixes the stride
            // at its own bundle.
            uint64_t stride = max_bundle;
            if (!uniform) {
                uint32_t widest = 0;
                for (uint32_t t = 144; t <= 151; ++t) widest = std::max(widest, block_bytes_of(t));
                stride = ((uint64_t)F * (E / 128) * 2 + (uint64_t)E * (F / 128)) * widest;
            }
            slot_stride = (uint32_t)((stride + 255) & ~uint64_t(255));
            per_arena = (uint32_t)(kArenaLimit / slot_stride);
            lookup = dev.buffer((uint64_t)kMaxArenas * per_arena * 4, Kind::host);
        } else if (max_bundle > slot_stride) {
            throw NativeError(-1, "expert bundle exceeds the slot stride of the first layer");
        }
        // A layer's bundles are contiguous in one arena, so kernels can address expert e as
        // base + e * slot_stride.
        if (used_slots % per_arena + NE > per_arena) used_slots += per_arena - used_slots % per_arena;
        std::vector<ExpertDesc> desc(NE);
        for (uint32_t e = 0; e < NE; ++e) {
            const uint32_t slot = used_slots++;
            const uint32_t ai = slot / per_arena;
            if (ai >= kMaxArenas) throw NativeError(-1, "too many arenas");
            while (arenas.size() <= ai)
                // 256 bytes of slack: decoders read whole words past a row's last block.
                arenas.push_back(dev.buffer((uint64_t)per_arena * slot_stride + 256, Kind::device));
            const uint64_t off = (uint64_t)(slot % per_arena) * slot_stride;
            const Buffer &arena = arenas[ai];
            upload(arena, off, d.gate[e], gb[e]);
            upload(arena, off + gb[e], d.up[e], ub[e]);
            upload(arena, off + gb[e] + ub[e], d.down[e], db[e]);
            L.max_scale = std::max({L.max_scale, max_block_scale(d.gate[e], gb[e], block_bytes_of(d.types[e * 3])),
                                    max_block_scale(d.up[e], ub[e], block_bytes_of(d.types[e * 3 + 1])),
                                    max_block_scale(d.down[e], db[e], block_bytes_of(d.types[e * 3 + 2]))});
            lookup.words()[il * NE + e] = slot;
            desc[e].gate = arena.gpu + off;
            desc[e].up = arena.gpu + off + gb[e];
            desc[e].down = arena.gpu + off + gb[e] + ub[e];
            desc[e].types = d.types[e * 3] | (d.types[e * 3 + 1] << 8) | (d.types[e * 3 + 2] << 16);
            desc[e].pad = 0;
            if (e == 0) L.base = desc[0].gate;
        }
        L.xtab = dev.buffer(NE * sizeof(ExpertDesc), Kind::device);
        upload(L.xtab, 0, desc.data(), NE * sizeof(ExpertDesc));
        L.router = dev.buffer((uint64_t)NE * E * 4, Kind::device);
        upload(L.router, 0, d.router, (uint64_t)NE * E * 4);
        if (NE <= 256 && E % 256 == 0) {  // the prefill path's router shapes
            const std::vector<uint32_t> sp = split_router_rows(d.router, NE, E);
            L.router16 = dev.buffer(sp.size() * 4, Kind::device);
            upload(L.router16, 0, sp.data(), sp.size() * 4);
        }
        if (d.router_bias) {
            L.has_bias = true;
            L.bias = dev.buffer(NE * 4, Kind::device);
            upload(L.bias, 0, d.router_bias, NE * 4);
        }
        std::vector<float> signs(E + F, 1.0f);
        if (d.gate_signs) {
            L.has_gate_signs = true;
            std::memcpy(signs.data(), d.gate_signs, E * 4);
        }
        if (d.down_signs) {
            L.has_down_signs = true;
            std::memcpy(signs.data() + E, d.down_signs, F * 4);
        }
        L.signs = dev.buffer((E + F) * 4, Kind::device);
        upload(L.signs, 0, signs.data(), (E + F) * 4);
        if (d.norm_weight) {
            L.has_norm = true;
            L.norm = dev.buffer((uint64_t)E * 4, Kind::device);
            upload(L.norm, 0, d.norm_weight, (uint64_t)E * 4);
        }
        if (!(d.norm_eps >= 0.0f)) throw NativeError(-1, "norm_eps must be a non-negative number");
        L.norm_eps = d.norm_eps;
        if (d.SF) {
            if (!d.sh_gate || !d.sh_up || !d.sh_down || !d.sh_gate_inp) throw NativeError(-1, "shared expert weights missing");
            if (d.sh_type > GM_SHARED_F32) throw NativeError(-1, "unknown shared expert row format");
            if (d.SF % 64 || E % 64) throw NativeError(-1, "the shared expert needs E and SF multiples of 64");
            L.SF = d.SF;
            L.sh_kind = d.sh_type;
            const uint64_t SF = d.SF, kind = d.sh_type;
            const uint64_t src_e = shared_src_row(kind, E), src_f = shared_src_row(kind, SF);
            L.sh_row_e = (uint32_t)shared_dev_row(kind, E);
            L.sh_row_f = (uint32_t)shared_dev_row(kind, SF);
            L.sh_gu = dev.buffer(2 * SF * L.sh_row_e, Kind::device);
            L.sh_down = dev.buffer((uint64_t)E * L.sh_row_f, Kind::device);
            if (kind == GM_SHARED_Q8_0) {
                // Raw GGUF blocks into a temporary buffer, then q8_repack into the mv_q8 layout
                // (src/gpu_engine.zig:289-306).
                Buffer raw = dev.buffer(std::max(2 * SF * src_e, (uint64_t)E * src_f), Kind::device);
                upload(raw, 0, d.sh_gate, SF * src_e);
                upload(raw, SF * src_e, d.sh_up, SF * src_e);
                repack_q8(raw, 2 * SF, E, L.sh_gu, L.sh_row_e);
                upload(raw, 0, d.sh_down, (uint64_t)E * src_f);
                repack_q8(raw, E, SF, L.sh_down, L.sh_row_f);
                dev.release(raw);
            } else {
                upload(L.sh_gu, 0, d.sh_gate, SF * src_e);
                upload(L.sh_gu, SF * src_e, d.sh_up, SF * src_e);
                upload(L.sh_down, 0, d.sh_down, (uint64_t)E * src_f);
            }
            L.sh_gate = dev.buffer((uint64_t)E * 4, Kind::device);
            upload(L.sh_gate, 0, d.sh_gate_inp, (uint64_t)E * 4);
            // Binary16 copies for the prefill GEMMs, each matrix scaled by its own power of two.
            const uint64_t half = SF * E * 2;
            std::vector<float> fl;
            std::vector<uint16_t> h16;
            L.sh_gu16 = dev.buffer(2 * half, Kind::device);
            shared_to_floats(kind, d.sh_gate, SF, E, fl);
            L.sh_unscale[0] = floats_to_scaled_half(fl.data(), fl.size(), h16);
            upload(L.sh_gu16, 0, h16.data(), half);
            shared_to_floats(kind, d.sh_up, SF, E, fl);
            L.sh_unscale[1] = floats_to_scaled_half(fl.data(), fl.size(), h16);
            upload(L.sh_gu16, half, h16.data(), half);
            L.sh_down16 = dev.buffer(half, Kind::device);
            shared_to_floats(kind, d.sh_down, E, SF, fl);
            L.sh_unscale[2] = floats_to_scaled_half(fl.data(), fl.size(), h16);
            upload(L.sh_down16, 0, h16.data(), half);
            if (!x16.handle) x16 = dev.buffer((uint64_t)max_tok * E * 2, Kind::device);
            if (d.SF > sh_width) {
                for (Buffer *b : {&sh_h, &sh_a, &sh_o, &sh_g, &sh_s})
                    if (b->handle) dev.release(*b);
                const uint64_t T = max_tok;
                sh_h = dev.buffer(T * 2 * d.SF * 4, Kind::device);
                sh_a = dev.buffer(T * d.SF * 4, Kind::device);
                sh_o = dev.buffer(T * E * 4, Kind::device);
                sh_g = dev.buffer(T * 4, Kind::device);
                sh_s = dev.buffer(T * E * 4, Kind::device);
                sh_width = d.SF;
            }
        }
        layers.push_back(L);
        return il;
    }

    // Reference dispatch sequence, src/gpu_engine.zig:1052-1119: routed experts of one Gyro type
    // and the optional shared expert.
    void ffn_reference(uint32_t il, uint32_t n, uint32_t x_uav, uint32_t x_off, uint32_t out_uav,
                       uint32_t out_off) {
        const Layer &L = layers.at(il);
        if (!L.type_id) throw NativeError(-1, "the reference path needs one Gyro type per layer");
        const uint32_t bb = block_bytes_of(L.type_id);
        // Router logits, in chunks of 8 tokens (src/gpu_engine.zig:838-864); a bias is
        // preloaded and accumulated (mode 1).
        if (L.has_bias)
            dispatch("ew", {L.bias.uav, 0, 0, L.bias.uav, 0, 0, router_out.uav, 0, NE, NE, n, 5},
                     (NE * n + 255) / 256);
        uint32_t rpw = 1;
        while (NE / (8 * rpw * 2) >= 1024) rpw *= 2;
        const uint32_t groups = (NE + 8 * rpw - 1) / (8 * rpw);
        for (uint32_t done = 0; done < n; done += 8) {
            const uint32_t m = std::min(n - done, 8u);
            dispatch("mv_f32", {L.router.srv, 0, NE, E, x_uav, x_off + done * E, E, m, router_out.uav, done * NE,
                                NE, L.has_bias ? 1u : 0u, 0, bits(1.0f), E * 4, rpw},
                     groups);
        }
        if (L.has_gate_signs)
            dispatch("rotate128", {x_uav, x_off, xh.uav, 0, L.signs.srv, 0, E, E}, E / 128, n);
        else
            dispatch("ew", {x_uav, x_off, E, x_uav, x_off, E, xh.uav, 0, E, E, n, 3}, (E * n + 255) / 256);
        dev.barrier();
        dispatch("moe_route", {router_out.uav, 0, NE, U, ids.uav, 0, weights.uav, 0, kNone, 0, bits(L.scale), n}, n);
        dev.barrier();
        const uint32_t n_slots = n * U;
        std::vector<uint32_t> rs = {ids.uav, 0, n_slots, table.uav, lookup.uav, il * NE, per_arena, slot_stride,
                                    L.gate_bytes, (uint32_t)arenas.size(), 0, 0};
        for (uint32_t i = 0; i < 8; ++i) rs.push_back(i < arenas.size() ? arenas[i].srv : 0);
        dispatch("moe_resolve", rs, (n_slots + 63) / 64);
        dev.barrier();
        dispatch("moe_gyro", {table.uav, codebook.srv, xh.uav, 0, E, gu.uav, 0, F, E, L.type_id, bb, 0, U, 0, 0, 0},
                 (F + 31) / 32, n_slots, 2);
        dev.barrier();
        dispatch("moe_act", {gu.uav, 0, act.uav, 0, L.signs.srv, E, F, L.has_down_signs ? 1u : 0u}, n_slots);
        dev.barrier();
        dispatch("moe_gyro", {table.uav, codebook.srv, act.uav, 0, F, down.uav, 0, E, F, L.type_id, bb, 2, U, 1, 0, 0},
                 (E + 31) / 32, n_slots, 1);
        dev.barrier();
        uint32_t sh = sh_zero.uav, shg = sh_zero.uav;  // no shared expert: sigmoid(0) * 0
        if (L.SF) {
            shared_expert(L, n, x_uav, x_off, engine_shared());
            sh = sh_o.uav;
            shg = sh_g.uav;
        }
        dispatch("moe_combine", {down.uav, 0, weights.uav, 0, out_uav, out_off, U, E, sh, 0, shg, 0}, (E + 255) / 256, n);
        dev.barrier();
    }

    // Rows per wave of the reference's matrix-vector grid (src/gpu_engine.zig:851-853).
    static uint32_t mv_rpw(uint32_t rows) {
        uint32_t rpw = 1;
        while (rows / (8 * rpw * 2) >= 1024) rpw *= 2;
        return rpw;
    }
    void mv(const char *kernel, uint32_t w_srv, uint32_t rows, uint32_t cols, uint32_t row_bytes, uint32_t x_uav,
            uint32_t x_off, uint32_t x_stride, uint32_t n, uint32_t y_uav, uint32_t y_off, uint32_t y_stride) {
        const uint32_t rpw = mv_rpw(rows), groups = (rows + 8 * rpw - 1) / (8 * rpw);
        for (uint32_t done = 0; done < n; done += 8) {
            const uint32_t m = std::min(n - done, 8u);
            dispatch(kernel, {w_srv, 0, rows, cols, x_uav, x_off + done * x_stride, x_stride, m, y_uav,
                              y_off + done * y_stride, y_stride, 0, 0, bits(1.0f), row_bytes, rpw},
                     groups);
        }
    }

    // Shared expert of src/engine.zig:644-653 on the unrotated input, in the reference's kernels
    // (src/gpu_engine.zig:1061-1074): the gate and up rows by the mv kernel of the row format
    // (mv_bf16, mv_q8, mv_f32) into h, the ew SwiGLU into a, the down rows into o = W_d (silu(W_g x)
    // * W_u x), and g = g_sh . x by mv_f32. Buffers are (table index, word offset) pairs.
    SharedBufs engine_shared() const { return {sh_h.uav, 0, sh_a.uav, 0, sh_o.uav, 0, sh_g.uav, 0, sh_s.uav, 0}; }
    static const char *mv_kernel(uint32_t kind) {
        return kind == GM_SHARED_Q8_0 ? "mv_q8" : kind == GM_SHARED_F32 ? "mv_f32" : "mv_bf16";
    }
    void shared_expert(const Layer &L, uint32_t n, uint32_t x_uav, uint32_t x_off, const SharedBufs &S) {
        const uint32_t SF = L.SF;
        const char *k = mv_kernel(L.sh_kind);
        mv(k, L.sh_gu.srv, 2 * SF, E, L.sh_row_e, x_uav, x_off, E, n, S.h, S.h_off, 2 * SF);
        dispatch("ew", {S.h, S.h_off, 2 * SF, S.h, S.h_off + SF, 2 * SF, S.a, S.a_off, SF, SF, n, 0}, (SF * n + 255) / 256);
        mv(k, L.sh_down.srv, E, SF, L.sh_row_f, S.a, S.a_off, SF, n, S.o, S.o_off, E);
        mv("mv_f32", L.sh_gate.srv, 1, E, E * 4, x_uav, x_off, E, n, S.g, S.g_off, 1);
    }

    // Any layer (mixed Gyro types, optional shared expert), in the reference's dispatch style:
    // router, rotation, route, moe_gyro_x gate/up, moe_act, moe_gyro_x down, shared expert,
    // combine.
    void ffn_generic(uint32_t il, uint32_t n, uint32_t x_uav, uint32_t x_off, uint32_t out_uav, uint32_t out_off) {
        const Layer &L = layers.at(il);
        if (L.has_bias)
            dispatch("ew", {L.bias.uav, 0, 0, L.bias.uav, 0, 0, router_out.uav, 0, NE, NE, n, 5}, (NE * n + 255) / 256);
        const uint32_t rpw = mv_rpw(NE), groups = (NE + 8 * rpw - 1) / (8 * rpw);
        for (uint32_t done = 0; done < n; done += 8) {
            const uint32_t m = std::min(n - done, 8u);
            dispatch("mv_f32", {L.router.srv, 0, NE, E, x_uav, x_off + done * E, E, m, router_out.uav, done * NE,
                                NE, L.has_bias ? 1u : 0u, 0, bits(1.0f), E * 4, rpw},
                     groups);
        }
        if (L.has_gate_signs)
            dispatch("rotate128", {x_uav, x_off, xh.uav, 0, L.signs.srv, 0, E, E}, E / 128, n);
        else
            dispatch("ew", {x_uav, x_off, E, x_uav, x_off, E, xh.uav, 0, E, E, n, 3}, (E * n + 255) / 256);
        dispatch("moe_route", {router_out.uav, 0, NE, U, ids.uav, 0, weights.uav, 0, kNone, 0, bits(L.scale), n}, n);
        const uint32_t n_slots = n * U;
        dispatch("moe_gyro_x", {ids.uav, 0, L.xtab.srv, codebook.srv, xh.uav, 0, E, gu.uav, 0, F, E, 0, U, 0, NE},
                 (F + 31) / 32, n_slots, 2);
        dispatch("moe_act", {gu.uav, 0, act.uav, 0, L.signs.srv, E, F, L.has_down_signs ? 1u : 0u}, n_slots);
        dispatch("moe_gyro_x", {ids.uav, 0, L.xtab.srv, codebook.srv, act.uav, 0, F, down.uav, 0, E, F, 2, U, 1, NE},
                 (E + 31) / 32, n_slots, 1);
        uint32_t sh = sh_zero.uav, shg = sh_zero.uav;
        if (L.SF) {
            shared_expert(L, n, x_uav, x_off, engine_shared());
            sh = sh_o.uav;
            shg = sh_g.uav;
        }
        dispatch("moe_combine", {down.uav, 0, weights.uav, 0, out_uav, out_off, U, E, sh, 0, shg, 0}, (E + 255) / 256, n);
    }

    // Routed experts: uniform TQ2_T layers take moe_decode_gu (one token) or moe_decode_gu_b (2-8)
    // and moe_decode_down (E 1024 or 2048,
    // F 512, top-8) or moe_decode_gu_g and moe_decode_down_g / _gl (E a multiple of 256 up to 4096,
    // F a multiple of 128 up to 1024, top-1..16); other layers the type-generic kernels (_x for E
    // a multiple of 1024, F 512, top-8; _xg otherwise).
    // Shared expert: a bf16 one of width <= 1024 (a multiple of 256) on E <= 2048 at the _x shapes
    // runs fused into moe_router and moe_decode_down_x; any other (bf16, Q8_0 or fp32, any width
    // a multiple of 64) runs in the mv kernels first and enters the down kernel as its residual
    // input, sigmoid(g . x) * W_d (silu(W_g x) * W_u x).
    bool decode_supported(const Layer &L, uint32_t n) const {
        if (NE > 256 || n > 8 || E > 4096) return false;
        if (decode_fused_shared(L)) return true;
        const bool general = E % 256 == 0 && F % 128 == 0 && F <= 1024 && U >= 1 && U <= 16;
        if (L.type_id == 144) return general;
        return decode_generic_tuned() || general;
    }
    bool decode_generic_tuned() const { return E % 1024 == 0 && F == 512 && U == 8; }
    // Uniform TQ2_T layers take moe_decode_gu / moe_decode_down at their compile-time shape
    // (hidden 1024 or 2048, F 512, top-8), moe_decode_gu_g / moe_decode_down_g(l) otherwise.
    bool decode_tuned_tq2() const { return E % 1024 == 0 && F == 512 && U == 8 && parts <= 2; }
    uint32_t cus_or(uint32_t fallback) const { return cus ? cus : fallback; }
    bool decode_fused_shared(const Layer &L) const {
        return L.SF && L.sh_kind == GM_SHARED_BF16 && decode_generic_tuned() && L.SF <= 1024 && L.SF % 256 == 0 &&
               E <= 2048;
    }
    // Layers other than uniform TQ2_T (or with the fused shared expert) take the type-generic kernels.
    bool decode_generic_types(const Layer &L) const { return L.type_id != 144 || decode_fused_shared(L); }



    struct UnfusedPrefillScope {
        Engine *e;
        bool was;
        explicit UnfusedPrefillScope(Engine *eng) : e(eng), was(eng->prefill_fused) { e->prefill_fused = false; }
        ~UnfusedPrefillScope() { e->prefill_fused = was; }
    };
    // Reads and clears the give-up word of the persistent GEMMs: set when a down unit stopped waiting
    // for its tile's gate/up rows (the call's outputs are then invalid).
    bool take_gemm_error() {
        if (!gemm_sched.handle) return false;
        uint32_t w = 0;
        check(gd_readback(dev.ctx, gemm_sched.handle, 4, 4, &w, kTimeoutMs), "gd_readback");
        if (!w) return false;
        const uint32_t zero = 0;
        upload(gemm_sched, 4, &zero, 4);
        return true;
    }


    // MI355X decode path: router + rotation, routed gate/up, down + combine.
    void ffn_decode(uint32_t il, uint32_t n, uint32_t x_uav, uint32_t x_off, uint32_t out_uav, uint32_t out_off,
                    int bracket = 0, std::vector<uint32_t> *marks = nullptr, StackStep st = {},
                    const DecodeBufs *bufs = nullptr) {
        const Layer &L = layers.at(il);
        const DecodeBufs B = bufs ? *bufs : engine_bufs();
        if (!decode_supported(L, n))
            throw NativeError(-1, "decode path needs <= 256 experts, n <= 8, E a multiple of 256 up to 4096, F a "
                                  "multiple of 128 up to 1024 and top-1..16 (or, for other than uniform TQ2_T "
                                  "experts, E a multiple of 1024 with F 512 and top-8)");
        const bool fused_sh = decode_fused_shared(L);
        if (L.SF && !fused_sh) {
            // The shared expert first; its gated output (plus a stack's stream) is the residual
            // input of the down kernel.
            const SharedBufs &S = B.shared;
            shared_expert(L, n, x_uav, x_off, S);
            dispatch("ew", {S.o, S.o_off, E, S.g, S.g_off, 1, S.s, S.s_off, E, E, n, 4}, (E * n + 255) / 256);
            if (st.res_uav != kNone)
                dispatch("ew", {S.s, S.s_off, E, st.res_uav, st.res_off, E, S.s, S.s_off, E, E, n, 2}, (E * n + 255) / 256);
            st.res_uav = S.s;
            st.res_off = S.s_off;
        }
        const uint32_t rsf = fused_sh ? L.SF : 0u;  // shared rows computed inside moe_router
        const uint32_t base_lo = (uint32_t)L.base, base_hi = (uint32_t)(L.base >> 32);
        const bool generic = decode_generic_types(L);
        dispatch_maybe_timed(bracket == 1, marks, "moe_router",
                             {x_uav, x_off, E, n, L.router.srv, 0, NE, E, L.has_bias ? L.bias.srv : kNone, 0,
                              B.logits, B.logits_off, L.has_gate_signs ? L.signs.srv : kNone, 0, B.xh, B.xh_off,
                              st.on ? (L.has_norm ? 2u : 1u) : 0u, L.has_norm ? L.norm.srv : 0u, 0,
                              bits(L.norm_eps), 2 * rsf, rsf ? L.sh_gu.srv : 0u, rsf ? B.sh_h : 0u,
                              rsf ? L.sh_gate.srv : 0u, rsf ? B.sh_g : 0u},
                             NE + E / 128 + (rsf ? 2 * rsf / 4 + 1 : 0));
        if (!generic || !decode_generic_tuned()) {
            if (!generic && decode_tuned_tq2()) {
                // One token: the build that holds a block's activations in registers at once;
                // more: the half-block build, which lets four groups share a compute unit.
                dispatch_maybe_timed(bracket == 2, marks, n == 1 ? "moe_decode_gu" : "moe_decode_gu_b",
                                     {B.logits, B.logits_off, NE, U, bits(L.scale), B.ids, B.ids_off, B.weights, B.weights_off, B.xh,
                                      B.xh_off, base_lo, base_hi, slot_stride, L.gate_bytes, codebook.srv, B.gu, B.gu_off, E, F, n},
                                     F / 64, 2 * parts, n * U);
                dispatch_maybe_timed(bracket == 3, marks, "moe_decode_down",
                                     {B.gu, B.gu_off, B.ids, B.ids_off, B.weights, B.weights_off, base_lo, base_hi, slot_stride,
                                      2 * L.gate_bytes, codebook.srv, L.has_down_signs ? L.signs.srv : kNone, E, out_uav,
                                      out_off, E, F, U, n, parts, NE, st.res_uav != kNone ? 1u : 0u, st.res_uav,
                                      st.res_off},
                                     E / 8, n);
                return;
            }
            // Other shapes: runs of RPG (token, slot, row) rows per gate/up group (at most 1024
            // (row, block) items) and R output rows per down group (R divides E; at most 1024
            // (slot, block, half, row pair) items and 512 (row, slot) sums), about one group per
            // CU for a token. Layers of other types take the same kernels in their type-generic
            // form (_xg: rows through the expert table, each expert's types).
            const uint32_t nb = E / 128, total = n * U * F, target = cus_or(256);
            const uint32_t rpg = std::max(1u, std::min({(total + target - 1) / target, F, 1024u / nb}));
            uint32_t R = std::max(1u, E / target);
            while (R > 1 && (E % R || U * (F / 128) * 2 * ((R + 1) / 2) > 1024 || R * U > 512)) --R;
            const uint32_t xt = generic ? L.xtab.srv : 0u;
            dispatch_maybe_timed(bracket == 2, marks, generic ? "moe_decode_gu_xg" : "moe_decode_gu_g",
                                 {B.logits, B.logits_off, NE, U, bits(L.scale), B.ids, B.ids_off, B.weights, B.weights_off, B.xh,
                                  B.xh_off, generic ? 0u : base_lo, generic ? 0u : base_hi, generic ? 0u : slot_stride,
                                  generic ? 0u : L.gate_bytes, codebook.srv, B.gu, B.gu_off, E, F, n, rpg, xt},
                                 (total + rpg - 1) / rpg);
            const char *down = generic ? "moe_decode_down_xg"
                                       : (U * (F / 128) <= 64 ? "moe_decode_down_g" : "moe_decode_down_gl");
            dispatch_maybe_timed(bracket == 3, marks, down,
                                 {B.gu, B.gu_off, B.ids, B.ids_off, B.weights, B.weights_off, generic ? 0u : base_lo,
                                  generic ? 0u : base_hi, generic ? 0u : slot_stride, generic ? 0u : 2 * L.gate_bytes,
                                  codebook.srv, L.has_down_signs ? L.signs.srv : kNone, E, out_uav, out_off, E, F, U, n, R, NE,
                                  st.res_uav != kNone ? 1u : 0u, st.res_uav, st.res_off, xt},
                                 E / R, n);
            return;
        }
        dispatch_maybe_timed(bracket == 2, marks, n == 1 ? "moe_decode_gu_x" : "moe_decode_gu_xb",
                             {B.logits, B.logits_off, NE, U, bits(L.scale), B.ids, B.ids_off, B.weights, B.weights_off, B.xh, B.xh_off,
                              L.xtab.srv, codebook.srv, B.gu, B.gu_off, E, F, n},
                             F / 64, 2 * parts, n * U);
        // One token: 8 rows per group (E / 8 groups fill the GPU); more: 16 (E / 16 per token),
        // the same sums in the same order.
        const bool dx8 = n == 1;
        dispatch_maybe_timed(bracket == 3, marks, dx8 ? "moe_decode_down_x" : "moe_decode_down_xb",
                             {B.gu, B.gu_off, B.ids, B.ids_off, B.weights, B.weights_off, L.xtab.srv, 0, 0, 0, codebook.srv,
                              L.has_down_signs ? L.signs.srv : kNone, E, out_uav, out_off, E, F, U, n, parts, NE,
                              st.res_uav != kNone ? 1u : 0u, st.res_uav, st.res_off, rsf ? 1u : 0u, B.sh_h, 0,
                              B.sh_g, 0, rsf ? L.sh_down.srv : 0u, rsf},
                             dx8 ? E / 8 : E / 16, n);
    }

    // The grouped-GEMM path feeds binary16 weights (block scale x codebook value) to the MFMA;
    // every such product must be finite in binary16. Uniform TQ2_T layers take moe_prefill_gu /
    // moe_prefill_down, other layers the type-generic moe_prefill_gu_x / moe_prefill_down_x.
    // A shared expert runs as moe_prefill_shared (SF a multiple of 64).
    // F a multiple of 128 (an odd block count per down row is handled), top-U for U <= 16.
    bool prefill_supported(const Layer &L) const { return prefill_shape_ok(L) && prefill_range_ok(L); }
    bool prefill_shape_ok(const Layer &L) const {
        return L.SF % 64 == 0 && (L.SF == 0 || E <= 4096) && E % 256 == 0 && F % 128 == 0 && F >= 256 && U >= 1 &&
               U <= 16 && NE <= 256;
    }
    bool prefill_range_ok(const Layer &L) const { return L.max_scale * max_codebook < 65504.0f; }
    // A layer of a prefill shape whose block scale x codebook products leave the binary16 range
    // (one outlier block suffices) runs its prefill calls on the generic path, which keeps the
    // reference's fp32 weights, instead of being refused.
    bool prefill_on_generic(const Layer &L) const { return prefill_shape_ok(L) && !prefill_range_ok(L); }

    // MI355X prefill path: router GEMM + rotation, top-k, counting sort, grouped gate/up and
    // down GEMMs (one persistent launch), shared expert, combine.
    // bracket: 1 router, 2 gate/up (the persistent launch: both GEMMs), 3 down (none with the
    // persistent launch), 4 top-k, 5 sort, 6 combine, 7 shared gate/up, 8 shared down.
    void ffn_prefill(uint32_t il, uint32_t n, uint32_t x_uav, uint32_t x_off, uint32_t out_uav, uint32_t out_off,
                     int bracket = 0, std::vector<uint32_t> *marks = nullptr, uint32_t res_uav = kNone,
                     uint32_t res_off = 0, const NormNext *norm_next = nullptr) {
        const Layer &L = layers.at(il);
        if (!prefill_supported(L))
            throw NativeError(-1, "prefill path needs E a multiple of 256, F a multiple of 128 and at least 256, top-1 to top-16 of <= 256 experts, a shared expert (if "
                                  "any) of width a multiple of 64 on E <= 4096 and binary16-finite scale x codebook "
                                  "products");
        if (n * U > 32768u) throw NativeError(-1, "prefill calls take at most 32768 token slots (n x n_used)");
        const uint32_t base_lo = (uint32_t)L.base, base_hi = (uint32_t)(L.base >> 32);
        const uint32_t tiles = max_tiles(n);
        const uint32_t signs = L.has_down_signs ? L.signs.srv : kNone;
        // K split of the router: small batches get more groups (up to router_groups), each K
        // range writing its own logit plane (at most two planes of max_tok rows).
        const bool wide = router_wide_min && n >= router_wide_min;
        const uint32_t rt_gy = wide ? (NE + 255) / 256 : (NE + 31) / 32;
        const uint32_t rt_tiles = ((n + 31) / 32) * rt_gy;
        uint32_t ks = 1;
        while (rt_tiles * ks * 2 <= router_groups && E % (128 * ks * 2) == 0 && ks * 2 <= 16 &&
               (uint64_t)ks * 2 * n <= (wide ? 2ull : 1ull) * max_tok)
            ks *= 2;
        dispatch_maybe_timed(bracket == 1, marks, wide ? "moe_prefill_router_w" : "moe_prefill_router",
                             {x_uav, x_off, n, E, L.router16.srv, 0, NE, L.has_bias ? L.bias.srv : kNone, 0,
                              router_out.uav, 0, L.has_gate_signs ? L.signs.srv : kNone, 0, xh.uav, 0,
                              L.SF ? 1u : 0u, L.SF ? x16.uav : 0u, 0, ks, flag_uav(), hist.uav, 0, hist_words(n)},
                             (n + 31) / 32, rt_gy, ks);
        dispatch_maybe_timed(bracket == 4, marks, "moe_prefill_topk",
                             {router_out.uav, 0, NE, n, bits(L.scale), ids.uav, 0, weights.uav, 0, ks, n * NE, U,
                              hist.uav, 0},
                             (n + 3) / 4);
        const bool fused = prefill_fused;  // both GEMMs in one persistent launch
        dispatch_maybe_timed(bracket == 5, marks, "moe_prefill_sort",
                             {ids.uav, 0, n * U, NE, order.uav, 0, meta.uav, kTileRows, fused ? gemm_sched.uav : 0u,
                              hist.uav, 0},
                             (n * U + kSortChunk - 1) / kSortChunk);
        if (fused && L.type_id != 144) {
            // Layers of other or mixed types: one persistent launch of one group per compute unit
            // (152.5 KB of LDS; bracket 2).
            dispatch_maybe_timed(bracket == 2, marks, "moe_prefill_gemm_x",
                                 {meta.uav, order.uav, 0, xh.uav, 0, L.xtab.srv, codebook.srv, signs, E, act.uav, 0, E,
                                  F, U, 1u, down.uav, 0, gemm_sched.uav, prefill_spin_limit},
                                 cus_or(256));
        } else if (fused) {
            // Both GEMMs in one persistent launch of two groups per compute unit (bracket 2).
            const bool small = use_small(n);
            dispatch_maybe_timed(bracket == 2, marks, small ? "moe_prefill_gemm_s" : "moe_prefill_gemm",
                                 {meta.uav, order.uav, 0, xh.uav, 0, base_lo, base_hi, slot_stride, L.gate_bytes,
                                  codebook.srv, signs, E, act.uav, 0, E, F, U, 1u, down.uav, 0, gemm_sched.uav,
                                  prefill_spin_limit, small ? small_rows() : 0u},
                                 2 * cus_or(256));
        } else if (L.type_id == 144) {
            dispatch_maybe_timed(bracket == 2, marks, "moe_prefill_gu",
                                 {meta.uav, order.uav, 0, xh.uav, 0, base_lo, base_hi, slot_stride, L.gate_bytes,
                                  codebook.srv, signs, E, act.uav, 0, E, F, U, 1u},
                                 F / 128, tiles);
            dispatch_maybe_timed(bracket == 3, marks, "moe_prefill_down",
                                 {meta.uav, order.uav, 0, act.uav, 0, base_lo, base_hi, slot_stride, 2 * L.gate_bytes,
                                  codebook.srv, down.uav, 0, E, F},
                                 E / 256, tiles);
        } else {
            dispatch_maybe_timed(bracket == 2, marks, "moe_prefill_gu_x",
                                 {meta.uav, order.uav, 0, xh.uav, 0, L.xtab.srv, codebook.srv, signs, E, act.uav, 0, E,
                                  F, U, 1u},
                                 F / 128, tiles);
            dispatch_maybe_timed(bracket == 3, marks, "moe_prefill_down_x",
                                 {meta.uav, order.uav, 0, act.uav, 0, L.xtab.srv, codebook.srv, down.uav, 0, E, F},
                                 E / 256, tiles);
        }
        if (L.SF) {
            // Shared expert (bracket 7): a = silu(W_g x) * W_u x into sh_a (binary16), then
            // W_d a into sh_o; the combine adds sigmoid(x . shared_gate) * sh_o.
            const uint32_t tt = (n + 31) / 32;
            dispatch_maybe_timed(bracket == 7, marks, "moe_prefill_shared",
                                 {0, x16.uav, 0, E, L.sh_gu16.srv, 0, E, sh_a.uav, 0, n, L.SF, bits(L.sh_unscale[0]),
                                  bits(L.sh_unscale[1]), L.SF, flag_uav()},
                                 L.SF / 64, tt);
            dispatch_maybe_timed(bracket == 8, marks, "moe_prefill_shared",
                                 {1, sh_a.uav, 0, L.SF, L.sh_down16.srv, 0, L.SF, sh_o.uav, 0, n, 0,
                                  bits(L.sh_unscale[2]), 0, E},
                                 E / 128, tt);
        }
        if (norm_next) {
            if (E > 4096) throw NativeError(-1, "the fused stack norm covers E <= 4096");
            dispatch_maybe_timed(bracket == 6, marks, "moe_prefill_combine_norm",
                                 {down.uav, 0, weights.uav, 0, out_uav, out_off, E, U, res_uav != kNone ? 1u : 0u,
                                  res_uav, res_off, L.SF ? 1u : 0u, L.SF ? sh_o.uav : 0u, 0, x_uav, x_off,
                                  L.SF ? L.sh_gate.srv : 0u, norm_next->w_srv, hn.uav, 0, norm_next->eps_bits},
                                 n);
            return;
        }
        dispatch_maybe_timed(bracket == 6, marks, "moe_prefill_combine",
                             {down.uav, 0, weights.uav, 0, out_uav, out_off, E, U, res_uav != kNone ? 1u : 0u, res_uav,
                              res_off, L.SF ? 1u : 0u, L.SF ? sh_o.uav : 0u, 0, x_uav, x_off,
                              L.SF ? L.sh_gate.srv : 0u},
                             (E + 1023) / 1024,
                             n);
    }

    void ffn(uint32_t path, uint32_t il, uint32_t n, uint32_t x_uav, uint32_t x_off, uint32_t out_uav,
             uint32_t out_off, int bracket = 0, std::vector<uint32_t> *marks = nullptr) {
        if (path == GM_PATH_REFERENCE)
            ffn_reference(il, n, x_uav, x_off, out_uav, out_off);
        else if (path == GM_PATH_DECODE)
            ffn_decode(il, n, x_uav, x_off, out_uav, out_off, bracket, marks);
        else if (path == GM_PATH_PREFILL && prefill_on_generic(layers.at(il)))
            ffn_generic(il, n, x_uav, x_off, out_uav, out_off);
        else if (path == GM_PATH_PREFILL)
            ffn_prefill(il, n, x_uav, x_off, out_uav, out_off, bracket, marks);
        else if (path == GM_PATH_GENERIC)
            ffn_generic(il, n, x_uav, x_off, out_uav, out_off);
        else
            throw NativeError(-1, "path not available");
    }

    // One stack pass over n tokens whose residual stream starts at x (x_uav, x_off) and ends in
    // (y_uav, y_off); y may be x. Per layer l, with s the stream (x before the first layer, y
    // after): y = s + MoE_l(RMSNorm_l(s)).
    //   decode:    the router normalises s itself and the down kernel adds s (three launches);
    //   prefill:   moe_stack_norm writes RMSNorm_l(s) to hn, the combine adds s and (unless
    //              stack_norm_fused is off) writes RMSNorm_{l+1} of the new stream to hn, so
    //              only the first layer runs moe_stack_norm;
    //   others:    moe_stack_norm also adds the previous layer's output (in `out`) to the stream
    //              and writes it to y; the path writes `out`; ew adds the last one.
    void stack(const uint32_t *list, uint32_t n_layers, uint32_t path, uint32_t n, uint32_t x_uav, uint32_t x_off,
               uint32_t y_uav, uint32_t y_off) {
        if (E > 4096) throw NativeError(-1, "stack RMSNorm covers E <= 4096");
        // A prefill stack with a layer whose weights leave the binary16 range (see
        // prefill_on_generic) runs every layer on the generic path: the prefill layers' fused
        // residual and the generic layers' deferred one do not mix within one pass.
        if (path == GM_PATH_PREFILL)
            for (uint32_t l = 0; l < n_layers; ++l)
                if (prefill_on_generic(layers.at(list[l]))) {
                    path = GM_PATH_GENERIC;
                    break;
                }
        bool normed = false;  // hn already holds this layer's normalised input
        for (uint32_t l = 0; l < n_layers; ++l) {
            const Layer &L = layers.at(list[l]);
            const bool first = l == 0;
            const uint32_t s_uav = first ? x_uav : y_uav, s_off = first ? x_off : y_off;
            const uint32_t w_srv = L.has_norm ? L.norm.srv : kNone;
            if (path == GM_PATH_DECODE && !L.SF) {
                StackStep st;
                st.on = true;
                st.res_uav = s_uav;
                st.res_off = s_off;
                ffn_decode(list[l], n, s_uav, s_off, y_uav, y_off, 0, nullptr, st);
            } else if (path == GM_PATH_DECODE) {
                // The shared expert reads the normalised input, so the norm is its own step.
                dispatch("moe_stack_norm",
                         {s_uav, s_off, kNone, 0, w_srv, 0, hn.uav, 0, E, bits(L.norm_eps), kNone, 0}, n);
                StackStep st;
                st.res_uav = s_uav;
                st.res_off = s_off;
                ffn_decode(list[l], n, hn.uav, 0, y_uav, y_off, 0, nullptr, st);
            } else if (path == GM_PATH_PREFILL) {
                if (!normed)
                    dispatch("moe_stack_norm",
                             {s_uav, s_off, kNone, 0, w_srv, 0, hn.uav, 0, E, bits(L.norm_eps), kNone, 0}, n);
                NormNext nn;
                const bool fuse = stack_norm_fused && l + 1 < n_layers;
                if (fuse) {
                    const Layer &N = layers.at(list[l + 1]);
                    nn.w_srv = N.has_norm ? N.norm.srv : kNone;
                    nn.eps_bits = bits(N.norm_eps);
                }
                ffn_prefill(list[l], n, hn.uav, 0, y_uav, y_off, 0, nullptr, s_uav, s_off, fuse ? &nn : nullptr);
                normed = fuse;
            } else {
                dispatch("moe_stack_norm", {s_uav, s_off, first ? kNone : out.uav, 0, w_srv, 0, hn.uav, 0, E,
                                            bits(L.norm_eps), y_uav, y_off},
                         n);
                ffn(path, list[l], n, hn.uav, 0, out.uav, 0);
                if (l + 1 == n_layers)
                    dispatch("ew", {y_uav, y_off, E, out.uav, 0, E, y_uav, y_off, E, E, n, 2}, (E * n + 255) / 256);
            }
        }
    }

    void check_stack(const uint32_t *list, uint32_t n_layers) const {
        if (!list || !n_layers) throw NativeError(-1, "empty layer list");
        for (uint32_t l = 0; l < n_layers; ++l)
            if (list[l] >= layers.size()) throw NativeError(-1, "layer index out of range");
    }

    // The prefill path rounds activations to binary16 for its MFMA products; a call whose
    // activations left the binary16 range is recomputed on the generic path, which keeps them in
    // fp32. (The decode path keeps every activation in fp32.)
    static bool fast_path(uint32_t path) { return path == GM_PATH_PREFILL; }

    void forward_stack(const uint32_t *list, uint32_t n_layers, uint32_t path, const float *x, uint32_t n, float *y) {
        if (n == 0 || n > max_tok) throw NativeError(-1, "token count exceeds max_tok");
        check_stack(list, n_layers);
        upload(x_in, 0, x, (uint64_t)n * E * 4);
        dev.begin();
        stack(list, n_layers, path, n, x_in.uav, 0, x_in.uav, 0);
        dev.wait(dev.submit());
        if (path == GM_PATH_PREFILL && take_gemm_error()) {
            UnfusedPrefillScope unfused{this};
            upload(x_in, 0, x, (uint64_t)n * E * 4);
            dev.begin();
            stack(list, n_layers, path, n, x_in.uav, 0, x_in.uav, 0);
            dev.wait(dev.submit());
        }
        if (fast_path(path) && take_range_flag()) {
            upload(x_in, 0, x, (uint64_t)n * E * 4);
            dev.begin();
            stack(list, n_layers, GM_PATH_GENERIC, n, x_in.uav, 0, x_in.uav, 0);
            dev.wait(dev.submit());
        }
        check(gd_readback(dev.ctx, x_in.handle, 0, n * E * 4, y, kTimeoutMs), "gd_readback");
    }

    // Reads and clears the activation range flags; true when a fast-path kernel rounded an
    // activation outside the binary16 range since the last call.
    bool take_range_flag() {
        uint32_t f = 0, g = 0;
        check(gd_readback(dev.ctx, range_flag.handle, 0, 4, &f, kTimeoutMs), "gd_readback");
        if (meta.handle) check(gd_readback(dev.ctx, meta.handle, kMetaRangeFlag * 4, 4, &g, kTimeoutMs), "gd_readback");
        if (!f && !g) return false;
        const uint32_t zero = 0;
        upload(range_flag, 0, &zero, 4);
        if (meta.handle) upload(meta, kMetaRangeFlag * 4, &zero, 4);
        return true;
    }
    // The flag's table index for kernels of the fast paths (none on direct launches, whose
    // callers do not read it).
    uint32_t flag_uav() const { return direct ? 0u : range_flag.uav; }

    // gm_forward_decode_noalloc: the decode path on device-resident x and y, its intermediate
    // buffers carved out of this GPU's scratch array (256-byte aligned, word offsets), queued on
    // `stream`. Nothing is allocated, copied or waited for.
    void forward_decode_noalloc(uint32_t il, const float *x, uint32_t n, float *y, void *stream) {
        if (n == 0 || n > 8) throw NativeError(-1, "gm_forward_decode_noalloc takes 1 to 8 tokens");
        const Layer &L = layers.at(il);
        if (!decode_supported(L, n)) throw NativeError(-1, "the layer is not on the decode path");
        uint64_t at = kNoallocBase;
        auto take = [&at](uint64_t bytes) {
            const uint64_t off = at;
            at = (at + bytes + 255) & ~uint64_t(255);
            return (uint32_t)(off / 4);
        };
        DecodeBufs B;
        B.logits = B.ids = B.weights = B.xh = B.gu = na_base.uav;
        B.logits_off = take((uint64_t)n * NE * 4);
        B.ids_off = take((uint64_t)n * U * 4);
        B.weights_off = take((uint64_t)n * U * 4);
        B.xh_off = take((uint64_t)n * E * 4);
        B.gu_off = take((uint64_t)parts * n * U * 2 * F * 4);
        B.sh_h = na_shh.uav;
        B.sh_g = na_shg.uav;
        B.shared = {};
        if (L.SF && !decode_fused_shared(L)) {
            SharedBufs &S = B.shared;
            S.h = S.a = S.o = S.g = S.s = na_base.uav;
            S.h_off = take((uint64_t)n * 2 * L.SF * 4);
            S.a_off = take((uint64_t)n * L.SF * 4);
            S.o_off = take((uint64_t)n * E * 4);
            S.g_off = take((uint64_t)n * 4);
            S.s_off = take((uint64_t)n * E * 4);
        }
        if (at > GM_NOALLOC_SCRATCH_BYTES ||
            (decode_fused_shared(L) && ((uint64_t)n * 2 * L.SF * 4 > kNoallocShHBytes || (uint64_t)n * 4 > kNoallocShGBytes)))
            throw NativeError(-1, "the layer's decode buffers exceed the GM_NOALLOC_SCRATCH_BYTES scratch array");
        direct = true;
        direct_stream = stream;
        struct Restore {
            Engine *e;
            ~Restore() {
                e->direct = false;
                e->direct_stream = nullptr;
            }
        } restore{this};
        const uint64_t xa = (uint64_t)(uintptr_t)x, ya = (uint64_t)(uintptr_t)y;
        dispatch("gd_table_set",
                 {2u, na_x.uav, (uint32_t)xa, (uint32_t)(xa >> 32), na_out.uav, (uint32_t)ya, (uint32_t)(ya >> 32)}, 1);
        ffn_decode(il, n, na_x.uav, 0, na_out.uav, 0, 0, nullptr, StackStep{}, &B);
    }

    void forward(uint32_t il, uint32_t path, const float *x, uint32_t n, float *y) {
        if (n == 0 || n > max_tok) throw NativeError(-1, "token count exceeds max_tok");
        upload(x_in, 0, x, (uint64_t)n * E * 4);
        dev.begin();
        ffn(path, il, n, x_in.uav, 0, out.uav, 0);
        dev.wait(dev.submit());
        if (path == GM_PATH_PREFILL && take_gemm_error()) {
            UnfusedPrefillScope unfused{this};
            dev.begin();
            ffn(path, il, n, x_in.uav, 0, out.uav, 0);
            dev.wait(dev.submit());
        }
        if (fast_path(path) && take_range_flag()) {
            dev.begin();
            ffn(GM_PATH_GENERIC, il, n, x_in.uav, 0, out.uav, 0);
            dev.wait(dev.submit());
        }
        check(gd_readback(dev.ctx, out.handle, 0, n * E * 4, y, kTimeoutMs), "gd_readback");
    }
};

}  // namespace gyro

using gyro::Engine;

struct gm_engine {
    Engine e;
};

template <typename Fn>
static int guarded(gm_engine *g, Fn fn) {
    if (!g) return -1;
    try {
        fn();
        return 0;
    } catch (const gyro::NativeError &err) {
        g->e.error = err.what();
        return err.code < 0 ? err.code : -1;
    } catch (const std::exception &err) {
        g->e.error = err.what();
        return -1;
    }
}

extern "C" int gm_create(const char *kernel_dir, uint32_t adapter, uint32_t max_tok, gm_engine **out) {
    if (!kernel_dir || !out || !max_tok) return -1;
    auto g = std::make_unique<gm_engine>();
    int rc = guarded(g.get(), [&] { g->e.create(kernel_dir, adapter, max_tok); });
    if (rc) {
        std::fprintf(stderr, "gm_create: %s\n", g->e.error.c_str());
        return rc;
    }
    *out = g.release();
    return 0;
}

extern "C" void gm_destroy(gm_engine *g) {
    if (!g) return;
    g->e.dev.deinit();
    delete g;
}

extern "C" const char *gm_last_error(gm_engine *g) { return g ? g->e.error.c_str() : "no engine"; }

extern "C" int gm_add_layer(gm_engine *g, const gm_layer_desc *d, uint32_t *out_index) {
    if (!d || !out_index) return -1;
    return guarded(g, [&] { *out_index = g->e.add_layer(*d); });
}

extern "C" int gm_forward(gm_engine *g, uint32_t layer, uint32_t path, const float *x, uint32_t n, float *y) {
    if (!x || !y) return -1;
    return guarded(g, [&] { g->e.forward(layer, path, x, n, y); });
}

extern "C" int gm_forward_stack(gm_engine *g, const uint32_t *layers, uint32_t n_layers, uint32_t path,
                                const float *x, uint32_t n, float *out) {
    if (!x || !out) return -1;
    return guarded(g, [&] { g->e.forward_stack(layers, n_layers, path, x, n, out); });
}

extern "C" int gm_last_routes(gm_engine *g, uint32_t n, uint32_t *ids, float *weights) {
    if (!ids || !weights) return -1;
    return guarded(g, [&] {
        Engine &e = g->e;
        gyro::check(gd_readback(e.dev.ctx, e.ids.handle, 0, n * e.U * 4, ids, gyro::kTimeoutMs), "gd_readback");
        gyro::check(gd_readback(e.dev.ctx, e.weights.handle, 0, n * e.U * 4, weights, gyro::kTimeoutMs),
                    "gd_readback");
    });
}

extern "C" int gm_last_sort(gm_engine *g, uint32_t n, uint32_t *order, uint32_t *order_start) {
    if (!order || !order_start) return -1;
    return guarded(g, [&] {
        Engine &e = g->e;
        if (n == 0 || n > e.max_tok) throw gyro::NativeError(-1, "token count exceeds max_tok");
        gyro::check(gd_readback(e.dev.ctx, e.order.handle, 0, n * e.U * 4, order, gyro::kTimeoutMs), "gd_readback");
        gyro::check(gd_readback(e.dev.ctx, e.meta.handle, 0, (e.NE + 1) * 4, order_start, gyro::kTimeoutMs),
                    "gd_readback");
    });
}

extern "C" int gm_last_tiles(gm_engine *g, uint32_t max_tiles, uint32_t *tiles, uint32_t *count) {
    if (!tiles || !count) return -1;
    return guarded(g, [&] {
        Engine &e = g->e;
        uint32_t n = 0;
        gyro::check(gd_readback(e.dev.ctx, e.meta.handle, 1023 * 4, 4, &n, gyro::kTimeoutMs), "gd_readback");
        if (n > max_tiles) throw gyro::NativeError(-1, "tile list longer than max_tiles");
        if (n) gyro::check(gd_readback(e.dev.ctx, e.meta.handle, 1024 * 4, n * 16, tiles, gyro::kTimeoutMs), "gd_readback");
        *count = n;
    });
}

extern "C" int gm_dequant_as(gm_engine *g, uint32_t layer, uint32_t expert, uint32_t proj, uint32_t row0,
                             uint32_t rows, uint32_t decoder, float *out) {
    if (!out) return -1;
    return guarded(g, [&] {
        Engine &e = g->e;
        const gyro::Layer &L = e.layers.at(layer);
        const uint32_t cols = proj == 2 ? e.F : e.E, total_rows = proj == 2 ? e.E : e.F;
        if (expert >= e.NE || proj > 2 || decoder > GM_DEQUANT_PREFILL_B16 || !rows || row0 + rows > total_rows)
            throw gyro::NativeError(-1, "range");
        gyro::Buffer o = e.dev.buffer((uint64_t)rows * cols * 4, gyro::Kind::device);
        const uint32_t units = rows * (cols / 128) * (decoder ? 2u : 1u);
        e.dev.begin();
        e.dispatch("moe_dequant", {L.xtab.srv, expert, proj, row0, rows, cols, e.codebook.srv, o.uav, 0, decoder},
                   (units + 255) / 256);
        e.dev.wait(e.dev.submit());
        gyro::check(gd_readback(e.dev.ctx, o.handle, 0, rows * cols * 4, out, gyro::kTimeoutMs), "gd_readback");
        e.dev.release(o);
    });
}

extern "C" int gm_dequant(gm_engine *g, uint32_t layer, uint32_t expert, uint32_t proj, uint32_t row0,
                          uint32_t rows, float *out) {
    return gm_dequant_as(g, layer, expert, proj, row0, rows, GM_DEQUANT_DECODE, out);
}

extern "C" int gm_set_tokens(gm_engine *g, const float *x, uint32_t n_total) {
    if (!x || !n_total) return -1;
    return guarded(g, [&] {
        Engine &e = g->e;
        if (e.tokens.handle) e.dev.release(e.tokens);
        if (e.outputs.handle) e.dev.release(e.outputs);
        e.tokens = e.dev.buffer((uint64_t)n_total * e.E * 4, gyro::Kind::device);
        e.outputs = e.dev.buffer((uint64_t)n_total * e.E * 4, gyro::Kind::device);
        e.upload(e.tokens, 0, x, (uint64_t)n_total * e.E * 4);
        e.n_tokens = n_total;
    });
}

extern "C" int gm_run_bracketed(gm_engine *g, uint32_t path, uint32_t batch, uint32_t calls, uint32_t first_token,
                                const uint32_t *layer_list, uint32_t n_layers, uint32_t bracket, double *device_ms,
                                double *wall_ms, double *bracket_us) {
    if (!layer_list || !n_layers || !device_ms || !wall_ms) return -1;
    return guarded(g, [&] {
        Engine &e = g->e;
        if (!e.n_tokens || !batch || batch > e.max_tok || (uint64_t)first_token + (uint64_t)batch * calls > e.n_tokens)
            throw gyro::NativeError(-1, "run exceeds the uploaded tokens or max_tok");
        const uint32_t per_submit = bracket ? 1000u : 4000u;
        double dev = 0, br = 0;
        uint64_t br_n = 0;
        const auto t0 = std::chrono::steady_clock::now();
        for (uint32_t first = 0; first < calls; first += per_submit) {
            const uint32_t last = std::min(calls, first + per_submit);
            std::vector<uint32_t> marks;
            e.dev.begin();
            marks.push_back(e.dev.timestamp());
            for (uint32_t i = first; i < last; ++i) {
                const uint32_t off = (first_token + i * batch) * e.E;
                e.ffn(path, layer_list[i % n_layers], batch, e.tokens.uav, off, e.outputs.uav, off, (int)bracket,
                      &marks);
            }
            marks.push_back(e.dev.timestamp());
            e.dev.wait(e.dev.submit());
            std::vector<uint64_t> ticks(marks.size());
            const uint64_t freq = e.dev.timestamps(ticks.data(), (uint32_t)ticks.size());
            dev += (double)(ticks.back() - ticks.front()) * 1e3 / (double)freq;
            for (size_t j = 1; j + 2 < marks.size(); j += 2) {
                br += (double)(ticks[j + 1] - ticks[j]) * 1e6 / (double)freq;
                ++br_n;
            }
        }
        *wall_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        *device_ms = dev;
        if (bracket_us) *bracket_us = br_n ? br / (double)br_n : 0.0;
        if (path == GM_PATH_PREFILL && e.take_gemm_error())
            throw gyro::NativeError(-1, "a prefill GEMM unit gave up waiting for its tile's gate/up rows: the outputs of "
                                        "this run are invalid (gm_forward recomputes such calls with two GEMM launches)");
        if (Engine::fast_path(path) && e.take_range_flag())
            throw gyro::NativeError(-1, "an activation left the binary16 range on the prefill path: the outputs of this run "
                                        "are invalid (gm_forward recomputes such calls on GM_PATH_GENERIC)");
    });
}

extern "C" int gm_run(gm_engine *g, uint32_t path, uint32_t batch, uint32_t calls, uint32_t first_token,
                      const uint32_t *layer_list, uint32_t n_layers, double *device_ms, double *wall_ms) {
    return gm_run_bracketed(g, path, batch, calls, first_token, layer_list, n_layers, 0, device_ms, wall_ms, nullptr);
}

extern "C" int gm_run_stack(gm_engine *g, uint32_t path, uint32_t batch, uint32_t calls, uint32_t first_token,
                            const uint32_t *layer_list, uint32_t n_layers, double *device_ms, double *wall_ms) {
    if (!device_ms || !wall_ms) return -1;
    return guarded(g, [&] {
        Engine &e = g->e;
        e.check_stack(layer_list, n_layers);
        if (!e.n_tokens || !batch || batch > e.max_tok || (uint64_t)first_token + (uint64_t)batch * calls > e.n_tokens)
            throw gyro::NativeError(-1, "run exceeds the uploaded tokens or max_tok");
        // About 4000 dispatches per submission.
        const uint32_t per_submit = std::max(1u, 4000u / (n_layers * 8u));
        double dev = 0;
        const auto t0 = std::chrono::steady_clock::now();
        for (uint32_t first = 0; first < calls; first += per_submit) {
            const uint32_t last = std::min(calls, first + per_submit);
            e.dev.begin();
            const uint32_t t_start = e.dev.timestamp();
            for (uint32_t i = first; i < last; ++i) {
                const uint32_t off = (first_token + i * batch) * e.E;
                e.stack(layer_list, n_layers, path, batch, e.tokens.uav, off, e.outputs.uav, off);
            }
            const uint32_t t_end = e.dev.timestamp();
            e.dev.wait(e.dev.submit());
            std::vector<uint64_t> ticks(t_end + 1);
            const uint64_t freq = e.dev.timestamps(ticks.data(), (uint32_t)ticks.size());
            dev += (double)(ticks[t_end] - ticks[t_start]) * 1e3 / (double)freq;
        }
        *wall_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        *device_ms = dev;
        if (path == GM_PATH_PREFILL && e.take_gemm_error())
            throw gyro::NativeError(-1, "a prefill GEMM unit gave up waiting for its tile's gate/up rows: the outputs of "
                                        "this run are invalid (gm_forward_stack recomputes such calls with two GEMM launches)");
        if (Engine::fast_path(path) && e.take_range_flag())
            throw gyro::NativeError(-1, "an activation left the binary16 range on the prefill path: the outputs of this run "
                                        "are invalid (gm_forward_stack recomputes such calls on GM_PATH_GENERIC)");
    });
}

extern "C" int gm_forward_decode_noalloc(gm_engine *g, uint32_t layer, const float *x, uint32_t n, float *out,
                                         void *stream) {
    if (!x || !out) return -1;
    return guarded(g, [&] { g->e.forward_decode_noalloc(layer, x, n, out, stream); });
}

extern "C" int gm_read_outputs(gm_engine *g, float *y, uint32_t n_total) {
    if (!y) return -1;
    return guarded(g, [&] {
        Engine &e = g->e;
        if (n_total > e.n_tokens) throw gyro::NativeError(-1, "more outputs than tokens");
        gyro::check(gd_readback(e.dev.ctx, e.outputs.handle, 0, (uint32_t)((uint64_t)n_total * e.E * 4), y,
                                gyro::kTimeoutMs),
                    "gd_readback");
    });
}
