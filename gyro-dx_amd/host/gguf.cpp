// GGUF v3 header reader and expert slicing (include/gyro_gguf.h), restating src/gguf.zig:
// the little-endian cursor (:19-62), metadata entries (:65-110), tensor layouts (:113-125),
// expertRange (:138-143) and parse (:263-330), with the same limits and error kinds.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <unordered_set>
#include <vector>

#include "gyro_gguf.h"

namespace {

constexpr uint64_t kMaxHeaderBytes = 64ull * 1024 * 1024;  // src/gguf.zig:5

enum ValueType : uint32_t {  // src/gguf.zig:13-17
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7, kString = 8,
    kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12,
};

struct Fail {
    int code;
};

struct Cursor {
    const uint8_t *bytes;
    size_t len, pos = 0;
    const uint8_t *take(uint64_t n) {
        if (n > len - pos) throw Fail{GG_UNEXPECTED_END};
        const uint8_t *r = bytes + pos;
        pos += n;
        return r;
    }
    template <class T>
    T num() {
        T v;
        std::memcpy(&v, take(sizeof(T)), sizeof(T));  // little-endian host
        return v;
    }
    std::string str() {
        const uint64_t n = num<uint64_t>();
        if (n > kMaxHeaderBytes) throw Fail{GG_LIMIT_EXCEEDED};
        const uint8_t *p = take(n);
        return std::string(reinterpret_cast<const char *>(p), n);
    }
    uint32_t tag() {
        const uint32_t t = num<uint32_t>();
        if (t > kF64) throw Fail{GG_INVALID_TYPE};
        return t;
    }
    void skip(uint32_t kind, int depth) {
        if (depth > 8) throw Fail{GG_LIMIT_EXCEEDED};
        switch (kind) {
            case kU8: case kI8: take(1); break;
            case kBool: if (num<uint8_t>() > 1) throw Fail{GG_INVALID_BOOLEAN}; break;
            case kU16: case kI16: take(2); break;
            case kU32: case kI32: case kF32: take(4); break;
            case kU64: case kI64: case kF64: take(8); break;
            case kString: str(); break;
            default: {  // array: element type, count, elements (booleans and nested lengths checked)
                const uint32_t et = tag();
                const uint64_t n = num<uint64_t>();
                if (n > 16ull * 1024 * 1024) throw Fail{GG_LIMIT_EXCEEDED};
                for (uint64_t i = 0; i < n; ++i) skip(et, depth + 1);
            }
        }
    }
};

uint64_t add(uint64_t a, uint64_t b) {
    if (a > UINT64_MAX - b) throw Fail{GG_INTEGER_OVERFLOW};
    return a + b;
}
uint64_t mul(uint64_t a, uint64_t b) {
    if (a && b > UINT64_MAX / a) throw Fail{GG_INTEGER_OVERFLOW};
    return a * b;
}

// src/gguf.zig:113-125: weights and bytes per block, or false for an unknown type.
bool layout(uint32_t type_id, uint64_t &block_weights, uint64_t &block_bytes) {
    static const uint32_t gyro_bb[8] = {34, 26, 30, 42, 50, 58, 22, 18};  // src/gyro.zig:32-41
    if (type_id >= 144 && type_id <= 151) {
        block_weights = 128;
        block_bytes = gyro_bb[type_id - 144];
        return true;
    }
    switch (type_id) {
        case 0: block_weights = 1; block_bytes = 4; return true;    // F32
        case 1: block_weights = 1; block_bytes = 2; return true;    // F16
        case 8: block_weights = 32; block_bytes = 34; return true;  // Q8_0
        case 30: block_weights = 1; block_bytes = 2; return true;   // BF16
        default: return false;
    }
}

struct Entry {
    std::string key;
    uint32_t kind;
    std::vector<uint8_t> raw;
};

struct Tensor {
    std::string name;
    uint32_t rank;
    uint64_t dims[4];
    uint32_t type_id;
    uint64_t relative_offset, file_offset = 0, byte_length = UINT64_MAX;
};

}  // namespace

struct gg_model {
    uint32_t version = 0, alignment = 32;
    uint64_t data_offset = 0, file_size = 0;
    std::vector<Entry> metadata;
    std::vector<Tensor> tensors;
};

namespace {

void parse(const uint8_t *prefix, size_t prefix_len, uint64_t file_size, gg_model &m) {
    Cursor c{prefix, prefix_len};
    if (std::memcmp(c.take(4), "GGUF", 4) != 0) throw Fail{GG_BAD_MAGIC};
    m.version = c.num<uint32_t>();
    if (m.version != 3) throw Fail{GG_UNSUPPORTED_VERSION};
    const uint64_t tensor_count = c.num<uint64_t>(), metadata_count = c.num<uint64_t>();
    if (tensor_count > 1000000 || metadata_count > 1000000) throw Fail{GG_LIMIT_EXCEEDED};
    // An entry needs a one-byte key, its type and at least one value byte.
    if (metadata_count > (c.len - c.pos) / 14) throw Fail{GG_UNEXPECTED_END};
    std::unordered_set<std::string> keys;
    m.alignment = 32;
    for (uint64_t i = 0; i < metadata_count; ++i) {
        Entry e;
        e.key = c.str();
        if (e.key.empty() || e.key.size() > 65535) throw Fail{GG_INVALID_METADATA};
        if (!keys.insert(e.key).second) throw Fail{GG_DUPLICATE_KEY};
        e.kind = c.tag();
        const size_t start = c.pos;
        c.skip(e.kind, 0);
        e.raw.assign(prefix + start, prefix + c.pos);
        if (e.key == "general.alignment") {
            if (e.kind != kU32) throw Fail{GG_INVALID_ALIGNMENT};
            uint32_t v;
            std::memcpy(&v, e.raw.data(), 4);
            m.alignment = v;
        }
        m.metadata.push_back(std::move(e));
    }
    if (m.alignment == 0 || m.alignment > 65536 || (m.alignment & (m.alignment - 1))) throw Fail{GG_INVALID_ALIGNMENT};
    if (tensor_count > (c.len - c.pos) / 33) throw Fail{GG_UNEXPECTED_END};
    keys.clear();
    for (uint64_t i = 0; i < tensor_count; ++i) {
        Tensor t;
        t.name = c.str();
        if (t.name.empty() || t.name.size() > 4096) throw Fail{GG_INVALID_METADATA};
        if (!keys.insert(t.name).second) throw Fail{GG_DUPLICATE_TENSOR};
        t.rank = c.num<uint32_t>();
        if (t.rank == 0 || t.rank > 4) throw Fail{GG_INVALID_DIMENSIONS};
        for (auto &d : t.dims) d = 1;
        for (uint32_t r = 0; r < t.rank; ++r) {
            t.dims[r] = c.num<uint64_t>();
            if (t.dims[r] == 0) throw Fail{GG_INVALID_DIMENSIONS};
        }
        t.type_id = c.num<uint32_t>();
        t.relative_offset = c.num<uint64_t>();
        if (t.relative_offset % m.alignment) throw Fail{GG_INVALID_ALIGNMENT};
        uint64_t bw, bb;
        if (layout(t.type_id, bw, bb)) {
            if (t.dims[0] % bw) throw Fail{GG_INVALID_DIMENSIONS};
            uint64_t n = mul(t.dims[0] / bw, bb);
            for (uint32_t r = 1; r < t.rank; ++r) n = mul(n, t.dims[r]);
            t.byte_length = n;
        }
        m.tensors.push_back(std::move(t));
    }
    const uint64_t mask = m.alignment - 1;
    m.data_offset = add(c.pos, mask) & ~mask;
    if (m.data_offset > kMaxHeaderBytes) throw Fail{GG_LIMIT_EXCEEDED};
    if (m.data_offset > file_size) throw Fail{GG_INVALID_TENSOR_RANGE};
    if (m.data_offset > prefix_len) throw Fail{GG_UNEXPECTED_END};
    m.file_size = file_size;
    for (auto &t : m.tensors) {
        t.file_offset = add(m.data_offset, t.relative_offset);
        if (t.file_offset >= file_size) throw Fail{GG_INVALID_TENSOR_RANGE};
        if (t.byte_length != UINT64_MAX && add(t.file_offset, t.byte_length) > file_size)
            throw Fail{GG_INVALID_TENSOR_RANGE};
    }
    std::stable_sort(m.tensors.begin(), m.tensors.end(),
                     [](const Tensor &a, const Tensor &b) { return a.file_offset < b.file_offset; });
    for (size_t i = 0; i + 1 < m.tensors.size(); ++i) {
        const Tensor &t = m.tensors[i], &u = m.tensors[i + 1];
        if (u.file_offset == t.file_offset) throw Fail{GG_OVERLAPPING_TENSORS};
        if (t.byte_length != UINT64_MAX && add(t.file_offset, t.byte_length) > u.file_offset)
            throw Fail{GG_OVERLAPPING_TENSORS};
    }
}

const Tensor *find(const gg_model *m, const char *name) {
    for (const auto &t : m->tensors)
        if (t.name == name) return &t;
    return nullptr;
}

void fill(const Tensor &t, gg_tensor_info *out) {
    out->name = t.name.c_str();
    out->rank = t.rank;
    for (int i = 0; i < 4; ++i) out->dims[i] = t.dims[i];
    out->type_id = t.type_id;
    out->relative_offset = t.relative_offset;
    out->file_offset = t.file_offset;
    out->byte_length = t.byte_length;
}

const Entry *entry(const gg_model *m, const char *key) {
    for (const auto &e : m->metadata)
        if (e.key == key) return &e;
    return nullptr;
}

// src/gguf.zig:65-110 (Entry accessors) and :163-180 (Model.required / number / text).
const Entry &required(const gg_model &m, const char *key) {
    const Entry *e = entry(&m, key);
    if (!e) throw Fail{GG_INVALID_METADATA};
    return *e;
}
uint64_t number(const gg_model &m, const char *key) {
    const Entry &e = required(m, key);
    Cursor c{e.raw.data(), e.raw.size()};
    switch (e.kind) {
        case kU8: return c.num<uint8_t>();
        case kU16: return c.num<uint16_t>();
        case kU32: return c.num<uint32_t>();
        case kU64: return c.num<uint64_t>();
        default: throw Fail{GG_INVALID_METADATA};
    }
}
std::string text(const Entry &e) {
    if (e.kind != kString) throw Fail{GG_INVALID_METADATA};
    Cursor c{e.raw.data(), e.raw.size()};
    return c.str();
}
bool boolean(const Entry &e) {
    if (e.kind != kBool || e.raw.size() != 1) throw Fail{GG_INVALID_METADATA};
    return e.raw[0] == 1;
}
std::vector<std::string> strings(const Entry &e) {
    if (e.kind != kArray) throw Fail{GG_INVALID_METADATA};
    Cursor c{e.raw.data(), e.raw.size()};
    if (c.tag() != kString) throw Fail{GG_INVALID_METADATA};
    const uint64_t n = c.num<uint64_t>();
    std::vector<std::string> out;
    for (uint64_t i = 0; i < n; ++i) out.push_back(c.str());
    return out;
}
std::vector<int32_t> ints32(const Entry &e) {
    if (e.kind != kArray) throw Fail{GG_INVALID_METADATA};
    Cursor c{e.raw.data(), e.raw.size()};
    if (c.tag() != kI32) throw Fail{GG_INVALID_METADATA};
    const uint64_t n = c.num<uint64_t>();
    std::vector<int32_t> out;
    for (uint64_t i = 0; i < n; ++i) out.push_back(c.num<int32_t>());
    return out;
}

// src/gguf.zig:182-250.
void validate_gyro(const gg_model &m) {
    bool has_gyro = false;
    for (const auto &t : m.tensors) has_gyro |= t.type_id >= 144 && t.type_id <= 151;
    if (!has_gyro) return;
    if (number(m, "agention.trellis.state_bits") != 15) throw Fail{GG_UNSUPPORTED_GYRO_METADATA};
    if (number(m, "prism.hadamard.version") != 1) throw Fail{GG_UNSUPPORTED_GYRO_METADATA};
    const uint64_t b = number(m, "prism.hadamard.block_size");
    if (b == 0 || b > 65536 || (b & (b - 1))) throw Fail{GG_INVALID_METADATA};
    if (text(required(m, "prism.hadamard.transform")) != "normalized-sylvester-walsh-hadamard")
        throw Fail{GG_UNSUPPORTED_GYRO_METADATA};
    if (text(required(m, "prism.hadamard.axis")) != "input-last-dimension") throw Fail{GG_UNSUPPORTED_GYRO_METADATA};
    const std::string mode = text(required(m, "prism.hadamard.sign_mode"));
    const bool expl = mode == "explicit";
    if (!expl && mode != "identity") throw Fail{GG_UNSUPPORTED_GYRO_METADATA};
    const std::vector<std::string> names = strings(required(m, "prism.hadamard.weight_names"));
    if (names.empty()) throw Fail{GG_INVALID_METADATA};
    const std::vector<int32_t> widths = expl ? ints32(required(m, "prism.hadamard.sign_widths")) : std::vector<int32_t>{};
    uint64_t sum = 0;
    for (size_t i = 0; i < widths.size(); ++i) {
        const int32_t w = widths[i];
        if (w <= 0 || (uint64_t)w % b) throw Fail{GG_INVALID_METADATA};
        for (size_t j = 0; j < i; ++j)
            if (widths[j] == w) throw Fail{GG_INVALID_METADATA};
        sum = add(sum, (uint64_t)w);
    }
    if (expl) {
        const std::vector<int32_t> signs = ints32(required(m, "prism.hadamard.sign_values"));
        if (signs.size() != sum) throw Fail{GG_INVALID_METADATA};
        for (int32_t v : signs)
            if (v != 1 && v != -1) throw Fail{GG_INVALID_METADATA};
    } else if (entry(&m, "prism.hadamard.sign_widths") || entry(&m, "prism.hadamard.sign_values")) {
        throw Fail{GG_INVALID_METADATA};
    }
    std::unordered_set<std::string> seen;
    for (const auto &name : names) {
        if (!seen.insert(name).second) throw Fail{GG_INVALID_METADATA};
        const Tensor *t = find(&m, name.c_str());
        if (!t || t->dims[0] % b) throw Fail{GG_INVALID_METADATA};
        // Widths compare as u64 with the tensor's first dimension (src/gguf.zig:237).
        if (expl && std::none_of(widths.begin(), widths.end(),
                                 [&](int32_t w) { return (uint64_t)w == t->dims[0]; }))
            throw Fail{GG_INVALID_METADATA};
    }
    for (const char *key : {"prism.hadamard.gdn_v_grouped", "prism.hadamard.tied_output"}) {
        const Entry *e = entry(&m, key);
        if (e && boolean(*e)) throw Fail{GG_UNSUPPORTED_GYRO_METADATA};
    }
    if (const Entry *e = entry(&m, "prism.hadamard.inverse_weight_names"))
        if (!strings(*e).empty()) throw Fail{GG_UNSUPPORTED_GYRO_METADATA};
}

bool ends_with(const std::string &s, const char *suffix) {
    const size_t n = std::strlen(suffix);
    return s.size() >= n && s.compare(s.size() - n, n, suffix) == 0;
}

// No C++ exception crosses the C boundary: allocation failures (std::bad_alloc, and the
// length errors of containers asked to grow past their limits) return GG_OUT_OF_MEMORY, the
// reference's allocator error.
template <typename Fn>
int guarded(Fn fn) {
    try {
        return fn();
    } catch (const Fail &f) {
        return f.code;
    } catch (...) {
        return GG_OUT_OF_MEMORY;
    }
}

int gg_open_impl(const char *path, gg_model **out) {
    if (!out) return GG_INVALID_METADATA;
    *out = nullptr;
    FILE *f = std::fopen(path, "rb");
    if (!f) return GG_IO;
    std::fseek(f, 0, SEEK_END);
    const long size = std::ftell(f);
    std::fseek(f, 0, SEEK_SET);
    if (size < 0) {
        std::fclose(f);
        return GG_IO;
    }
    std::vector<uint8_t> prefix((size_t)std::min<uint64_t>((uint64_t)size, kMaxHeaderBytes));
    const size_t got = prefix.empty() ? 0 : std::fread(prefix.data(), 1, prefix.size(), f);
    std::fclose(f);
    if (got != prefix.size()) return GG_IO;
    return gg_parse(prefix.data(), prefix.size(), (uint64_t)size, out);
}

}  // namespace

extern "C" {

int gg_parse(const uint8_t *prefix, size_t prefix_len, uint64_t file_size, gg_model **out) {
    if (!out || (!prefix && prefix_len)) return GG_INVALID_METADATA;
    *out = nullptr;
    return guarded([&] {
        std::unique_ptr<gg_model> m(new gg_model);
        parse(prefix, prefix_len, file_size, *m);
        *out = m.release();
        return (int)GG_OK;
    });
}

int gg_open(const char *path, gg_model **out) {
    return guarded([&] { return gg_open_impl(path, out); });
}

void gg_free(gg_model *m) { delete m; }
uint32_t gg_version(const gg_model *m) { return m ? m->version : 0; }
uint32_t gg_alignment(const gg_model *m) { return m ? m->alignment : 0; }
uint64_t gg_data_offset(const gg_model *m) { return m ? m->data_offset : 0; }
uint32_t gg_tensor_count(const gg_model *m) { return m ? (uint32_t)m->tensors.size() : 0; }

int gg_tensor_at(const gg_model *m, uint32_t index, gg_tensor_info *out) {
    if (!m || !out || index >= m->tensors.size()) return GG_NOT_FOUND;
    fill(m->tensors[index], out);
    return GG_OK;
}

int gg_find_tensor(const gg_model *m, const char *name, gg_tensor_info *out) {
    const Tensor *t = m && name ? find(m, name) : nullptr;
    if (!t || !out) return GG_NOT_FOUND;
    fill(*t, out);
    return GG_OK;
}

int gg_expert_range(const gg_model *m, const char *name, uint32_t expert, uint64_t *file_offset, uint64_t *bytes) {
    const Tensor *t = m && name ? find(m, name) : nullptr;
    if (!t) return GG_NOT_FOUND;
    if (t->rank != 3 || expert >= t->dims[2]) return GG_INVALID_EXPERT;
    if (t->byte_length == UINT64_MAX) return GG_UNSUPPORTED_TENSOR_TYPE;
    const uint64_t stride = t->byte_length / t->dims[2];
    try {
        if (file_offset) *file_offset = add(t->file_offset, mul(stride, expert));
    } catch (const Fail &f) {
        return f.code;
    }
    if (bytes) *bytes = stride;
    return GG_OK;
}

int gg_is_expert_tensor(const char *name) {
    if (!name) return 0;
    const size_t n = std::strlen(name);
    for (const char *suffix : {".ffn_gate_exps.weight", ".ffn_up_exps.weight", ".ffn_down_exps.weight"}) {
        const size_t k = std::strlen(suffix);
        if (n >= k && std::memcmp(name + n - k, suffix, k) == 0) return 1;
    }
    return 0;
}

int gg_metadata_u64(const gg_model *m, const char *key, uint64_t *out) {
    if (!m || !key || !out) return GG_NOT_FOUND;
    for (const auto &e : m->metadata) {
        if (e.key != key) continue;
        switch (e.kind) {
            case kU8: *out = e.raw[0]; return GG_OK;
            case kU16: { uint16_t v; std::memcpy(&v, e.raw.data(), 2); *out = v; return GG_OK; }
            case kU32: { uint32_t v; std::memcpy(&v, e.raw.data(), 4); *out = v; return GG_OK; }
            case kU64: { uint64_t v; std::memcpy(&v, e.raw.data(), 8); *out = v; return GG_OK; }
            default: return GG_INVALID_METADATA;
        }
    }
    return GG_NOT_FOUND;
}

int gg_metadata_raw(const gg_model *m, const char *key, uint32_t *kind, const uint8_t **raw, size_t *len) {
    const Entry *e = m && key ? entry(m, key) : nullptr;
    if (!e) return GG_NOT_FOUND;
    if (kind) *kind = e->kind;
    if (raw) *raw = e->raw.data();
    if (len) *len = e->raw.size();
    return GG_OK;
}

int gg_validate_gyro(const gg_model *m) {
    if (!m) return GG_INVALID_METADATA;
    return guarded([&] {
        validate_gyro(*m);
        return (int)GG_OK;
    });
}

}  // extern "C"
