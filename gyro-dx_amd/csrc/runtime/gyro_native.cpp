// HIP implementation of the gyro_native C ABI (include/gyro_native.h) for MI355X.
//
// The reference bridge (native/gyro_native.cpp) drives D3D12 command lists, a bindless
// descriptor heap and DirectStorage. Here the same contract maps onto one device: an in-order
// compute stream, a copy stream, a device-resident table of base pointers indexed by the
// SRV/UAV indices kernels receive in their constants, and hipEvents as fence tickets.
#include "gyro_native.h"

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sched.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <limits>
#include <memory>
#include <new>
#include <vector>

static_assert(sizeof(gd_options) == 20, "gd_options layout");
static_assert(sizeof(gd_caps) == 184, "gd_caps layout");
static_assert(sizeof(gd_range) == 24, "gd_range layout");
static_assert(offsetof(gd_caps, adapter_name) == 56, "gd_caps layout");
static_assert(sizeof(gd_buffer_info) == 32, "gd_buffer_info layout");
static_assert(offsetof(gd_buffer_info, mapped) == 8, "gd_buffer_info layout");

namespace {

constexpr gd_result kOk = 0;
constexpr gd_result kInvalidArg = (gd_result)0x80070057u;
constexpr gd_result kOutOfMemory = (gd_result)0x8007000Eu;
constexpr gd_result kFail = (gd_result)0x80004005u;
constexpr gd_result kPending = (gd_result)0x8000000Au;
constexpr gd_result kTimeout = (gd_result)0x80070102u;
constexpr gd_result kBusy = (gd_result)0x800700AAu;
constexpr gd_result kInvalidData = (gd_result)0x8007000Du;
constexpr gd_result kUnsupported = (gd_result)0x887A0004u;
constexpr gd_result kIllegalCall = (gd_result)0x8000000Eu;
constexpr gd_result kDeviceRemoved = (gd_result)0x887A0005u;
constexpr gd_result kUnexpected = (gd_result)0x8000FFFFu;

constexpr uint32_t kTableCapacity = 1u << 16;
// Every table entry that names no live buffer (index 0, indices never handed out, released ones)
// points at a zeroed device block of this size instead of address 0. A dispatch given a wrong
// table index then reads zeros and writes into the block instead of faulting the GPU; a context
// created with gd_options.enable_debug (the reference's debug-layer switch) checks the block in
// gd_wait_compute and reports such a write as E_FAIL.
constexpr size_t kGuardBytes = 1u << 20;
constexpr uint32_t kMaxConstants = 60;
constexpr uint32_t kMaxTimestamps = 4096;
constexpr uint32_t kInfinite = 0xFFFFFFFFu;

// Kernel argument block shared by every pipeline: the table pointer and 60 constants.
struct GdArgs {
    const uint64_t *table;
    uint32_t c[kMaxConstants];
};

gd_result from_hip(hipError_t e) {
    if (e == hipSuccess) return kOk;
    if (e == hipErrorOutOfMemory) return kOutOfMemory;
    if (e == hipErrorInvalidValue || e == hipErrorInvalidImage || e == hipErrorNotFound ||
        e == hipErrorInvalidKernelFile || e == hipErrorNoBinaryForGpu)
        return kInvalidArg;
    if (e == hipErrorLaunchFailure || e == hipErrorIllegalAddress) return kDeviceRemoved;
    return kFail;
}

#define GD_HIP(expr)                                   \
    do {                                               \
        hipError_t gd_e = (expr);                      \
        if (gd_e != hipSuccess) return from_hip(gd_e); \
    } while (0)
#define GD_TRY(expr)                 \
    do {                             \
        gd_result gd_r = (expr);     \
        if (gd_r < 0) return gd_r;   \
    } while (0)

// Polls an event until it completes or the timeout (milliseconds) passes.
gd_result wait_event(hipEvent_t ev, uint32_t timeout_ms) {
    auto start = std::chrono::steady_clock::now();
    uint32_t spins = 0;
    for (;;) {
        hipError_t q = hipEventQuery(ev);
        if (q == hipSuccess) return kOk;
        if (q != hipErrorNotReady) return from_hip(q);
        if (timeout_ms != kInfinite) {
            auto ms = std::chrono::duration_cast<std::chrono::milliseconds>(
                          std::chrono::steady_clock::now() - start)
                          .count();
            if ((uint64_t)ms >= timeout_ms) return kTimeout;
        }
        if (++spins > 64) sched_yield();
    }
}

}  // namespace

struct gd_file {
    gd_context *owner;
    int fd = -1;
    uint64_t bytes = 0;
    uint64_t last_storage = 0;
};

struct gd_buffer {
    gd_context *owner;
    void *device = nullptr;  // device address seen by kernels
    void *host = nullptr;    // mapped host address (host kind only)
    uint64_t bytes = 0;
    uint64_t padded = 0;
    bool host_kind = false;
    bool external = false;  // gd_wrap_memory: the caller owns the memory
    uint32_t srv_index = UINT32_MAX;
    uint32_t uav_index = UINT32_MAX;
    uint64_t last_storage = 0;
    uint64_t last_compute = 0;
};

struct gd_pipeline {
    gd_context *owner;
    hipModule_t module = nullptr;
    hipFunction_t function = nullptr;
    uint32_t block[3] = {1, 1, 1};
};

struct Ticket {
    uint64_t value;
    hipEvent_t event;
};

struct gd_context {
    int device = 0;
    hipStream_t compute = nullptr;
    hipStream_t copy = nullptr;
    gd_caps caps{};
    uint32_t staging_bytes = 32u << 20;
    uint32_t queue_capacity = 1024;
    void *staging = nullptr;  // pinned host staging for file reads
    uint64_t *table = nullptr;  // device table of base pointers
    void *guard = nullptr;      // the block unassigned table entries point at (kGuardBytes)
    bool guard_check = false;   // enable_debug: gd_wait_compute checks the block
    std::vector<uint32_t> table_free;
    uint32_t table_next = 1;  // index 0 is never handed out
    std::vector<gd_buffer *> buffers;
    std::vector<gd_file *> files;
    std::vector<gd_pipeline *> pipelines;
    // Compute tickets: events recorded at submit, oldest first.
    uint64_t next_compute = 0;
    uint64_t completed_compute = 0;
    std::deque<Ticket> compute_events;
    uint64_t frame_ticket[3] = {0, 0, 0};
    uint32_t next_frame = 0;
    bool recording = false;
    // Storage tickets.
    uint64_t next_storage = 0;
    uint64_t completed_storage = 0;
    std::deque<Ticket> storage_events;
    // Timestamps: events of the recording, and of the last submission.
    std::vector<hipEvent_t> ts_pool;
    uint32_t ts_count = 0;
    uint32_t ts_submitted = 0;
    uint64_t ts_ticket = 0;
    std::vector<hipEvent_t> free_events;

    hipEvent_t take_event() {
        if (!free_events.empty()) {
            hipEvent_t e = free_events.back();
            free_events.pop_back();
            return e;
        }
        hipEvent_t e = nullptr;
        if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) return nullptr;
        return e;
    }

    // Retires finished compute tickets and returns the last completed value.
    uint64_t poll_compute() {
        while (!compute_events.empty()) {
            if (hipEventQuery(compute_events.front().event) != hipSuccess) break;
            completed_compute = compute_events.front().value;
            free_events.push_back(compute_events.front().event);
            compute_events.pop_front();
        }
        return completed_compute;
    }

    uint64_t poll_storage() {
        while (!storage_events.empty()) {
            if (hipEventQuery(storage_events.front().event) != hipSuccess) break;
            completed_storage = storage_events.front().value;
            free_events.push_back(storage_events.front().event);
            storage_events.pop_front();
        }
        return completed_storage;
    }

    gd_result wait_compute(uint64_t ticket, uint32_t timeout) {
        if (ticket <= poll_compute()) return kOk;
        for (auto &t : compute_events)
            if (t.value >= ticket) {
                GD_TRY(wait_event(t.event, timeout));
                poll_compute();
                return kOk;
            }
        return kOk;
    }

    // enable_debug: after the submissions up to `ticket` finished, any nonzero word of the
    // guard block means a dispatch wrote through an unassigned table index. The block is zeroed
    // again and the wait fails.
    gd_result check_guard() {
        if (!guard_check) return kOk;
        std::vector<uint64_t> words(kGuardBytes / 8);
        if (hipMemcpy(words.data(), guard, kGuardBytes, hipMemcpyDeviceToHost) != hipSuccess) return kFail;
        for (uint64_t w : words)
            if (w) {
                std::fprintf(stderr, "gyro_native: a dispatch wrote through an unassigned table index\n");
                if (hipMemset(guard, 0, kGuardBytes) != hipSuccess) return kDeviceRemoved;
                return kFail;
            }
        return kOk;
    }

    gd_result wait_storage(uint64_t ticket, uint32_t timeout) {
        if (ticket <= poll_storage()) return kOk;
        for (auto &t : storage_events)
            if (t.value >= ticket) {
                GD_TRY(wait_event(t.event, timeout));
                poll_storage();
                return kOk;
            }
        return kOk;
    }

    const hipEvent_t *find(std::deque<Ticket> &q, uint64_t ticket) {
        for (auto &t : q)
            if (t.value >= ticket) return &t.event;
        return nullptr;
    }

    uint32_t alloc_index() {
        if (!table_free.empty()) {
            uint32_t i = table_free.back();
            table_free.pop_back();
            return i;
        }
        if (table_next >= kTableCapacity) return UINT32_MAX;
        return table_next++;
    }

    gd_result set_index(uint32_t index, const void *ptr) {
        uint64_t v = (uint64_t)(uintptr_t)(ptr ? ptr : guard);
        // The table is read by kernels on the compute stream; order the update with them.
        GD_HIP(hipMemcpyAsync(table + index, &v, sizeof(v), hipMemcpyHostToDevice, compute));
        return hipStreamSynchronize(compute) == hipSuccess ? kOk : kFail;
    }
};

#define GD_CATCH                              \
    catch (const std::bad_alloc &) {          \
        return kOutOfMemory;                  \
    }                                         \
    catch (...) {                             \
        return kFail;                         \
    }

extern "C" gd_result gd_create(const gd_options *options, gd_context **out) {
    if (!out) return kInvalidArg;
    *out = nullptr;
    try {
        gd_options opts{};
        if (options) opts = *options;
        auto c = std::make_unique<gd_context>();
        if (opts.staging_bytes) c->staging_bytes = opts.staging_bytes;
        if (opts.queue_capacity) c->queue_capacity = opts.queue_capacity;
        if (c->queue_capacity < 128 || c->queue_capacity > 65536 ||
            (c->queue_capacity & (c->queue_capacity - 1)) != 0)
            return kInvalidArg;
        if (c->staging_bytes < 4096) return kInvalidArg;
        int count = 0;
        GD_HIP(hipGetDeviceCount(&count));
        if ((int)opts.adapter_index >= count) return kInvalidArg;
        c->device = (int)opts.adapter_index;
        GD_HIP(hipSetDevice(c->device));
        hipDeviceProp_t prop{};
        GD_HIP(hipGetDeviceProperties(&prop, c->device));
        c->caps.abi_version = 1;
        c->caps.vendor_id = 0x1002;
        c->caps.device_id = (uint32_t)strtoul(prop.gcnArchName + 3, nullptr, 16);
        c->caps.shader_model = 0x66;
        bool mfma = std::strncmp(prop.gcnArchName, "gfx9", 4) == 0;
        c->caps.linalg_tier = 0;
        c->caps.wave16_fp16_fp32_flags = mfma ? 1u : 0u;
        c->caps.vector_fp16_fp32_flags = 1;
        c->caps.experimental_features_enabled = 0;
        c->caps.dedicated_video_bytes = prop.totalGlobalMem;
        std::strncpy(c->caps.adapter_name, prop.name, sizeof(c->caps.adapter_name) - 1);
        if (opts.require_linalg && !mfma) return kUnsupported;
        GD_HIP(hipStreamCreateWithFlags(&c->compute, hipStreamNonBlocking));
        GD_HIP(hipStreamCreateWithFlags(&c->copy, hipStreamNonBlocking));
        GD_HIP(hipMalloc(&c->table, kTableCapacity * sizeof(uint64_t)));
        GD_HIP(hipMalloc(&c->guard, kGuardBytes));
        GD_HIP(hipMemset(c->guard, 0, kGuardBytes));
        {
            // Every entry names the guard block until a buffer takes it; read back to make sure
            // the table holds that before any dispatch can use it.
            std::vector<uint64_t> init(kTableCapacity, (uint64_t)(uintptr_t)c->guard);
            GD_HIP(hipMemcpy(c->table, init.data(), kTableCapacity * sizeof(uint64_t), hipMemcpyHostToDevice));
            std::vector<uint64_t> back(kTableCapacity, 0);
            GD_HIP(hipMemcpy(back.data(), c->table, kTableCapacity * sizeof(uint64_t), hipMemcpyDeviceToHost));
            if (back != init) return kFail;
        }
        c->guard_check = opts.enable_debug != 0;
        GD_HIP(hipHostMalloc(&c->staging, c->staging_bytes, hipHostMallocDefault));
        GD_HIP(hipStreamSynchronize(c->compute));
        size_t free_b = 0, total_b = 0;
        if (hipMemGetInfo(&free_b, &total_b) == hipSuccess) {
            c->caps.local_budget_bytes = total_b;
            c->caps.local_usage_bytes = total_b - free_b;
        }
        *out = c.release();
        return kOk;
    }
    GD_CATCH
}

extern "C" gd_result gd_get_caps(gd_context *c, gd_caps *out) {
    if (!c || !out) return kInvalidArg;
    GD_HIP(hipSetDevice(c->device));
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) == hipSuccess) {
        c->caps.local_budget_bytes = total_b;
        c->caps.local_usage_bytes = total_b - free_b;
    }
    *out = c->caps;
    return kOk;
}

extern "C" gd_result gd_open_file(gd_context *c, const char *path, gd_file **out) {
    if (!c || !path || !out) return kInvalidArg;
    *out = nullptr;
    try {
        int fd = open(path, O_RDONLY | O_CLOEXEC);
        if (fd < 0) return (gd_result)(0x80070000u | 2u);  // HRESULT_FROM_WIN32(FILE_NOT_FOUND)
        struct stat st{};
        if (fstat(fd, &st) != 0) {
            close(fd);
            return kFail;
        }
        auto f = std::make_unique<gd_file>();
        f->owner = c;
        f->fd = fd;
        f->bytes = (uint64_t)st.st_size;
        c->files.push_back(f.get());
        *out = f.release();
        return kOk;
    }
    GD_CATCH
}

extern "C" gd_result gd_file_size(gd_file *f, uint64_t *out) {
    if (!f || !out) return kInvalidArg;
    *out = f->bytes;
    return kOk;
}

extern "C" gd_result gd_create_buffer(gd_context *c, uint64_t bytes, gd_buffer **out) {
    if (!c || !out || !bytes || bytes > UINT64_MAX - 15) return kInvalidArg;
    *out = nullptr;
    try {
        auto b = std::make_unique<gd_buffer>();
        b->owner = c;
        b->bytes = bytes;
        b->padded = (bytes + 15) & ~uint64_t(15);
        GD_HIP(hipSetDevice(c->device));
        GD_HIP(hipMalloc(&b->device, b->padded));
        c->buffers.push_back(b.get());
        *out = b.release();
        return kOk;
    }
    GD_CATCH
}

extern "C" gd_result gd_poll(gd_context *c, uint64_t *storage_complete, uint64_t *compute_complete) {
    if (!c || !storage_complete || !compute_complete) return kInvalidArg;
    *storage_complete = c->poll_storage();
    *compute_complete = c->poll_compute();
    return kOk;
}

extern "C" gd_result gd_wait_storage(gd_context *c, uint64_t ticket, uint32_t timeout) {
    if (!c || ticket > c->next_storage) return kInvalidArg;
    return c->wait_storage(ticket, timeout);
}

// Copies ranges of a file into a buffer on the copy stream, after the given compute ticket.
static gd_result read_ranges(gd_context *c, gd_file *f, gd_buffer *b, const gd_range *ranges,
                             uint32_t count, uint64_t after_compute, bool check_overlap,
                             uint64_t *ticket) {
    for (uint32_t i = 0; i < count; ++i) {
        const gd_range &r = ranges[i];
        if (!r.bytes || r.reserved || r.bytes > c->staging_bytes || r.file_offset > f->bytes ||
            r.bytes > f->bytes - r.file_offset || r.buffer_offset > b->bytes ||
            r.bytes > b->bytes - r.buffer_offset)
            return kInvalidArg;
        if (check_overlap)
            for (uint32_t j = 0; j < i; ++j) {
                const gd_range &s = ranges[j];
                if (r.buffer_offset < s.buffer_offset + s.bytes &&
                    s.buffer_offset < r.buffer_offset + r.bytes)
                    return kInvalidArg;
            }
    }
    if (c->next_storage == UINT64_MAX - 1) return kUnexpected;
    GD_HIP(hipSetDevice(c->device));
    if (after_compute) {
        const hipEvent_t *ev = c->find(c->compute_events, after_compute);
        if (ev) GD_HIP(hipStreamWaitEvent(c->copy, *ev, 0));
    }
    for (uint32_t i = 0; i < count; ++i) {
        const gd_range &r = ranges[i];
        // The staging buffer is reused per range: the previous copy must have drained.
        GD_HIP(hipStreamSynchronize(c->copy));
        uint64_t done = 0;
        while (done < r.bytes) {
            ssize_t got = pread(f->fd, (char *)c->staging + done, r.bytes - done,
                                (off_t)(r.file_offset + done));
            if (got <= 0) return kFail;
            done += (uint64_t)got;
        }
        GD_HIP(hipMemcpyAsync((char *)b->device + r.buffer_offset, c->staging, r.bytes,
                              hipMemcpyHostToDevice, c->copy));
    }
    hipEvent_t ev = c->take_event();
    if (!ev) return kOutOfMemory;
    GD_HIP(hipEventRecord(ev, c->copy));
    uint64_t value = ++c->next_storage;
    c->storage_events.push_back({value, ev});
    b->last_storage = f->last_storage = *ticket = value;
    return kOk;
}

extern "C" gd_result gd_read_ranges(gd_context *c, gd_file *f, gd_buffer *b, const gd_range *ranges,
                                    uint32_t count, uint64_t *ticket) {
    if (!c || !f || !b || !ranges || !ticket || f->owner != c || b->owner != c || !count ||
        count > c->queue_capacity / 2 - 2)
        return kInvalidArg;
    *ticket = 0;
    try {
        if (b->last_storage > c->poll_storage()) return kBusy;
        return read_ranges(c, f, b, ranges, count, b->last_compute, true, ticket);
    }
    GD_CATCH
}

extern "C" gd_result gd_read_ranges_after(gd_context *c, gd_file *f, gd_buffer *b,
                                          const gd_range *ranges, uint32_t count,
                                          uint64_t compute_ticket, uint64_t *ticket) {
    if (!c || !f || !b || !ranges || !ticket || f->owner != c || b->owner != c || !count ||
        count > c->queue_capacity / 2 - 2 || compute_ticket > c->next_compute)
        return kInvalidArg;
    *ticket = 0;
    try {
        return read_ranges(c, f, b, ranges, count, compute_ticket, false, ticket);
    }
    GD_CATCH
}

extern "C" gd_result gd_queue_wait_storage(gd_context *c, uint64_t storage_ticket) {
    if (!c || storage_ticket > c->next_storage) return kInvalidArg;
    if (storage_ticket <= c->poll_storage()) return kOk;
    const hipEvent_t *ev = c->find(c->storage_events, storage_ticket);
    if (ev) GD_HIP(hipStreamWaitEvent(c->compute, *ev, 0));
    return kOk;
}

extern "C" gd_result gd_readback(gd_context *c, gd_buffer *b, uint64_t offset, uint32_t bytes,
                                 void *destination, uint32_t timeout) {
    if (!c || !b || b->owner != c || !destination || !bytes || offset > b->bytes ||
        bytes > b->bytes - offset)
        return kInvalidArg;
    try {
        GD_TRY(c->wait_storage(b->last_storage, timeout));
        GD_HIP(hipSetDevice(c->device));
        GD_HIP(hipMemcpyAsync(destination, (char *)b->device + offset, bytes, hipMemcpyDeviceToHost,
                              c->compute));
        hipEvent_t ev = c->take_event();
        if (!ev) return kOutOfMemory;
        GD_HIP(hipEventRecord(ev, c->compute));
        gd_result r = wait_event(ev, timeout);
        c->free_events.push_back(ev);
        return r;
    }
    GD_CATCH
}

// Loads a code object and resolves gd_main and its workgroup size.
static gd_result load_pipeline(gd_context *c, const void *code, size_t bytes, gd_pipeline *p) {
    const unsigned char *m = (const unsigned char *)code;
    bool elf = bytes >= 4 && m[0] == 0x7f && m[1] == 'E' && m[2] == 'L' && m[3] == 'F';
    bool bundle = bytes >= 24 && std::memcmp(m, "__CLANG_OFFLOAD_BUNDLE__", 24) == 0;
    if (!elf && !bundle) return kInvalidArg;
    GD_HIP(hipSetDevice(c->device));
    GD_HIP(hipModuleLoadData(&p->module, code));
    // The kernel is named by the module's gd_entry string (gd_main when absent).
    char entry[33] = "gd_main";
    hipDeviceptr_t name_ptr = nullptr;
    size_t name_bytes = 0;
    if (hipModuleGetGlobal(&name_ptr, &name_bytes, p->module, "gd_entry") == hipSuccess && name_bytes == 32) {
        if (hipMemcpyDtoH(entry, name_ptr, 32) != hipSuccess) entry[0] = 0;
        entry[32] = 0;
    }
    hipError_t e = hipModuleGetFunction(&p->function, p->module, entry);
    if (e != hipSuccess) {
        hipModuleUnload(p->module);
        p->module = nullptr;
        return kInvalidArg;
    }
    hipDeviceptr_t wg = nullptr;
    size_t wg_bytes = 0;
    e = hipModuleGetGlobal(&wg, &wg_bytes, p->module, "gd_workgroup");
    if (e != hipSuccess || wg_bytes != 12 ||
        hipMemcpyDtoH(p->block, wg, sizeof(p->block)) != hipSuccess || !p->block[0] ||
        !p->block[1] || !p->block[2] || p->block[0] * p->block[1] * p->block[2] > 1024) {
        hipModuleUnload(p->module);
        p->module = nullptr;
        return kInvalidArg;
    }
    return kOk;
}

extern "C" gd_result gd_create_pipeline(gd_context *c, const void *code, size_t bytes, gd_pipeline **out) {
    if (!c || !code || !bytes || !out) return kInvalidArg;
    *out = nullptr;
    try {
        auto p = std::make_unique<gd_pipeline>();
        p->owner = c;
        GD_TRY(load_pipeline(c, code, bytes, p.get()));
        c->pipelines.push_back(p.get());
        *out = p.release();
        return kOk;
    }
    GD_CATCH
}

extern "C" gd_result gd_release_pipeline(gd_context *c, gd_pipeline *p, uint32_t timeout) {
    if (!c || !p || p->owner != c) return kInvalidArg;
    GD_TRY(c->wait_compute(c->next_compute, timeout));
    GD_HIP(hipStreamSynchronize(c->compute));
    if (p->module) hipModuleUnload(p->module);
    c->pipelines.erase(std::find(c->pipelines.begin(), c->pipelines.end(), p));
    delete p;
    return kOk;
}

static gd_result launch(gd_context *c, gd_pipeline *p, const uint64_t *table, const uint32_t *constants,
                        uint32_t count, uint32_t x, uint32_t y, uint32_t z, hipStream_t stream,
                        hipEvent_t start = nullptr, hipEvent_t stop = nullptr) {
    GdArgs args;
    args.table = table;
    std::memset(args.c, 0, sizeof(args.c));
    if (count) std::memcpy(args.c, constants, count * sizeof(uint32_t));
    size_t size = sizeof(args);
    void *config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, &args, HIP_LAUNCH_PARAM_BUFFER_SIZE, &size,
                      HIP_LAUNCH_PARAM_END};
    if (start) {
        GD_HIP(hipExtModuleLaunchKernel(p->function, x * p->block[0], y * p->block[1], z * p->block[2], p->block[0],
                                        p->block[1], p->block[2], 0, stream, nullptr, config, start, stop, 0));
        return kOk;
    }
    GD_HIP(hipModuleLaunchKernel(p->function, x, y, z, p->block[0], p->block[1], p->block[2], 0,
                                 stream, nullptr, config));
    return kOk;
}

// gd_validate_gyro and gd_validate_linalg run a private pipeline on private buffers through
// a small private table.
struct Scoped {
    std::vector<void *> device;
    gd_pipeline pipe{};
    ~Scoped() {
        for (void *p : device) hipFree(p);
        if (pipe.module) hipModuleUnload(pipe.module);
    }
    void *alloc(size_t bytes) {
        void *p = nullptr;
        if (hipMalloc(&p, bytes) != hipSuccess) return nullptr;
        device.push_back(p);
        return p;
    }
};

extern "C" gd_result gd_validate_gyro(gd_context *c, const void *code, size_t code_bytes,
                                      const void *codebook, size_t codebook_bytes, const void *packed,
                                      size_t packed_bytes, uint32_t type_id, const float *expected,
                                      uint32_t value_count, float *max_error, uint32_t timeout) {
    static const uint32_t block_bytes_by_type[] = {34, 26, 30, 42, 50, 58, 22, 18};
    if (!c || !code || !code_bytes || !codebook || codebook_bytes != 8192 || !packed || !expected ||
        !max_error || type_id < 144 || type_id > 151 || !value_count || value_count % 128 != 0 ||
        value_count > 16777216)
        return kInvalidArg;
    const uint32_t blocks = value_count / 128;
    if (packed_bytes != (size_t)blocks * block_bytes_by_type[type_id - 144]) return kInvalidArg;
    for (uint32_t i = 0; i < value_count; ++i)
        if (!std::isfinite(expected[i])) return kInvalidArg;
    *max_error = std::numeric_limits<float>::infinity();
    try {
        Scoped s;
        s.pipe.owner = c;
        GD_TRY(load_pipeline(c, code, code_bytes, &s.pipe));
        const size_t packed_size = (packed_bytes + 15) & ~size_t(15);
        const size_t out_size = (size_t)value_count * 4;
        void *in = s.alloc(packed_size), *book = s.alloc(codebook_bytes), *out = s.alloc(out_size);
        uint64_t *table = (uint64_t *)s.alloc(3 * sizeof(uint64_t));
        if (!in || !book || !out || !table) return kOutOfMemory;
        std::vector<unsigned char> staged(packed_size, 0);
        std::memcpy(staged.data(), packed, packed_bytes);
        std::vector<uint32_t> sentinel(value_count, 0x7fc00000u);
        uint64_t ptrs[3] = {(uint64_t)(uintptr_t)in, (uint64_t)(uintptr_t)book, (uint64_t)(uintptr_t)out};
        hipStream_t st = c->compute;
        GD_HIP(hipMemcpyAsync(in, staged.data(), packed_size, hipMemcpyHostToDevice, st));
        GD_HIP(hipMemcpyAsync(book, codebook, codebook_bytes, hipMemcpyHostToDevice, st));
        GD_HIP(hipMemcpyAsync(out, sentinel.data(), out_size, hipMemcpyHostToDevice, st));
        GD_HIP(hipMemcpyAsync(table, ptrs, sizeof(ptrs), hipMemcpyHostToDevice, st));
        // Constants: input byte offset, block count, type id, output byte offset, then the
        // table slots of input, codebook and output, and the input and output sizes.
        const uint32_t constants[] = {0, blocks, type_id, 0, 0, 1, 2, (uint32_t)packed_size,
                                      (uint32_t)out_size};
        GD_TRY(launch(c, &s.pipe, table, constants, 9, (blocks + 63) / 64, 1, 1, st));
        std::vector<float> actual(value_count);
        GD_HIP(hipMemcpyAsync(actual.data(), out, out_size, hipMemcpyDeviceToHost, st));
        hipEvent_t ev = c->take_event();
        if (!ev) return kOutOfMemory;
        GD_HIP(hipEventRecord(ev, st));
        gd_result w = wait_event(ev, timeout);
        c->free_events.push_back(ev);
        GD_TRY(w);
        float error = 0;
        bool identical = true;
        for (uint32_t i = 0; i < value_count; ++i) {
            if (std::memcmp(&actual[i], &expected[i], 4) != 0) identical = false;
            if (!std::isfinite(actual[i]))
                error = std::numeric_limits<float>::infinity();
            else
                error = std::max(error, std::fabs(actual[i] - expected[i]));
        }
        *max_error = error;
        return identical ? kOk : kInvalidData;
    }
    GD_CATCH
}

extern "C" gd_result gd_validate_linalg(gd_context *c, const void *code, size_t code_bytes,
                                        float *max_error, uint32_t timeout) {
    if (!c || !code || !code_bytes || !max_error) return kInvalidArg;
    *max_error = std::numeric_limits<float>::infinity();
    if (!(c->caps.wave16_fp16_fp32_flags & 1u)) return kUnsupported;
    try {
        Scoped s;
        s.pipe.owner = c;
        GD_TRY(load_pipeline(c, code, code_bytes, &s.pipe));
        // Small integers are exact in binary16 (0, 1, 2, 3), as the reference uses.
        static const uint16_t half_values[] = {0, 0x3c00, 0x4000, 0x4200};
        uint16_t host[512];
        for (uint32_t i = 0; i < 256; ++i) {
            host[i] = half_values[(i * 3 + i / 16) % 4];
            host[256 + i] = half_values[(i + 2 * (i / 16)) % 4];
        }
        void *a = s.alloc(512), *b = s.alloc(512), *out = s.alloc(1024);
        uint64_t *table = (uint64_t *)s.alloc(3 * sizeof(uint64_t));
        if (!a || !b || !out || !table) return kOutOfMemory;
        uint64_t ptrs[3] = {(uint64_t)(uintptr_t)a, (uint64_t)(uintptr_t)b, (uint64_t)(uintptr_t)out};
        hipStream_t st = c->compute;
        GD_HIP(hipMemcpyAsync(a, host, 512, hipMemcpyHostToDevice, st));
        GD_HIP(hipMemcpyAsync(b, host + 256, 512, hipMemcpyHostToDevice, st));
        GD_HIP(hipMemsetAsync(out, 0xff, 1024, st));
        GD_HIP(hipMemcpyAsync(table, ptrs, sizeof(ptrs), hipMemcpyHostToDevice, st));
        const uint32_t constants[] = {0, 1, 2};
        GD_TRY(launch(c, &s.pipe, table, constants, 3, 1, 1, 1, st));
        float actual[256];
        GD_HIP(hipMemcpyAsync(actual, out, 1024, hipMemcpyDeviceToHost, st));
        hipEvent_t ev = c->take_event();
        if (!ev) return kOutOfMemory;
        GD_HIP(hipEventRecord(ev, st));
        gd_result w = wait_event(ev, timeout);
        c->free_events.push_back(ev);
        GD_TRY(w);
        float error = 0;
        for (uint32_t row = 0; row < 16; ++row)
            for (uint32_t col = 0; col < 16; ++col) {
                float expect = 0;
                for (uint32_t k = 0; k < 16; ++k) {
                    uint32_t ai = row * 16 + k, bi = k * 16 + col;
                    expect += float((ai * 3 + ai / 16) % 4) * float((bi + 2 * (bi / 16)) % 4);
                }
                float v = actual[row * 16 + col];
                if (!std::isfinite(v))
                    error = std::numeric_limits<float>::infinity();
                else
                    error = std::max(error, std::fabs(v - expect));
            }
        *max_error = error;
        return error == 0 ? kOk : kInvalidData;
    }
    GD_CATCH
}

extern "C" gd_result gd_create_resource(gd_context *c, uint64_t bytes, uint32_t kind, gd_buffer **out,
                                        gd_buffer_info *info) {
    if (!c || !out || !info || !bytes || kind > GD_RESOURCE_HOST) return kInvalidArg;
    *out = nullptr;
    *info = {};
    const uint64_t padded = (bytes + 255) & ~uint64_t(255);
    if (padded > (uint64_t(1) << 32)) return kInvalidArg;
    try {
        auto b = std::make_unique<gd_buffer>();
        b->owner = c;
        b->bytes = bytes;
        b->padded = padded;
        b->host_kind = kind == GD_RESOURCE_HOST;
        GD_HIP(hipSetDevice(c->device));
        if (b->host_kind) {
            GD_HIP(hipHostMalloc(&b->host, padded, hipHostMallocMapped | hipHostMallocCoherent));
            std::memset(b->host, 0, padded);
            GD_HIP(hipHostGetDevicePointer(&b->device, b->host, 0));
        } else {
            GD_HIP(hipMalloc(&b->device, padded));
        }
        b->srv_index = c->alloc_index();
        b->uav_index = c->alloc_index();
        if (b->srv_index == UINT32_MAX || b->uav_index == UINT32_MAX) {
            if (b->srv_index != UINT32_MAX) c->table_free.push_back(b->srv_index);
            if (b->uav_index != UINT32_MAX) c->table_free.push_back(b->uav_index);
            if (b->host_kind) hipHostFree(b->host); else hipFree(b->device);
            return kOutOfMemory;
        }
        GD_TRY(c->set_index(b->srv_index, b->device));
        GD_TRY(c->set_index(b->uav_index, b->device));
        info->srv_index = b->srv_index;
        info->uav_index = b->uav_index;
        info->mapped = b->host;
        info->gpu_address = (uint64_t)(uintptr_t)b->device;
        info->allocated_bytes = padded;
        c->buffers.push_back(b.get());
        *out = b.release();
        return kOk;
    }
    GD_CATCH
}

extern "C" gd_result gd_begin(gd_context *c, uint32_t timeout) {
    if (!c) return kInvalidArg;
    if (c->recording) return kIllegalCall;
    GD_TRY(c->wait_compute(c->frame_ticket[c->next_frame], timeout));
    GD_HIP(hipSetDevice(c->device));
    c->recording = true;
    c->ts_count = 0;
    return kOk;
}

extern "C" gd_result gd_dispatch(gd_context *c, gd_pipeline *p, const uint32_t *constants,
                                 uint32_t count, uint32_t x, uint32_t y, uint32_t z) {
    if (!c || !p || p->owner != c || !c->recording || count > kMaxConstants ||
        (count && !constants) || !x || !y || !z || x > 65535 || y > 65535 || z > 65535)
        return kInvalidArg;
    return launch(c, p, c->table, constants, count, x, y, z, c->compute);
}

// Reserves the next timestamp slot of the recording (events of a completed submission only).
static gd_result take_timestamp(gd_context *c, uint32_t *index) {
    if (c->ts_count >= kMaxTimestamps) return kOutOfMemory;
    while (c->ts_pool.size() <= c->ts_count) {
        hipEvent_t e = nullptr;
        GD_HIP(hipEventCreate(&e));
        c->ts_pool.push_back(e);
    }
    if (c->ts_ticket) GD_TRY(c->wait_compute(c->ts_ticket, kInfinite));
    c->ts_ticket = 0;
    *index = c->ts_count++;
    return kOk;
}

extern "C" gd_result gd_dispatch_timed(gd_context *c, gd_pipeline *p, const uint32_t *constants, uint32_t count,
                                       uint32_t x, uint32_t y, uint32_t z, uint32_t *out_index) {
    if (!c || !p || p->owner != c || !c->recording || count > kMaxConstants || (count && !constants) || !x ||
        !y || !z || x > 65535 || y > 65535 || z > 65535 || !out_index)
        return kInvalidArg;
    uint32_t first = 0, second = 0;
    GD_TRY(take_timestamp(c, &first));
    GD_TRY(take_timestamp(c, &second));
    *out_index = first;
    return launch(c, p, c->table, constants, count, x, y, z, c->compute, c->ts_pool[first], c->ts_pool[second]);
}

extern "C" gd_result gd_dispatch_on(gd_context *c, gd_pipeline *p, const uint32_t *constants, uint32_t count,
                                    uint32_t x, uint32_t y, uint32_t z, void *stream) {
    if (!c || !p || p->owner != c || count > kMaxConstants || (count && !constants) || !x || !y || !z ||
        x > 65535 || y > 65535 || z > 65535)
        return kInvalidArg;
    GD_HIP(hipSetDevice(c->device));
    return launch(c, p, c->table, constants, count, x, y, z, stream ? (hipStream_t)stream : c->compute);
}

extern "C" gd_result gd_wrap_memory(gd_context *c, void *device_address, uint64_t bytes, gd_buffer **out,
                                    gd_buffer_info *info) {
    if (!c || !out || !info || bytes > (uint64_t(1) << 32)) return kInvalidArg;
    *out = nullptr;
    *info = {};
    try {
        auto b = std::make_unique<gd_buffer>();
        b->owner = c;
        b->bytes = bytes;
        b->padded = bytes;
        b->external = true;
        b->device = device_address;
        b->srv_index = c->alloc_index();
        b->uav_index = c->alloc_index();
        if (b->srv_index == UINT32_MAX || b->uav_index == UINT32_MAX) {
            if (b->srv_index != UINT32_MAX) c->table_free.push_back(b->srv_index);
            if (b->uav_index != UINT32_MAX) c->table_free.push_back(b->uav_index);
            return kOutOfMemory;
        }
        GD_HIP(hipSetDevice(c->device));
        GD_TRY(c->set_index(b->srv_index, device_address));
        GD_TRY(c->set_index(b->uav_index, device_address));
        info->srv_index = b->srv_index;
        info->uav_index = b->uav_index;
        info->gpu_address = (uint64_t)(uintptr_t)device_address;
        info->allocated_bytes = bytes;
        c->buffers.push_back(b.get());
        *out = b.release();
        return kOk;
    }
    GD_CATCH
}

extern "C" gd_result gd_barrier(gd_context *c) {
    if (!c || !c->recording) return kInvalidArg;
    return kOk;  // the compute stream executes dispatches in order
}

extern "C" gd_result gd_timestamp(gd_context *c, uint32_t *out_index) {
    if (!c || !out_index || !c->recording) return kInvalidArg;
    // Events of the previous submission are reused only once it completed.
    GD_TRY(take_timestamp(c, out_index));
    GD_HIP(hipEventRecord(c->ts_pool[*out_index], c->compute));
    return kOk;
}

extern "C" gd_result gd_submit(gd_context *c, uint64_t *ticket) {
    if (!c || !ticket || !c->recording) return kInvalidArg;
    if (c->next_compute == UINT64_MAX - 1) return kUnexpected;
    hipEvent_t ev = c->take_event();
    if (!ev) return kOutOfMemory;
    GD_HIP(hipEventRecord(ev, c->compute));
    c->recording = false;
    *ticket = ++c->next_compute;
    c->compute_events.push_back({*ticket, ev});
    c->frame_ticket[c->next_frame] = *ticket;
    c->next_frame = (c->next_frame + 1) % 3;
    if (c->ts_count) {
        c->ts_submitted = c->ts_count;
        c->ts_ticket = *ticket;
    }
    return kOk;
}

extern "C" gd_result gd_wait_compute(gd_context *c, uint64_t ticket, uint32_t timeout) {
    if (!c || ticket > c->next_compute) return kInvalidArg;
    GD_TRY(c->wait_compute(ticket, timeout));
    return c->check_guard();
}

extern "C" gd_result gd_read_timestamps(gd_context *c, uint32_t count, uint64_t *out, uint64_t *frequency) {
    if (!c || !out || !frequency || count > kMaxTimestamps) return kInvalidArg;
    if (count > c->ts_submitted) return kInvalidArg;
    if (c->ts_ticket) GD_TRY(c->wait_compute(c->ts_ticket, kInfinite));
    for (uint32_t i = 0; i < count; ++i) {
        float ms = 0;
        if (i > 0) GD_HIP(hipEventElapsedTime(&ms, c->ts_pool[0], c->ts_pool[i]));
        out[i] = (uint64_t)std::llround((double)ms * 1e6);
    }
    *frequency = 1000000000ull;
    return kOk;
}

extern "C" gd_result gd_release_buffer(gd_context *c, gd_buffer *b, uint32_t timeout) {
    if (!c || !b || b->owner != c) return kInvalidArg;
    GD_TRY(c->wait_storage(b->last_storage, timeout));
    // Bindless dispatches do not record which buffers they touch: wait for all compute work.
    GD_TRY(c->wait_compute(c->next_compute, timeout));
    if (hipStreamSynchronize(c->compute) != hipSuccess) return kFail;
    if (b->srv_index != UINT32_MAX) {
        c->set_index(b->srv_index, nullptr);
        c->table_free.push_back(b->srv_index);
    }
    if (b->uav_index != UINT32_MAX) {
        c->set_index(b->uav_index, nullptr);
        c->table_free.push_back(b->uav_index);
    }
    if (b->external) {
    } else if (b->host_kind) {
        hipHostFree(b->host);
    } else {
        hipFree(b->device);
    }
    c->buffers.erase(std::find(c->buffers.begin(), c->buffers.end(), b));
    delete b;
    return kOk;
}

extern "C" gd_result gd_release_file(gd_context *c, gd_file *f, uint32_t timeout) {
    if (!c || !f || f->owner != c) return kInvalidArg;
    GD_TRY(c->wait_storage(f->last_storage, timeout));
    close(f->fd);
    c->files.erase(std::find(c->files.begin(), c->files.end(), f));
    delete f;
    return kOk;
}

extern "C" gd_result gd_destroy(gd_context *c, uint32_t timeout) {
    if (!c) return kOk;
    GD_TRY(c->wait_storage(c->next_storage, timeout));
    GD_TRY(c->wait_compute(c->next_compute, timeout));
    hipSetDevice(c->device);
    hipStreamSynchronize(c->compute);
    hipStreamSynchronize(c->copy);
    for (gd_pipeline *p : c->pipelines) {
        if (p->module) hipModuleUnload(p->module);
        delete p;
    }
    for (gd_buffer *b : c->buffers) {
        if (b->external) {
        } else if (b->host_kind) {
            hipHostFree(b->host);
        } else {
            hipFree(b->device);
        }
        delete b;
    }
    for (gd_file *f : c->files) {
        close(f->fd);
        delete f;
    }
    for (auto &t : c->compute_events) hipEventDestroy(t.event);
    for (auto &t : c->storage_events) hipEventDestroy(t.event);
    for (hipEvent_t e : c->free_events) hipEventDestroy(e);
    for (hipEvent_t e : c->ts_pool) hipEventDestroy(e);
    hipFree(c->table);
    hipFree(c->guard);
    hipHostFree(c->staging);
    hipStreamDestroy(c->compute);
    hipStreamDestroy(c->copy);
    delete c;
    return kOk;
}
