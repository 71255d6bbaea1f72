#include "device.h"

#include <cstdio>

namespace gyro {

void check(gd_result result, const char *what) {
    if (result < 0) {
        char msg[256];
        std::snprintf(msg, sizeof(msg), "%s: native result 0x%08x", what, (uint32_t)result);
        throw NativeError(result, msg);
    }
}

void Device::init(uint32_t adapter) {
    gd_options opts{adapter, 0, 0, 32u << 20, 1024};
    check(gd_create(&opts, &ctx), "gd_create");
    check(gd_get_caps(ctx, &caps), "gd_get_caps");
    if (caps.shader_model < 0x66) {
        gd_destroy(ctx, kTimeoutMs);
        ctx = nullptr;
        throw NativeError(-1, "shader model 6.6 contract required");
    }
}

void Device::deinit() {
    if (ctx) gd_destroy(ctx, kTimeoutMs);
    ctx = nullptr;
}

Buffer Device::buffer(uint64_t bytes, Kind kind) {
    const uint64_t size = bytes < 256 ? 256 : bytes;
    gd_buffer *handle = nullptr;
    gd_buffer_info info{};
    check(gd_create_resource(ctx, size, (uint32_t)kind, &handle, &info), "gd_create_resource");
    if (kind == Kind::device)
        allocated_device_bytes += info.allocated_bytes;
    else
        allocated_host_bytes += info.allocated_bytes;
    Buffer b;
    b.handle = handle;
    b.srv = info.srv_index;
    b.uav = info.uav_index;
    b.bytes = size;
    b.gpu = info.gpu_address;
    b.mapped = static_cast<uint8_t *>(info.mapped);
    return b;
}

Buffer Device::wrap(void *device_address, uint64_t bytes) {
    gd_buffer *handle = nullptr;
    gd_buffer_info info{};
    check(gd_wrap_memory(ctx, device_address, bytes, &handle, &info), "gd_wrap_memory");
    Buffer b;
    b.handle = handle;
    b.srv = info.srv_index;
    b.uav = info.uav_index;
    b.bytes = bytes;
    b.gpu = info.gpu_address;
    return b;
}

void Device::release(Buffer &b) {
    if (b.handle) gd_release_buffer(ctx, b.handle, kTimeoutMs);
    b = Buffer{};
}

gd_pipeline *Device::pipeline(const std::vector<uint8_t> &code) {
    gd_pipeline *p = nullptr;
    check(gd_create_pipeline(ctx, code.data(), code.size(), &p), "gd_create_pipeline");
    return p;
}

void Device::begin() { check(gd_begin(ctx, kTimeoutMs), "gd_begin"); }

void Device::dispatch(gd_pipeline *p, const uint32_t *constants, uint32_t count, uint32_t x, uint32_t y,
                      uint32_t z) {
    check(gd_dispatch(ctx, p, constants, count, x, y, z), "gd_dispatch");
}

uint32_t Device::dispatch_timed(gd_pipeline *p, const uint32_t *constants, uint32_t count, uint32_t x, uint32_t y,
                                uint32_t z) {
    uint32_t index = 0;
    check(gd_dispatch_timed(ctx, p, constants, count, x, y, z, &index), "gd_dispatch_timed");
    return index;
}

void Device::barrier() { check(gd_barrier(ctx), "gd_barrier"); }

uint32_t Device::timestamp() {
    uint32_t index = 0;
    check(gd_timestamp(ctx, &index), "gd_timestamp");
    return index;
}

uint64_t Device::submit() {
    uint64_t ticket = 0;
    check(gd_submit(ctx, &ticket), "gd_submit");
    return ticket;
}

void Device::wait(uint64_t ticket) { check(gd_wait_compute(ctx, ticket, kTimeoutMs), "gd_wait_compute"); }

uint64_t Device::timestamps(uint64_t *out, uint32_t count) {
    uint64_t frequency = 0;
    check(gd_read_timestamps(ctx, count, out, &frequency), "gd_read_timestamps");
    return frequency;
}

}  // namespace gyro
