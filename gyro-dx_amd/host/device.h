// Host wrapper over the gyro_native C ABI, restating src/gpu.zig:1-159: `check` turns a
// negative result into an error that carries the code, Device owns one context, buffers are
// at least 256 bytes, and every call uses the reference's 60-second timeout.
#pragma once
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "gyro_native.h"

namespace gyro {

constexpr uint32_t kTimeoutMs = 60000;  // src/gpu.zig:5

struct NativeError : std::runtime_error {
    gd_result code;
    NativeError(gd_result c, const std::string &what) : std::runtime_error(what), code(c) {}
};

// src/gpu.zig:7-13.
void check(gd_result result, const char *what);

struct Buffer {
    gd_buffer *handle = nullptr;
    uint32_t srv = 0, uav = 0;
    uint64_t bytes = 0;
    uint64_t gpu = 0;
    uint8_t *mapped = nullptr;
    float *floats() const { return reinterpret_cast<float *>(mapped); }
    uint32_t *words() const { return reinterpret_cast<uint32_t *>(mapped); }
};

enum class Kind : uint32_t { device = GD_RESOURCE_DEVICE, host = GD_RESOURCE_HOST };

class Device {
  public:
    gd_context *ctx = nullptr;
    gd_caps caps{};
    uint64_t allocated_device_bytes = 0;
    uint64_t allocated_host_bytes = 0;

    void init(uint32_t adapter);  // src/gpu.zig:41-53
    void deinit();
    Buffer buffer(uint64_t bytes, Kind kind);  // src/gpu.zig:68-75
    // Table entries for memory owned elsewhere (gd_wrap_memory); release frees the entries only.
    Buffer wrap(void *device_address, uint64_t bytes);
    void release(Buffer &b);
    gd_pipeline *pipeline(const std::vector<uint8_t> &code);  // src/gpu.zig:81-85
    void begin();
    void dispatch(gd_pipeline *p, const uint32_t *constants, uint32_t count, uint32_t x, uint32_t y,
                  uint32_t z);
    // Dispatch whose own start and end become timestamps (returns the first index).
    uint32_t dispatch_timed(gd_pipeline *p, const uint32_t *constants, uint32_t count, uint32_t x, uint32_t y,
                            uint32_t z);
    void barrier();
    uint32_t timestamp();
    uint64_t submit();
    void wait(uint64_t ticket);
    uint64_t timestamps(uint64_t *out, uint32_t count);  // returns the tick frequency
};

}  // namespace gyro
