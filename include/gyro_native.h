/*
 * gyro_native: the C ABI between the Gyro DX engine and the GPU, implemented for MI355X
 * (gfx950) on HIP. Drop-in replacement for the reference bridge: the entry points, argument
 * meanings, struct layouts and HRESULT-style results are those of the reference header
 * native/include/gyro_native.h:19-137, which src/native_abi.zig:50-85 mirrors.
 *
 * MI355X mapping:
 *  - A context owns one device, one in-order compute stream and one copy stream (both at the
 *    default priority).
 *  - Resources are device memory (hipMalloc) or pinned, mapped host memory (hipHostMalloc).
 *    Each receives two indices (SRV and UAV) into a device-resident table of 65,536 base
 *    pointers; both indices name the same memory.
 *  - A pipeline is a gfx950 code object exporting one kernel taking GdArgs, a `gd_workgroup[3]`
 *    constant and a `gd_entry` string naming the kernel (default `gd_main`); GdArgs is
 *    {const uint64_t *table; uint32_t constants[60];}.
 *  - gd_dispatch launches immediately on the compute stream; gd_barrier is a no-op because
 *    the stream is in order; gd_submit records an event and returns its ticket.
 *  - File reads use pread into pinned staging and asynchronous copies on the copy stream.
 *
 * All methods require serialized access to each context. Results: 0 on success, negative
 * HRESULT codes on failure (E_INVALIDARG 0x80070057, E_OUTOFMEMORY 0x8007000E, E_FAIL
 * 0x80004005, E_PENDING 0x8000000A, timeout 0x80070102, ERROR_BUSY 0x800700AA,
 * ERROR_INVALID_DATA 0x8007000D, unsupported 0x887A0004, E_ILLEGAL_METHOD_CALL 0x8000000E).
 */
#ifndef GYRO_NATIVE_H
#define GYRO_NATIVE_H

#include <stddef.h>
#include <stdint.h>

#define GD_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gd_context gd_context;
typedef struct gd_file gd_file;
typedef struct gd_buffer gd_buffer;
typedef struct gd_pipeline gd_pipeline;
typedef int32_t gd_result;

/* 20 bytes (src/native_abi.zig:89). */
typedef struct gd_options {
    uint32_t adapter_index;  /* HIP device ordinal */
    uint32_t enable_debug;   /* nonzero: gd_wait_compute fails (E_FAIL) when a finished dispatch
                                wrote through a table index that names no buffer (such indices
                                point at a zeroed guard block, never at address 0) */
    uint32_t require_linalg; /* fail creation if MFMA fp16 is unavailable */
    uint32_t staging_bytes;  /* pinned staging per file read (>= 4096; default 32 MiB) */
    uint32_t queue_capacity; /* power of two in [128, 65536]; bounds ranges per read */
} gd_options;

/* 184 bytes, adapter_name at offset 56 (src/native_abi.zig:90,92). */
typedef struct gd_caps {
    uint32_t abi_version;
    uint32_t vendor_id;      /* 0x1002 */
    uint32_t device_id;      /* gfx target number, 0x950 on MI355X */
    uint32_t shader_model;   /* 0x66: the bindless dispatch contract is available */
    uint32_t linalg_tier;
    uint32_t wave16_fp16_fp32_flags; /* bit 0: MFMA fp16 x fp16 -> fp32 */
    uint32_t vector_fp16_fp32_flags;
    uint32_t experimental_features_enabled;
    uint64_t dedicated_video_bytes;
    uint64_t local_budget_bytes;
    uint64_t local_usage_bytes;
    char adapter_name[128];
} gd_caps;

/* 24 bytes (src/native_abi.zig:91). */
typedef struct gd_range {
    uint64_t file_offset;
    uint64_t buffer_offset;
    uint32_t bytes;
    uint32_t reserved;
} gd_range;

enum { GD_RESOURCE_DEVICE = 0, GD_RESOURCE_HOST = 1 };

/* 32 bytes, mapped at offset 8 (src/native_abi.zig:93-94). */
typedef struct gd_buffer_info {
    uint32_t srv_index;
    uint32_t uav_index;
    void *mapped;
    uint64_t gpu_address;
    uint64_t allocated_bytes;
} gd_buffer_info;

/* Replaces gd_create (reference native/gyro_native.cpp:266-392). */
GD_API gd_result gd_create(const gd_options *options, gd_context **out_context);
/* Replaces gd_get_caps (:394-406); refreshes the memory budget and usage. */
GD_API gd_result gd_get_caps(gd_context *context, gd_caps *out_caps);
/* Replaces gd_open_file (:408-427): a read-only POSIX file. */
GD_API gd_result gd_open_file(gd_context *context, const char *utf8_path, gd_file **out_file);
/* Replaces gd_file_size (:429-433). */
GD_API gd_result gd_file_size(gd_file *file, uint64_t *out_bytes);
/* Replaces gd_create_buffer (:435-449): device memory without table entries. */
GD_API gd_result gd_create_buffer(gd_context *context, uint64_t bytes, gd_buffer **out_buffer);
/* Replaces gd_read_ranges (:463-503): raw byte transfers from a file into a buffer, ordered
 * after the buffer's last compute use. ERROR_BUSY if the buffer has an unfinished read. */
GD_API gd_result gd_read_ranges(gd_context *context, gd_file *file, gd_buffer *buffer,
    const gd_range *ranges, uint32_t count, uint64_t *out_storage_ticket);
/* Replaces gd_poll (:451-456). */
GD_API gd_result gd_poll(gd_context *context, uint64_t *storage_completed, uint64_t *compute_completed);
/* Replaces gd_wait_storage (:458-461). */
GD_API gd_result gd_wait_storage(gd_context *context, uint64_t ticket, uint32_t timeout_ms);
/* Replaces gd_readback (:505-530): copies device bytes to host memory after prior work. */
GD_API gd_result gd_readback(gd_context *context, gd_buffer *buffer, uint64_t offset,
    uint32_t bytes, void *destination, uint32_t timeout_ms);
/* Replaces gd_validate_linalg (:532-595): the code object must come from the linalg_smoke
 * kernel; one 16x16x16 fp16 MFMA product is compared exactly against the CPU. */
GD_API gd_result gd_validate_linalg(gd_context *context, const void *code, size_t code_bytes,
    float *out_max_abs_error, uint32_t timeout_ms);
/* Replaces gd_validate_gyro (:597-729): the code object must come from the gyro_decode
 * kernel. value_count is a positive multiple of 128 (at most 16,777,216), packed_bytes must
 * match the type and block count, expected holds finite fp32 values; any bitwise difference
 * fails with ERROR_INVALID_DATA. */
GD_API gd_result gd_validate_gyro(gd_context *context, const void *code, size_t code_bytes,
    const void *codebook, size_t codebook_bytes, const void *packed, size_t packed_bytes,
    uint32_t type_id, const float *expected, uint32_t value_count,
    float *out_max_abs_error, uint32_t timeout_ms);
/* Replaces gd_create_resource (:763-847). Sizes are padded to 256 bytes and limited to 4 GiB
 * (kernels use 32-bit byte offsets). Host resources are zero-filled. */
GD_API gd_result gd_create_resource(gd_context *context, uint64_t bytes, uint32_t kind,
    gd_buffer **out_buffer, gd_buffer_info *out_info);
/* Replaces gd_create_pipeline (:849-864): code is a gfx950 code object (ELF or offload
 * bundle) exporting its kernel, gd_entry and gd_workgroup. */
GD_API gd_result gd_create_pipeline(gd_context *context, const void *code, size_t code_bytes,
    gd_pipeline **out_pipeline);
/* Replaces gd_release_pipeline (:866-872). */
GD_API gd_result gd_release_pipeline(gd_context *context, gd_pipeline *pipeline, uint32_t timeout_ms);
/* Replaces gd_begin (:874-889): at most three submissions in flight; nesting is refused. */
GD_API gd_result gd_begin(gd_context *context, uint32_t timeout_ms);
/* Replaces gd_dispatch (:891-900): at most 60 constants, grid dimensions 1..65535. */
GD_API gd_result gd_dispatch(gd_context *context, gd_pipeline *pipeline, const uint32_t *constants,
    uint32_t constant_count, uint32_t groups_x, uint32_t groups_y, uint32_t groups_z);
/* Replaces gd_barrier (:902-909). */
GD_API gd_result gd_barrier(gd_context *context);
/* Replaces gd_timestamp (:911-917): up to 4096 marks per submission. */
GD_API gd_result gd_timestamp(gd_context *context, uint32_t *out_index);
/* Replaces gd_submit (:919-934). */
GD_API gd_result gd_submit(gd_context *context, uint64_t *out_compute_ticket);
/* Replaces gd_wait_compute (:936-939). With gd_options.enable_debug, also E_FAIL when a dispatch
 * finished by `ticket` wrote through an unassigned table index (the guard block is then cleared). */
GD_API gd_result gd_wait_compute(gd_context *context, uint64_t ticket, uint32_t timeout_ms);
/* Replaces gd_read_timestamps (:941-951): ticks of the last completed submission's marks, in
 * nanoseconds relative to its first mark (frequency 1e9). */
GD_API gd_result gd_read_timestamps(gd_context *context, uint32_t count, uint64_t *out_ticks,
    uint64_t *out_frequency);
/* Replaces gd_queue_wait_storage (:953-956). */
GD_API gd_result gd_queue_wait_storage(gd_context *context, uint64_t storage_ticket);
/* Replaces gd_read_ranges_after (:958-994). */
GD_API gd_result gd_read_ranges_after(gd_context *context, gd_file *file, gd_buffer *buffer,
    const gd_range *ranges, uint32_t count, uint64_t compute_ticket, uint64_t *out_storage_ticket);
/* Replaces gd_release_buffer (:731-742). */
GD_API gd_result gd_release_buffer(gd_context *context, gd_buffer *buffer, uint32_t timeout_ms);
/* Replaces gd_release_file (:744-750). */
GD_API gd_result gd_release_file(gd_context *context, gd_file *file, uint32_t timeout_ms);
/* Replaces gd_destroy (:752-759). */
GD_API gd_result gd_destroy(gd_context *context, uint32_t timeout_ms);

/* Extension with no counterpart in the reference ABI, for profilers and benchmarks: as
 * gd_dispatch, and records the dispatch's own start and end as timestamps *out_index and
 * *out_index + 1 of the recording (read with gd_read_timestamps), without adding packets
 * between dispatches. */
GD_API gd_result gd_dispatch_timed(gd_context *context, gd_pipeline *pipeline, const uint32_t *constants,
    uint32_t constant_count, uint32_t groups_x, uint32_t groups_y, uint32_t groups_z, uint32_t *out_index);

/* Extension with no counterpart in the reference ABI, for callers that run outside a recording
 * (the MoE engine's no-allocation entry point): launches at once on `stream`, a hipStream_t of
 * the context's device (NULL: the context's compute stream), with the checks of gd_dispatch but
 * no gd_begin / gd_submit bracket and no ticket. */
GD_API gd_result gd_dispatch_on(gd_context *context, gd_pipeline *pipeline, const uint32_t *constants,
    uint32_t constant_count, uint32_t groups_x, uint32_t groups_y, uint32_t groups_z, void *stream);
/* Extension with no counterpart in the reference ABI: gives memory the caller owns (device
 * address, may be NULL until a kernel writes the entry) SRV and UAV table indices, as
 * gd_create_resource does for memory it allocates. gd_release_buffer frees the indices only. */
GD_API gd_result gd_wrap_memory(gd_context *context, void *device_address, uint64_t bytes,
    gd_buffer **out_buffer, gd_buffer_info *out_info);

#ifdef __cplusplus
}
#endif
#endif
