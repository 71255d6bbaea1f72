/*
 * gyro_gguf: the GGUF v3 header reader and expert slicing of src/gguf.zig, for loading a real
 * model's routed experts into a gm_engine layer (gm_layer_desc takes one pointer per expert
 * projection: the bytes of expert e's slice of "blk.<l>.ffn_{gate,up,down}_exps.weight").
 *
 * The reader parses the header prefix of a file (at most 64 MiB), checks it as src/gguf.zig:263-330
 * does and returns 0 or a negative gg_error. No tensor data is read.
 */
#ifndef GYRO_GGUF_H
#define GYRO_GGUF_H

#include <stddef.h>
#include <stdint.h>

#define GG_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

/* src/gguf.zig:6-11 (ParseError), in that order. */
enum gg_error {
    GG_OK = 0,
    GG_UNEXPECTED_END = -1,
    GG_BAD_MAGIC = -2,
    GG_UNSUPPORTED_VERSION = -3,
    GG_INVALID_TYPE = -4,
    GG_INVALID_BOOLEAN = -5,
    GG_LIMIT_EXCEEDED = -6,
    GG_INTEGER_OVERFLOW = -7,
    GG_INVALID_ALIGNMENT = -8,
    GG_INVALID_DIMENSIONS = -9,
    GG_DUPLICATE_KEY = -10,
    GG_DUPLICATE_TENSOR = -11,
    GG_INVALID_TENSOR_RANGE = -12,
    GG_OVERLAPPING_TENSORS = -13,
    GG_UNSUPPORTED_TENSOR_TYPE = -14,
    GG_INVALID_EXPERT = -15,
    GG_INVALID_METADATA = -16,
    GG_IO = -17, /* the file could not be opened or read (gg_open only) */
    GG_NOT_FOUND = -18,
    GG_UNSUPPORTED_GYRO_METADATA = -19,
    GG_OUT_OF_MEMORY = -20, /* an allocation failed (the reference's allocator error) */
};

typedef struct gg_model gg_model;

/* src/gguf.zig:128-136 (Tensor). byte_length is UINT64_MAX for a type without a known layout
 * (src/gguf.zig:113-125: F32, F16, Q8_0, BF16 and the eight Gyro types). */
typedef struct gg_tensor_info {
    const char *name; /* NUL-terminated copy owned by the model */
    uint32_t rank;
    uint64_t dims[4];
    uint32_t type_id;
    uint64_t relative_offset;
    uint64_t file_offset;
    uint64_t byte_length;
} gg_tensor_info;

/* Replaces src/gguf.zig:263 `parse`: prefix holds the file's first bytes (the whole header),
 * file_size is the full file size. */
GG_API int gg_parse(const uint8_t *prefix, size_t prefix_len, uint64_t file_size, gg_model **out);
/* Reads the header prefix of a file (up to 64 MiB) and parses it. */
GG_API int gg_open(const char *path, gg_model **out);
GG_API void gg_free(gg_model *m);
GG_API uint32_t gg_version(const gg_model *m);
GG_API uint32_t gg_alignment(const gg_model *m);
GG_API uint64_t gg_data_offset(const gg_model *m);
/* Tensors in increasing file-offset order (src/gguf.zig:322). */
GG_API uint32_t gg_tensor_count(const gg_model *m);
GG_API int gg_tensor_at(const gg_model *m, uint32_t index, gg_tensor_info *out);
GG_API int gg_find_tensor(const gg_model *m, const char *name, gg_tensor_info *out);
/* src/gguf.zig:138-143 (Tensor.expertRange): the file range of expert `expert` of a rank-3
 * tensor, an equal 1 / dims[2] share of its bytes. */
GG_API int gg_expert_range(const gg_model *m, const char *name, uint32_t expert, uint64_t *file_offset,
                           uint64_t *bytes);
/* src/gguf.zig:145-151 (Tensor.isExpert): 1 for the three routed-expert tensor suffixes. */
GG_API int gg_is_expert_tensor(const char *name);
/* src/gguf.zig:70-77 (Entry.unsigned): an unsigned integer metadata value. */
GG_API int gg_metadata_u64(const gg_model *m, const char *key, uint64_t *out);

/* A metadata entry's value type (src/gguf.zig:13-17) and its raw value bytes (for arrays: the
 * element type, the count and the elements), owned by the model. */
GG_API int gg_metadata_raw(const gg_model *m, const char *key, uint32_t *kind, const uint8_t **raw, size_t *len);
/* src/gguf.zig:182-250 (Model.validateGyro): the released version-1 rotation metadata of a file
 * holding Gyro tensors (Trellis state bits 15, normalized Sylvester Walsh-Hadamard blocks along
 * the input's last dimension, explicit or identity signs, every listed tensor present with a
 * width the signs cover). 0, GG_INVALID_METADATA or GG_UNSUPPORTED_GYRO_METADATA. */
GG_API int gg_validate_gyro(const gg_model *m);

#ifdef __cplusplus
}
#endif
#endif
