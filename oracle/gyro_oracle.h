/*
 * CPU oracle for the routed-expert MoE path: TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU engine for this path. Only tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py may load it, and only as the
 * checker or the timed CPU baseline. The product (gyro-dx_amd/) never links or calls it.
 *
 * Every function cites the reference file:line it restates. What pins each function, that is
 * what fixes its output independently of this restatement (tests named are under tests/):
 *   go_init              codebook SHA-256 of src/gyro.zig:197-202 (test_codebook_hash).
 *   go_type_info,        type table and sizes through the golden fixture's 8 types and
 *   go_row_bytes         src/gyro.zig:204-214 (test_golden_decode_all_bits, test_fail_closed).
 *   go_fp16_to_fp32      src/gyro.zig:216-224 edge bits and numpy's exact binary16 conversion
 *                        (test_fp16_edges).
 *   go_trellis_state,    all 65,536 value bits of tests/gyro_vectors.bin (512 blocks, 8 types,
 *   go_decode_row        edge scales), the SPEC.md section 10 worked examples, and the vendored
 *                        C decoder third_party/agention-gyro/src/tq_ref.c built into oracle/_ref
 *                        (test_golden_decode_all_bits, test_spec_worked_examples,
 *                        test_against_vendored_reference_decoder).
 *   go_rotate,           rotation bit patterns of tests/gyro_vectors.bin, the closed form
 *   go_unrotate,         H[r][c] = (-1)^popcount(r&c)/sqrt(b), H.H = I and dot invariance
 *   go_rotate_f32signs   (test_golden_rotation_bits, test_rotation_closed_forms).
 *   go_softmax, go_topk  brute-force fp64 sort with lower-index ties (test_topk_ties_and_brute_force).
 *   go_dot_row,          fp64 dot of the strictly decoded row, to fp32 reduction tolerance
 *   go_decode_row_fast,  (test_fused_dot_matches_strict_decoder); their exact bits follow the
 *   go_dot_f32           reference's fast-math reductions and are parity unpinned bit-for-bit.
 *   go_silu, go_sigmoid, an independent fp64 numpy model of the layer with planted-mistake
 *   go_moe_ffn           checks (test_layer_matches_numpy_fp64, test_mixed_types_and_bias,
 *                        test_counting_sort_invariants, test_layer_thread_count_invariant).
 *   go_moe_dense_f64,    the same fp64 numpy model and numpy's x.W^T for the router logits
 *   go_router_f64        (test_layer_matches_numpy_fp64).
 *   go_dot_bf16          the bf16 shared expert against an fp64 numpy model of its algebra
 *                        (test_shared_expert_matches_numpy).
 *   go_rms_norm          closed forms (a constant row c gives sign(c) / sqrt(1 + eps / c^2) * w;
 *                        unit mean square at eps = 0; scale invariance) and an fp64 numpy model,
 *                        with planted mistakes (sum for mean, a dropped weight) that must fail
 *                        (test_rms_norm_closed_forms); the stack of layers is pinned through it
 *                        and the layer (test_stack_matches_numpy).
 */
#ifndef GYRO_ORACLE_H
#define GYRO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error codes mirror the error set of src/gyro.zig:43-53. */
enum {
    GO_OK = 0,
    GO_UNSUPPORTED_TYPE = -1,
    GO_MISSING_STATE_BITS = -2,
    GO_UNSUPPORTED_STATE_BITS = -3,
    GO_INVALID_ROW_LENGTH = -4,
    GO_INVALID_SOURCE_LENGTH = -5,
    GO_INVALID_BLOCK_SIZE = -7,
    GO_INVALID_SIGNS_LENGTH = -8,
    GO_INVALID_SIGN = -9,
};

/* Installs the normative codebook (8192 bytes of little-endian binary16, src/gyro_codebook.f16)
 * and expands it to fp32 as src/kernels.zig:14-23 does. Returns GO_INVALID_SOURCE_LENGTH if the
 * length is not 8192. Must be called before any decode. */
int go_init(const uint8_t *codebook, size_t len);

/* Type table (src/gyro.zig:32-41): returns 0 for an unknown id. */
int go_type_info(uint32_t id, uint32_t *k, uint32_t *steps, uint32_t *block_bytes);
/* src/gyro.zig:70-76; 0 on error. */
uint64_t go_row_bytes(uint32_t id, uint64_t weights);
/* src/gyro.zig:127-141. */
float go_fp16_to_fp32(uint16_t half);
/* src/gyro.zig:107-117. */
uint32_t go_trellis_state(uint32_t id, const uint8_t *stream, uint32_t step);
/* Strict decoder, src/gyro.zig:81-105. state_bits < 0 means "missing". */
int go_decode_row(uint32_t id, int32_t state_bits, const uint8_t *src, size_t src_len,
                  float *dst, size_t n);
/* Strict rotation, src/gyro.zig:143-195. signs may be NULL (identity). */
int go_rotate(float *v, size_t n, size_t block, const int8_t *signs);
int go_unrotate(float *v, size_t n, size_t block, const int8_t *signs);

/* Engine-level helpers (src/kernels.zig). */
void go_rotate_f32signs(float *x, size_t n, size_t block, const float *signs); /* :316-338 */
void go_softmax(float *x, size_t n);                                             /* :340-349 */
float go_silu(float x);                                                          /* :307-309 */
float go_sigmoid(float x);                                                       /* :303-305 */
float go_dot_f32(const float *row, const float *x, size_t n);                    /* :72-84 */
float go_dot_bf16(const uint16_t *row, const float *x, size_t n);                /* :86-105 */
float go_dot_dense(const float *a, const float *b, size_t n);                    /* :253-261 */
/* :201-210; also the dense types fp32 (0), bf16 (30) and Q8_0 (8, dotQ8 :107-120) */
float go_dot_row(uint32_t type_id, const uint8_t *row, const float *x, size_t cols);
void go_decode_row_fast(uint32_t type_id, const uint8_t *row, float *out, size_t cols); /* :213-235 */
void go_rms_norm(float *out, const float *x, const float *w, size_t n, float eps);  /* :281-291 */
/* src/engine.zig:670-687: top-k by value, ties to the lower index. */
void go_topk(const float *values, size_t n, uint32_t *ids, float *weights, size_t k);

/* Row bytes of those types (src/kernels.zig:56-67); 0 for other types or bad widths. */
size_t go_dense_row_bytes(uint32_t type_id, size_t cols);

/* One MoE layer as src/engine.zig:520-653 computes it. Expert matrices: per expert and
 * projection, a pointer to its packed rows and its type id (144..151), so a layer may mix
 * types. Gate/up rows have E columns (F rows per expert); down rows have F columns
 * (E rows per expert). */
typedef struct go_layer {
    uint32_t E, F, n_expert, n_used;
    float expert_weights_scale;
    const float *router;          /* [n_expert][E] fp32 */
    const float *router_bias;     /* [n_expert] added to the logits, or NULL */
    const uint8_t *const *gate;   /* [n_expert] -> F rows */
    const uint8_t *const *up;     /* [n_expert] -> F rows */
    const uint8_t *const *down;   /* [n_expert] -> E rows */
    const uint32_t *gate_type, *up_type, *down_type; /* [n_expert] */
    const float *gate_signs;      /* [E] or NULL */
    const float *down_signs;      /* [F] or NULL */
    /* Shared expert (optional): SF = 0 disables it. Rows in the GGML type sh_type: 0 fp32,
     * 30 bf16, 8 Q8_0 (src/kernels.zig:7-10, rowBytes :56-67). */
    uint32_t SF;
    const void *sh_gate, *sh_up; /* [SF] rows of E columns */
    const void *sh_down;         /* [E] rows of SF columns */
    const float *sh_gate_inp;    /* [E] fp32 */
    float sh_gate_const;         /* used when sh_gate_inp is NULL: gate = this value */
    uint32_t sh_type;
} go_layer;

/* Optional intermediate outputs of go_moe_ffn (any pointer may be NULL). */
typedef struct go_trace {
    float *logits;          /* [n][n_expert] router logits before softmax */
    uint32_t *route_ids;    /* [n][n_used] */
    float *route_w;         /* [n][n_used] */
    uint32_t *route_order;  /* [n*n_used] */
    uint32_t *order_start;  /* [n_expert+1] */
    float *xh;              /* [n][E] rotated expert input */
    float *act;             /* [n*n_used][F] down input (after SwiGLU and rotation) */
    float *down;            /* [n*n_used][E] */
    float *moe_out;         /* [n][E] routed output before the shared expert */
} go_trace;

/* Runs the layer on n tokens: out[n][E]. threads = pool size including the caller.
 * Returns 0, or a negative code for invalid arguments. */
int go_moe_ffn(const go_layer *layer, const float *x, size_t n, float *out, go_trace *trace,
               uint32_t threads);

/* fp64 dense reference of the routed and shared experts for given routes: decodes every
 * selected expert row bit-exactly to fp32 and accumulates in fp64. out[n][E] in fp64. */
int go_moe_dense_f64(const go_layer *layer, const float *x, size_t n, const uint32_t *route_ids,
                     const float *route_w, double *out);

/* Router logits in fp64 for margin checks: logits[n][n_expert]. */
void go_router_f64(const go_layer *layer, const float *x, size_t n, double *logits);

#ifdef __cplusplus
}
#endif
#endif
