/*
 * gyro_moe: the host-side MoE layer engine above the gyro_native C ABI.
 *
 * The reference's host side is Zig (src/gpu.zig Device, src/gpu_engine.zig Engine.ffn); no Zig
 * toolchain exists for this build, so the same dispatch logic is restated in C++ and exposed
 * here for tests and benchmarks. Every GPU operation goes through gd_* calls.
 *
 * Paths (gm_forward, gm_run):
 *   GM_PATH_REFERENCE  the reference dispatch sequence of src/gpu_engine.zig:1052-1119
 *                      (mv_f32 router, rotate128, moe_route, moe_resolve, moe_gyro gate/up,
 *                      moe_act, moe_gyro down, moe_combine), in passes of max_tok tokens.
 *   GM_PATH_DECODE     the MI355X decode path: moe_router, moe_decode_gu, moe_decode_down.
 *   GM_PATH_PREFILL    the MI355X grouped-GEMM path: moe_prefill_router, moe_prefill_topk,
 *                      moe_prefill_sort, moe_prefill_gu, moe_prefill_down, moe_prefill_combine.
 *   GM_PATH_GENERIC    any layer: Gyro types mixed per expert and projection (moe_gyro_x reads
 *                      each expert's projections and types from the layer's descriptor table)
 *                      and the optional bf16 shared expert (mv_bf16, ew, mv_f32 gate, combine),
 *                      in the reference's dispatch style; passes of max_tok tokens.
 * All return 0 or a negative code; gm_last_error describes the failure.
 */
#ifndef GYRO_MOE_H
#define GYRO_MOE_H

#include <stddef.h>
#include <stdint.h>

#define GM_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gm_engine gm_engine;

enum { GM_PATH_REFERENCE = 0, GM_PATH_DECODE = 1, GM_PATH_PREFILL = 2, GM_PATH_GENERIC = 3 };

/* One MoE layer in the reference's tensor layout (src/model.zig:115-123): per expert, gate and
 * up hold F rows of E columns and down holds E rows of F columns, each row a run of Gyro blocks.
 * types[e*3 + p] is the Gyro type id of expert e, projection p (0 gate, 1 up, 2 down). */
typedef struct gm_layer_desc {
    uint32_t E, F, n_expert, n_used;
    float expert_weights_scale;
    const float *router;      /* [n_expert][E] */
    const float *router_bias; /* [n_expert] or NULL */
    const float *gate_signs;  /* [E] or NULL */
    const float *down_signs;  /* [F] or NULL */
    const uint8_t *const *gate;
    const uint8_t *const *up;
    const uint8_t *const *down;
    const uint32_t *types;
    /* Optional shared SwiGLU expert (src/engine.zig:644-653), SF = 0 for none: gate and up [SF]
     * rows of E columns, down [E] rows of SF columns, in the row format sh_type names (bf16; GGUF
     * Q8_0 blocks; fp32), and the fp32 gate input [E]: out += sigmoid(g . x) * W_d (silu(W_g x)
     * * W_u x) on the unrotated input x. E and SF must be multiples of 64. */
    uint32_t SF;
    const void *sh_gate;
    const void *sh_up;
    const void *sh_down;
    const float *sh_gate_inp;
    /* RMSNorm applied to this layer's input inside a stack (gm_forward_stack, gm_run_stack): fp32
     * weight [E] or NULL (no weight), and eps (src/kernels.zig:281-291). */
    const float *norm_weight;
    float norm_eps;
    /* Row format of the shared expert's matrices: GM_SHARED_BF16 (default), GM_SHARED_Q8_0
     * (34-byte blocks of a binary16 scale and 32 int8 quants, repacked at upload as
     * src/gpu_engine.zig:289-306 does) or GM_SHARED_F32. */
    uint32_t sh_type;
} gm_layer_desc;

enum { GM_SHARED_BF16 = 0, GM_SHARED_Q8_0 = 1, GM_SHARED_F32 = 2 };

/* Creates an engine on device `adapter`, loading every <name>.co pipeline in kernel_dir.
 * max_tok bounds the tokens of one gm_forward/gm_run call (the reference uses passes of 64). */
GM_API int gm_create(const char *kernel_dir, uint32_t adapter, uint32_t max_tok, gm_engine **out);
GM_API void gm_destroy(gm_engine *e);
GM_API const char *gm_last_error(gm_engine *e);
/* Uploads a layer and returns its index. Layers of one engine share E, F, n_expert, n_used.
 * Every expert occupies one slot of a fixed stride set by the first layer: its own bundle when
 * its experts share one Gyro type, the widest type's bundle when they mix types; a later layer
 * whose bundle exceeds the stride is refused. */
GM_API int gm_add_layer(gm_engine *e, const gm_layer_desc *desc, uint32_t *out_index);
/* Runs n tokens (n <= max_tok) of x[n][E] through one layer on a path; writes out[n][E]. */
GM_API int gm_forward(gm_engine *e, uint32_t layer, uint32_t path, const float *x, uint32_t n, float *out);
/* Reads the routing of the last gm_forward: ids[n][n_used], weights[n][n_used]. */
GM_API int gm_last_routes(gm_engine *e, uint32_t n, uint32_t *ids, float *weights);
/* Reads the counting sort of the last GM_PATH_PREFILL gm_forward of n tokens (src/engine.zig:
 * 553-564): order[n * n_used] lists the slots t * n_used + k grouped by expert, stable in slot
 * order; order_start[n_expert + 1] is the exclusive prefix of the expert counts. */
GM_API int gm_last_sort(gm_engine *e, uint32_t n, uint32_t *order, uint32_t *order_start);
/* Reads the tile list of the last prefill-path call: count (out) tiles of 4 words each
 * {expert, first sorted row, rows, 0}, at most max_tiles of them. */
GM_API int gm_last_tiles(gm_engine *e, uint32_t max_tiles, uint32_t *tiles, uint32_t *count);
/* Decodes rows [row0, row0 + rows) of one expert projection (any Gyro type) to fp32 with the
 * decode path's block decoders (bit-exact check of the in-kernel dequantisation). */
GM_API int gm_dequant(gm_engine *e, uint32_t layer, uint32_t expert, uint32_t proj, uint32_t row0,
                      uint32_t rows, float *out);
/* As gm_dequant with the decoder of one path: GM_DEQUANT_DECODE (the decode kernels'),
 * GM_DEQUANT_PREFILL (the prefill GEMMs' B-operand decoders, both lane halves; fp32 scale x
 * codebook value) or GM_DEQUANT_PREFILL_B16 (the B operand as the MFMA reads it: the binary16
 * product of scale and codebook value, widened to fp32). */
enum { GM_DEQUANT_DECODE = 0, GM_DEQUANT_PREFILL = 1, GM_DEQUANT_PREFILL_B16 = 2 };
GM_API int gm_dequant_as(gm_engine *e, uint32_t layer, uint32_t expert, uint32_t proj, uint32_t row0,
                         uint32_t rows, uint32_t decoder, float *out);

/* Benchmark harness: tokens[n_total][E] are uploaded once; gm_run then processes `calls` calls
 * of `batch` tokens starting at token `first`, call i using layer layers[i % n_layers], with
 * every input already in device memory. Returns the device time between the first and last
 * dispatch (ms), measured with events on the compute stream, and the host wall time of the loop
 * including the final wait (ms). */
GM_API int gm_set_tokens(gm_engine *e, const float *tokens, uint32_t n_total);
GM_API int gm_run(gm_engine *e, uint32_t path, uint32_t batch, uint32_t calls, uint32_t first,
                  const uint32_t *layers, uint32_t n_layers, double *device_ms, double *wall_ms);
/* As gm_run, and also times every launch of one kernel of the path by its own start and end
 * (gd_dispatch_timed; bracket: 1 router, 2 gate/up, 3 down, 0 none); *bracket_us receives the
 * mean duration of one launch in microseconds. */
GM_API int gm_run_bracketed(gm_engine *e, uint32_t path, uint32_t batch, uint32_t calls, uint32_t first,
                            const uint32_t *layers, uint32_t n_layers, uint32_t bracket,
                            double *device_ms, double *wall_ms, double *bracket_us);
/* A stack of layers: x <- x + MoE_l(RMSNorm_l(x)) for l = layers[0..n_layers), on n <= max_tok
 * tokens of x[n][E]; writes the final x to out[n][E]. */
GM_API int gm_forward_stack(gm_engine *e, const uint32_t *layers, uint32_t n_layers, uint32_t path, const float *x,
                            uint32_t n, float *out);
/* As gm_run for a stack: each of `calls` calls takes `batch` device-resident tokens (from token
 * `first`, as gm_run) through every layer of the stack, writing the results to the outputs. */
GM_API int gm_run_stack(gm_engine *e, uint32_t path, uint32_t batch, uint32_t calls, uint32_t first,
                        const uint32_t *layers, uint32_t n_layers, double *device_ms, double *wall_ms);
/* Reads outputs[n_total][E] written by gm_run or gm_run_stack. */
GM_API int gm_read_outputs(gm_engine *e, float *out, uint32_t n_total);

/* Size of the device array that gm_forward_decode_noalloc keeps its intermediate buffers in
 * (one per GPU, held until the process ends). */
#define GM_NOALLOC_SCRATCH_BYTES (5u << 20)

/* No counterpart in the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc). The GM_PATH_DECODE forward
 * of gm_forward on n <= 8 tokens, with x[n][E] and out[n][E] in device memory, queued on
 * `stream` (a hipStream_t of the engine's device; NULL: the engine's compute stream) without
 * waiting for it. It calls no hipMalloc / hipFree and no memset or copy: router logits, routes,
 * the rotated input, the gate/up partials and the shared expert's rows live in a fixed device
 * array of GM_NOALLOC_SCRATCH_BYTES per GPU, and a small kernel points two table entries at x and
 * out. A layer shape whose buffers exceed that array is refused with an error. Every call on one
 * GPU shares the array and those two entries: calls that overlap on one GPU race, so a caller
 * serialises them (one stream, or its own ordering). Results equal gm_forward's bit for bit: the
 * decode path keeps its activations in fp32, so no call of it is ever recomputed on another path
 * (the binary16 range recompute of gm_forward concerns GM_PATH_PREFILL only). */
GM_API int gm_forward_decode_noalloc(gm_engine *e, uint32_t layer, const float *x, uint32_t n, float *out,
                                     void *stream);

#ifdef __cplusplus
}
#endif
#endif
