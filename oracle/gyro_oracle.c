/*
 * CPU oracle for the routed-expert MoE path: TEST INFRASTRUCTURE ONLY (see gyro_oracle.h).
 *
 * Restates the reference CPU engine: the strict Gyro decoder and rotation (src/gyro.zig), the
 * CPU kernels (src/kernels.zig), the layer (src/engine.zig ffn and topK) and the work
 * decomposition of the thread pool (src/pool.zig). Built with -ffp-contract=off so every
 * product and sum rounds as written.
 */
#define _GNU_SOURCE
#include "gyro_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- format core */

static float g_codebook[4096];  /* fp32 expansion, src/kernels.zig:14-23 */
static int g_codebook_ready = 0;

typedef struct { uint32_t id, k, steps, block_bytes; } type_row;
/* src/gyro.zig:32-41. */
static const type_row k_types[8] = {
    {144, 8, 32, 34}, {145, 6, 32, 26}, {146, 7, 32, 30}, {147, 5, 64, 42},
    {148, 6, 64, 50}, {149, 7, 64, 58}, {150, 5, 32, 22}, {151, 4, 32, 18},
};

static const type_row *find_type(uint32_t id) {
    for (int i = 0; i < 8; ++i)
        if (k_types[i].id == id) return &k_types[i];
    return NULL;
}

int go_type_info(uint32_t id, uint32_t *k, uint32_t *steps, uint32_t *block_bytes) {
    const type_row *t = find_type(id);
    if (!t) return 0;
    if (k) *k = t->k;
    if (steps) *steps = t->steps;
    if (block_bytes) *block_bytes = t->block_bytes;
    return 1;
}

/* src/gyro.zig:70-76. */
uint64_t go_row_bytes(uint32_t id, uint64_t weights) {
    const type_row *t = find_type(id);
    if (!t || weights % 128 != 0) return 0;
    return weights / 128 * t->block_bytes;
}

/* src/gyro.zig:127-141: exact binary16 to binary32, subnormals renormalised by a loop. */
float go_fp16_to_fp32(uint16_t half) {
    uint32_t sign = (uint32_t)(half & 0x8000u) << 16;
    uint32_t exponent = (half >> 10) & 31u;
    uint32_t mantissa = half & 1023u;
    uint32_t bits;
    if (exponent == 31) {
        bits = sign | 0x7f800000u | (mantissa << 13);
    } else if (exponent != 0) {
        bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    } else if (mantissa == 0) {
        bits = sign;
    } else {
        uint32_t out_exp = 113;
        while ((mantissa & 1024u) == 0) {
            mantissa <<= 1;
            out_exp -= 1;
        }
        bits = sign | (out_exp << 23) | ((mantissa & 1023u) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

int go_init(const uint8_t *codebook, size_t len) {
    if (!codebook || len != 8192) return GO_INVALID_SOURCE_LENGTH;
    for (int i = 0; i < 4096; ++i)
        g_codebook[i] = go_fp16_to_fp32((uint16_t)(codebook[2 * i] | (codebook[2 * i + 1] << 8)));
    g_codebook_ready = 1;
    return GO_OK;
}

/* src/gyro.zig:107-117 (TQ2_T byte pair; k-bit circular 16-bit window). */
uint32_t go_trellis_state(uint32_t id, const uint8_t *stream, uint32_t step) {
    const type_row *t = find_type(id);
    if (id == 144) return ((uint32_t)stream[(step + 31) % 32] << 8) | stream[step];
    uint32_t stream_len = t->steps * t->k / 8;
    uint32_t offset = (t->steps - 1 - step) * t->k;
    uint32_t byte = offset >> 3;
    uint32_t word = (uint32_t)stream[byte] | ((uint32_t)stream[(byte + 1) % stream_len] << 8) |
                    ((uint32_t)stream[(byte + 2) % stream_len] << 16);
    return (word >> (offset & 7)) & 0xffffu;
}

/* Strict decoder, src/gyro.zig:81-105: w = fp32(d) * fp32(cb), one rounding. */
int go_decode_row(uint32_t id, int32_t state_bits, const uint8_t *src, size_t src_len, float *dst,
                  size_t n) {
    if (state_bits < 0) return GO_MISSING_STATE_BITS;
    if (state_bits != 15) return GO_UNSUPPORTED_STATE_BITS;
    const type_row *t = find_type(id);
    if (!t) return GO_UNSUPPORTED_TYPE;
    if (n % 128 != 0) return GO_INVALID_ROW_LENGTH;
    if (src_len != n / 128 * t->block_bytes) return GO_INVALID_SOURCE_LENGTH;
    size_t out = 0;
    for (size_t off = 0; off < src_len; off += t->block_bytes) {
        const uint8_t *block = src + off;
        float scale = go_fp16_to_fp32((uint16_t)(block[0] | (block[1] << 8)));
        const uint8_t *stream = block + 2;
        uint32_t pairs = t->steps == 64 ? 1 : 2;
        for (uint32_t step = 0; step < t->steps; ++step) {
            uint32_t state = go_trellis_state(id, stream, step);
            uint32_t hash = (state & 0x7fffu) * 0x9e3779b1u;
            for (uint32_t p = 0; p < pairs; ++p) {
                uint32_t index = p == 0 ? hash >> 21 : (hash >> 10) & 2047u;
                dst[out] = scale * g_codebook[index * 2];
                dst[out + 1] = scale * g_codebook[index * 2 + 1];
                out += 2;
            }
        }
    }
    return GO_OK;
}

/* src/gyro.zig:143-150 (validateTransform). */
static int validate_transform(size_t n, size_t block, const int8_t *signs) {
    if (block == 0 || (block & (block - 1)) != 0) return GO_INVALID_BLOCK_SIZE;
    if (n % block != 0) return GO_INVALID_ROW_LENGTH;
    if (signs)
        for (size_t i = 0; i < n; ++i)
            if (signs[i] != 1 && signs[i] != -1) return GO_INVALID_SIGN;
    return GO_OK;
}

/* src/gyro.zig:152-172: butterfly widths 1, 2, 4, ...; then one multiply by 1/sqrt(b). */
static void hadamard(float *v, size_t n, size_t block) {
    const float norm = 1.0f / sqrtf((float)block);
    for (size_t start = 0; start < n; start += block) {
        float *b = v + start;
        for (size_t width = 1; width < block; width *= 2)
            for (size_t s = 0; s < block; s += 2 * width)
                for (size_t j = 0; j < width; ++j) {
                    float a = b[s + j], c = b[s + j + width];
                    b[s + j] = a + c;
                    b[s + j + width] = a - c;
                }
        for (size_t j = 0; j < block; ++j) b[j] *= norm;
    }
}

/* src/gyro.zig:177-184. */
int go_rotate(float *v, size_t n, size_t block, const int8_t *signs) {
    int rc = validate_transform(n, block, signs);
    if (rc) return rc;
    if (signs)
        for (size_t i = 0; i < n; ++i) v[i] *= (float)signs[i];
    hadamard(v, n, block);
    return GO_OK;
}

/* src/gyro.zig:188-195. */
int go_unrotate(float *v, size_t n, size_t block, const int8_t *signs) {
    int rc = validate_transform(n, block, signs);
    if (rc) return rc;
    hadamard(v, n, block);
    if (signs)
        for (size_t i = 0; i < n; ++i) v[i] *= (float)signs[i];
    return GO_OK;
}

/* ---------------------------------------------------------------- engine kernels */

/* src/kernels.zig:316-338: signs multiply, butterfly, normalise. */
void go_rotate_f32signs(float *x, size_t n, size_t block, const float *signs) {
    for (size_t i = 0; i < n; ++i) x[i] *= signs[i];
    hadamard(x, n, block);
}

/* src/kernels.zig:340-349. */
void go_softmax(float *x, size_t n) {
    float m = -INFINITY;
    for (size_t i = 0; i < n; ++i) m = fmaxf(m, x[i]);
    float sum = 0;
    for (size_t i = 0; i < n; ++i) {
        x[i] = expf(x[i] - m);
        sum += x[i];
    }
    for (size_t i = 0; i < n; ++i) x[i] /= sum;
}

float go_silu(float x) { return x / (1.0f + expf(-x)); }     /* src/kernels.zig:307-309 */
float go_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); } /* src/kernels.zig:303-305 */

/* src/kernels.zig:72-84: eight lane accumulators, then a reduction, then the tail. */
float go_dot_f32(const float *row, const float *x, size_t n) {
    float acc[8] = {0};
    size_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) acc[l] += row[i + l] * x[i + l];
    float sum = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    for (; i < n; ++i) sum += row[i] * x[i];
    return sum;
}

static float bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* src/kernels.zig:86-105 with bf = true. */
float go_dot_bf16(const uint16_t *row, const float *x, size_t n) {
    float acc[8] = {0};
    size_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) acc[l] += bf16_to_f32(row[i + l]) * x[i + l];
    float sum = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    for (; i < n; ++i) sum += bf16_to_f32(row[i]) * x[i];
    return sum;
}

/* src/kernels.zig:253-261. */
float go_dot_dense(const float *a, const float *b, size_t n) { return go_dot_f32(a, b, n); }

/* dotQ8, src/kernels.zig:107-120: per 32-block, d * (sum of q * x) (the block sum in 8 lanes). */
static float dot_q8(const uint8_t *row, const float *x, size_t n) {
    float total = 0;
    for (size_t b = 0; b < n / 32; ++b) {
        const uint8_t *block = row + b * 34;
        const float d = go_fp16_to_fp32((uint16_t)(block[0] | (block[1] << 8)));
        float acc[8] = {0};
        for (size_t i = 0; i < 32; i += 8)
            for (int l = 0; l < 8; ++l) acc[l] += (float)(int8_t)block[2 + i + l] * x[b * 32 + i + l];
        total += d * (((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7])));
    }
    return total;
}

size_t go_dense_row_bytes(uint32_t type_id, size_t cols) {
    switch (type_id) {
        case 0: return cols * 4;
        case 30: return cols * 2;
        case 8: return cols % 32 ? 0 : cols / 32 * 34;
        default: return 0;
    }
}


/* fp32 value i of a dense row (decodeRow, src/kernels.zig:213-235, for the dense types). */
static float dense_value(uint32_t type_id, const void *row, size_t i) {
    switch (type_id) {
        case 0: return ((const float *)row)[i];
        case 30: return bf16_to_f32(((const uint16_t *)row)[i]);
        case 8: {
            const uint8_t *block = (const uint8_t *)row + (i / 32) * 34;
            return go_fp16_to_fp32((uint16_t)(block[0] | (block[1] << 8))) * (float)(int8_t)block[2 + i % 32];
        }
        default: return 0;
    }
}

/* src/kernels.zig:136-159: one block of 128 values in the stored basis. */
static void decode_block(const type_row *t, const uint8_t *block, float out[128]) {
    float scale = go_fp16_to_fp32((uint16_t)(block[0] | (block[1] << 8)));
    const uint8_t *stream = block + 2;
    if (t->steps == 32) {
        for (uint32_t step = 0; step < 32; ++step) {
            uint32_t state = go_trellis_state(t->id, stream, step);
            uint32_t h = (state & 0x7fffu) * 0x9e3779b1u;
            uint32_t a = (h >> 21) * 2, b = ((h >> 10) & 2047u) * 2;
            out[step * 4 + 0] = scale * g_codebook[a];
            out[step * 4 + 1] = scale * g_codebook[a + 1];
            out[step * 4 + 2] = scale * g_codebook[b];
            out[step * 4 + 3] = scale * g_codebook[b + 1];
        }
    } else {
        for (uint32_t step = 0; step < 64; ++step) {
            uint32_t state = go_trellis_state(t->id, stream, step);
            uint32_t h = (state & 0x7fffu) * 0x9e3779b1u;
            uint32_t a = (h >> 21) * 2;
            out[step * 2 + 0] = scale * g_codebook[a];
            out[step * 2 + 1] = scale * g_codebook[a + 1];
        }
    }
}

/* src/kernels.zig:161-183: fused TQ2_T dot, codebook products summed per block in a 4-wide
 * accumulator, then the block scale applied once. */
static float dot_tq2(const uint8_t *row, const float *x, size_t cols) {
    float total = 0;
    for (size_t bi = 0; bi < cols / 128; ++bi) {
        const uint8_t *block = row + bi * 34;
        float scale = go_fp16_to_fp32((uint16_t)(block[0] | (block[1] << 8)));
        const uint8_t *stream = block + 2;
        const float *xb = x + bi * 128;
        float acc[4] = {0, 0, 0, 0};
        for (uint32_t step = 0; step < 32; ++step) {
            uint32_t state = ((uint32_t)stream[(step + 31) & 31] << 8) | stream[step];
            uint32_t h = (state & 0x7fffu) * 0x9e3779b1u;
            uint32_t a = (h >> 21) * 2, b = ((h >> 10) & 2047u) * 2;
            acc[0] += g_codebook[a] * xb[step * 4 + 0];
            acc[1] += g_codebook[a + 1] * xb[step * 4 + 1];
            acc[2] += g_codebook[b] * xb[step * 4 + 2];
            acc[3] += g_codebook[b + 1] * xb[step * 4 + 3];
        }
        total += scale * ((acc[0] + acc[1]) + (acc[2] + acc[3]));
    }
    return total;
}

/* src/kernels.zig:185-199: decode the block, then a dense dot of 128. */
static float dot_gyro_generic(const type_row *t, const uint8_t *row, const float *x, size_t cols) {
    float total = 0;
    float tmp[128];
    for (size_t bi = 0; bi < cols / 128; ++bi) {
        decode_block(t, row + bi * t->block_bytes, tmp);
        total += go_dot_f32(tmp, x + bi * 128, 128);
    }
    return total;
}

/* src/kernels.zig:201-210: the dense types of the shared expert (fp32, bf16, Q8_0) and the Gyro
 * types; 0 for any other type. */
float go_dot_row(uint32_t type_id, const uint8_t *row, const float *x, size_t cols) {
    switch (type_id) {
        case 0: return go_dot_f32((const float *)(const void *)row, x, cols);
        case 30: return go_dot_bf16((const uint16_t *)(const void *)row, x, cols);
        case 8: return dot_q8(row, x, cols);
        case 144: return dot_tq2(row, x, cols);
        default: {
            const type_row *t = find_type(type_id);
            return t ? dot_gyro_generic(t, row, x, cols) : 0.0f;
        }
    }
}

/* src/kernels.zig:213-235 (Gyro types). */
void go_decode_row_fast(uint32_t type_id, const uint8_t *row, float *out, size_t cols) {
    const type_row *t = find_type(type_id);
    for (size_t b = 0; b < cols / 128; ++b) decode_block(t, row + b * t->block_bytes, out + b * 128);
}

/* src/kernels.zig:281-291. */
void go_rms_norm(float *out, const float *x, const float *w, size_t n, float eps) {
    float ss = 0;
    for (size_t i = 0; i < n; ++i) ss += x[i] * x[i];
    float scale = 1.0f / sqrtf(ss / (float)n + eps);
    for (size_t i = 0; i < n; ++i) out[i] = w ? x[i] * scale * w[i] : x[i] * scale;
}

/* src/engine.zig:670-687: insertion into a descending list; an entry moves up only past a
 * strictly smaller value, so earlier (lower) indices win ties. */
void go_topk(const float *values, size_t n, uint32_t *ids, float *weights, size_t k) {
    for (size_t j = 0; j < k; ++j) {
        ids[j] = UINT32_MAX;
        weights[j] = -INFINITY;
    }
    for (size_t i = 0; i < n; ++i) {
        float v = values[i];
        if (v <= weights[k - 1] && ids[k - 1] != UINT32_MAX) continue;
        size_t pos = k - 1;
        while (pos > 0 && (v > weights[pos - 1] || ids[pos - 1] == UINT32_MAX)) {
            weights[pos] = weights[pos - 1];
            ids[pos] = ids[pos - 1];
            pos -= 1;
        }
        weights[pos] = v;
        ids[pos] = (uint32_t)i;
    }
}

/* ---------------------------------------------------------------- thread pool */

/* src/pool.zig:84-120: the caller participates, chunks come from one atomic counter, and
 * run() returns when every chunk has finished. Workers live for one go_moe_ffn call. */
typedef void (*pool_fn)(void *ctx, size_t start, size_t end);

typedef struct pool {
    pthread_t *threads;
    uint32_t workers;
    pthread_mutex_t mu;
    pthread_cond_t cv_start, cv_done;
    uint64_t generation;
    uint32_t pending;
    int quit;
    pool_fn fn;
    void *ctx;
    size_t count, chunk;
    atomic_size_t next;
} pool;

static void pool_drain(pool *p) {
    for (;;) {
        size_t start = atomic_fetch_add_explicit(&p->next, p->chunk, memory_order_relaxed);
        if (start >= p->count) break;
        size_t end = start + p->chunk < p->count ? start + p->chunk : p->count;
        p->fn(p->ctx, start, end);
    }
}

static void *pool_worker(void *arg) {
    pool *p = (pool *)arg;
    uint64_t seen = 0;
    for (;;) {
        pthread_mutex_lock(&p->mu);
        while (p->generation == seen && !p->quit) pthread_cond_wait(&p->cv_start, &p->mu);
        if (p->quit) {
            pthread_mutex_unlock(&p->mu);
            return NULL;
        }
        seen = p->generation;
        pthread_mutex_unlock(&p->mu);
        pool_drain(p);
        pthread_mutex_lock(&p->mu);
        if (--p->pending == 0) pthread_cond_signal(&p->cv_done);
        pthread_mutex_unlock(&p->mu);
    }
}

static int pool_init(pool *p, uint32_t threads) {
    memset(p, 0, sizeof(*p));
    p->workers = threads > 1 ? threads - 1 : 0;
    pthread_mutex_init(&p->mu, NULL);
    pthread_cond_init(&p->cv_start, NULL);
    pthread_cond_init(&p->cv_done, NULL);
    if (!p->workers) return 0;
    p->threads = (pthread_t *)calloc(p->workers, sizeof(pthread_t));
    if (!p->threads) return -1;
    for (uint32_t i = 0; i < p->workers; ++i) pthread_create(&p->threads[i], NULL, pool_worker, p);
    return 0;
}

static void pool_deinit(pool *p) {
    pthread_mutex_lock(&p->mu);
    p->quit = 1;
    pthread_cond_broadcast(&p->cv_start);
    pthread_mutex_unlock(&p->mu);
    for (uint32_t i = 0; i < p->workers; ++i) pthread_join(p->threads[i], NULL);
    free(p->threads);
    pthread_mutex_destroy(&p->mu);
    pthread_cond_destroy(&p->cv_start);
    pthread_cond_destroy(&p->cv_done);
}

static void pool_run(pool *p, size_t count, size_t chunk, void *ctx, pool_fn fn) {
    if (count == 0) return;
    if (chunk < 1) chunk = 1;
    if (p->workers == 0 || count <= chunk) {
        fn(ctx, 0, count);
        return;
    }
    pthread_mutex_lock(&p->mu);
    p->fn = fn;
    p->ctx = ctx;
    p->count = count;
    p->chunk = chunk;
    atomic_store(&p->next, 0);
    p->pending = p->workers;
    p->generation += 1;
    pthread_cond_broadcast(&p->cv_start);
    pthread_mutex_unlock(&p->mu);
    pool_drain(p);
    pthread_mutex_lock(&p->mu);
    while (p->pending) pthread_cond_wait(&p->cv_done, &p->mu);
    pthread_mutex_unlock(&p->mu);
}

/* The pool persists across calls (src/runtime.zig:135 creates one pool per runtime); it is
 * rebuilt only when the requested thread count changes. */
static pool g_pool;
static uint32_t g_pool_threads = 0;
static pthread_mutex_t g_pool_mu = PTHREAD_MUTEX_INITIALIZER;

static pool *pool_get(uint32_t threads) {
    if (g_pool_threads != threads) {
        if (g_pool_threads) pool_deinit(&g_pool);
        if (pool_init(&g_pool, threads)) {
            g_pool_threads = 0;
            return NULL;
        }
        g_pool_threads = threads;
    }
    return &g_pool;
}

/* src/pool.zig:117-120. */
static size_t chunk_for(const pool *p, size_t count, size_t min_chunk) {
    size_t target = count / ((p->workers + 1) * 4);
    return target > min_chunk ? target : min_chunk;
}

/* ---------------------------------------------------------------- the layer */

#define MAX_COLS 16384 /* src/kernels.zig:12 */

typedef struct ffn_ctx {
    const go_layer *l;
    size_t n;
    const float *x;      /* [n][E] */
    const float *xh;     /* [n][E] */
    float *logits;       /* [n][n_expert] */
    float *act, *act_up; /* [n*U][F] */
    float *down;         /* [n*U][E] */
    const uint32_t *route_order;
    const uint32_t *starts;
    const float *y_in;   /* matmul input for the shared expert */
    float *y_out;
    const uint8_t *mat;
    uint32_t mat_type;
    size_t mat_rows, mat_cols;
} ffn_ctx;

/* kernels.matmul (src/kernels.zig:237-268) for the fp32 router: y[t][r] = W[r] . x[t]. */
static void router_range(void *c_, size_t start, size_t end) {
    ffn_ctx *c = (ffn_ctx *)c_;
    const go_layer *l = c->l;
    for (size_t r = start; r < end; ++r)
        for (size_t t = 0; t < c->n; ++t) {
            float v = go_dot_f32(l->router + r * l->E, c->x + t * l->E, l->E);
            if (l->router_bias) v += l->router_bias[r];
            c->logits[t * l->n_expert + r] = v;
        }
}

/* kernels.matmul for a dense matrix of the shared expert, one row at a time for every token
 * (src/kernels.zig:244-250 matvecRange, dotRow per row). */
static void dense_range(void *c_, size_t start, size_t end) {
    ffn_ctx *c = (ffn_ctx *)c_;
    const size_t rb = go_dense_row_bytes(c->mat_type, c->mat_cols);
    for (size_t r = start; r < end; ++r)
        for (size_t t = 0; t < c->n; ++t)
            c->y_out[t * c->mat_rows + r] =
                go_dot_row(c->mat_type, c->mat + r * rb, c->y_in + t * c->mat_cols, c->mat_cols);
}

/* Phase 1, src/engine.zig:568-602: one task per (expert, row) of gate and up. */
static void phase1(void *c_, size_t start, size_t end) {
    ffn_ctx *c = (ffn_ctx *)c_;
    const go_layer *l = c->l;
    const size_t F = l->F, E = l->E, U = l->n_used;
    float wbuf[MAX_COLS];
    for (size_t task = start; task < end; ++task) {
        size_t e = task / F, row = task % F;
        uint32_t first = c->starts[e], last = c->starts[e + 1];
        if (first == last) continue;
        uint32_t gt = l->gate_type[e], ut = l->up_type[e];
        const uint8_t *g = l->gate[e] + row * go_row_bytes(gt, E);
        const uint8_t *u = l->up[e] + row * go_row_bytes(ut, E);
        if (last - first == 1) {
            uint32_t slot = c->route_order[first];
            const float *x = c->xh + (slot / U) * E;
            c->act[slot * F + row] = go_dot_row(gt, g, x, E);
            c->act_up[slot * F + row] = go_dot_row(ut, u, x, E);
            continue;
        }
        go_decode_row_fast(gt, g, wbuf, E);
        for (uint32_t i = first; i < last; ++i) {
            uint32_t slot = c->route_order[i];
            c->act[slot * F + row] = go_dot_dense(wbuf, c->xh + (slot / U) * E, E);
        }
        go_decode_row_fast(ut, u, wbuf, E);
        for (uint32_t i = first; i < last; ++i) {
            uint32_t slot = c->route_order[i];
            c->act_up[slot * F + row] = go_dot_dense(wbuf, c->xh + (slot / U) * E, E);
        }
    }
}

/* Phase 2, src/engine.zig:609-633: one task per (expert, output row) of down. */
static void phase2(void *c_, size_t start, size_t end) {
    ffn_ctx *c = (ffn_ctx *)c_;
    const go_layer *l = c->l;
    const size_t F = l->F, E = l->E;
    float wbuf[MAX_COLS];
    for (size_t task = start; task < end; ++task) {
        size_t e = task / E, row = task % E;
        uint32_t first = c->starts[e], last = c->starts[e + 1];
        if (first == last) continue;
        uint32_t dt = l->down_type[e];
        const uint8_t *d = l->down[e] + row * go_row_bytes(dt, F);
        if (last - first == 1) {
            uint32_t slot = c->route_order[first];
            c->down[slot * E + row] = go_dot_row(dt, d, c->act + slot * F, F);
            continue;
        }
        go_decode_row_fast(dt, d, wbuf, F);
        for (uint32_t i = first; i < last; ++i) {
            uint32_t slot = c->route_order[i];
            c->down[slot * E + row] = go_dot_dense(wbuf, c->act + slot * F, F);
        }
    }
}

static int check_layer(const go_layer *l) {
    if (!l || !l->router || !l->gate || !l->up || !l->down || !l->gate_type || !l->up_type ||
        !l->down_type)
        return GO_INVALID_SOURCE_LENGTH;
    if (l->E % 128 || l->F % 128 || l->E > MAX_COLS || l->F > MAX_COLS || l->n_expert == 0 || l->n_expert > 512 || l->n_used == 0 ||
        l->n_used > l->n_expert)
        return GO_INVALID_ROW_LENGTH;
    for (uint32_t e = 0; e < l->n_expert; ++e)
        if (!find_type(l->gate_type[e]) || !find_type(l->up_type[e]) || !find_type(l->down_type[e]))
            return GO_UNSUPPORTED_TYPE;
    if (l->SF && (!l->sh_gate || !l->sh_up || !l->sh_down || !go_dense_row_bytes(l->sh_type, l->E) ||
                  !go_dense_row_bytes(l->sh_type, l->SF)))
        return GO_UNSUPPORTED_TYPE;
    if (!g_codebook_ready) return GO_INVALID_SOURCE_LENGTH;
    return GO_OK;
}

/* src/engine.zig:520-653. */
int go_moe_ffn(const go_layer *l, const float *x, size_t n, float *out, go_trace *trace,
               uint32_t threads) {
    int rc = check_layer(l);
    if (rc) return rc;
    if (n == 0) return GO_OK;
    const size_t E = l->E, F = l->F, U = l->n_used, NE = l->n_expert;
    pthread_mutex_lock(&g_pool_mu);
    pool *pp = pool_get(threads ? threads : 1);
    if (!pp) {
        pthread_mutex_unlock(&g_pool_mu);
        return GO_INVALID_SOURCE_LENGTH;
    }
    pool *const pool_ptr = pp;
    float *logits = (float *)malloc(n * NE * sizeof(float));
    uint32_t *ids = (uint32_t *)malloc(n * U * sizeof(uint32_t));
    float *wts = (float *)malloc(n * U * sizeof(float));
    float *xh = (float *)malloc(n * E * sizeof(float));
    uint32_t *order = (uint32_t *)malloc(n * U * sizeof(uint32_t));
    float *act = (float *)malloc(n * U * F * sizeof(float));
    float *act_up = (float *)malloc(n * U * F * sizeof(float));
    float *down = (float *)malloc(n * U * E * sizeof(float));
    ffn_ctx c = {.l = l, .n = n, .x = x, .xh = xh, .logits = logits, .act = act, .act_up = act_up,
                 .down = down, .route_order = order};

    /* Router (src/engine.zig:526): matmul with chunkFor(rows, 8). */
    pool_run(pool_ptr, NE, chunk_for(pool_ptr, NE, 8), &c, router_range);
    if (trace && trace->logits) memcpy(trace->logits, logits, n * NE * sizeof(float));
    /* Softmax, top-k, renormalisation (src/engine.zig:527-540). */
    for (size_t t = 0; t < n; ++t) {
        float *probs = logits + t * NE;
        go_softmax(probs, NE);
        go_topk(probs, NE, ids + t * U, wts + t * U, U);
        float sum = 0;
        for (size_t k = 0; k < U; ++k) sum += wts[t * U + k];
        sum = fmaxf(sum, 6.103515625e-5f);
        for (size_t k = 0; k < U; ++k) {
            wts[t * U + k] /= sum;
            if (l->expert_weights_scale != 0 && l->expert_weights_scale != 1)
                wts[t * U + k] *= l->expert_weights_scale;
        }
    }
    /* Rotated expert input (src/engine.zig:547-551). */
    memcpy(xh, x, n * E * sizeof(float));
    if (l->gate_signs)
        for (size_t t = 0; t < n; ++t) go_rotate_f32signs(xh + t * E, E, 128, l->gate_signs);
    /* Counting sort by expert (src/engine.zig:553-564). */
    for (size_t i = 0; i < n * E; ++i) out[i] = 0;
    uint32_t count[512] = {0};
    uint32_t starts[513] = {0};
    for (size_t i = 0; i < n * U; ++i) count[ids[i]] += 1;
    for (size_t e = 0; e < NE; ++e) starts[e + 1] = starts[e] + count[e];
    uint32_t fill[513];
    memcpy(fill, starts, sizeof(fill));
    for (size_t i = 0; i < n * U; ++i) order[fill[ids[i]]++] = (uint32_t)i;
    c.starts = starts;
    /* Phase 1 (src/engine.zig:567-602). */
    pool_run(pool_ptr, NE * F, 16, &c, phase1);
    /* SwiGLU and the down-input rotation (src/engine.zig:603-607). */
    for (size_t slot = 0; slot < n * U; ++slot) {
        float *a = act + slot * F;
        const float *u = act_up + slot * F;
        for (size_t i = 0; i < F; ++i) a[i] = go_silu(a[i]) * u[i];
        if (l->down_signs) go_rotate_f32signs(a, F, 128, l->down_signs);
    }
    /* Phase 2 (src/engine.zig:608-633). */
    pool_run(pool_ptr, NE * E, 64, &c, phase2);
    /* Combine in k order (src/engine.zig:634-641). */
    for (size_t t = 0; t < n; ++t)
        for (size_t k = 0; k < U; ++k) {
            size_t slot = t * U + k;
            float w = wts[slot];
            for (size_t i = 0; i < E; ++i) out[t * E + i] += w * down[slot * E + i];
        }
    if (trace) {
        if (trace->route_ids) memcpy(trace->route_ids, ids, n * U * sizeof(uint32_t));
        if (trace->route_w) memcpy(trace->route_w, wts, n * U * sizeof(float));
        if (trace->route_order) memcpy(trace->route_order, order, n * U * sizeof(uint32_t));
        if (trace->order_start) memcpy(trace->order_start, starts, (NE + 1) * sizeof(uint32_t));
        if (trace->xh) memcpy(trace->xh, xh, n * E * sizeof(float));
        if (trace->act) memcpy(trace->act, act, n * U * F * sizeof(float));
        if (trace->down) memcpy(trace->down, down, n * U * E * sizeof(float));
        if (trace->moe_out) memcpy(trace->moe_out, out, n * E * sizeof(float));
    }
    /* Shared expert with its sigmoid gate (src/engine.zig:644-653). */
    if (l->SF) {
        const size_t SF = l->SF;
        float *sg = (float *)malloc(n * SF * sizeof(float));
        float *su = (float *)malloc(n * SF * sizeof(float));
        float *sd = (float *)malloc(n * E * sizeof(float));
        c.y_in = x;
        c.mat_cols = E;
        c.mat_rows = SF;
        c.mat_type = l->sh_type;
        c.mat = (const uint8_t *)l->sh_gate;
        c.y_out = sg;
        pool_run(pool_ptr, SF, chunk_for(pool_ptr, SF, 8), &c, dense_range);
        c.mat = (const uint8_t *)l->sh_up;
        c.y_out = su;
        pool_run(pool_ptr, SF, chunk_for(pool_ptr, SF, 8), &c, dense_range);
        for (size_t i = 0; i < n * SF; ++i) sg[i] = go_silu(sg[i]) * su[i];
        c.y_in = sg;
        c.mat_cols = SF;
        c.mat_rows = E;
        c.mat = (const uint8_t *)l->sh_down;
        c.y_out = sd;
        pool_run(pool_ptr, E, chunk_for(pool_ptr, E, 8), &c, dense_range);
        for (size_t t = 0; t < n; ++t) {
            float gate = l->sh_gate_inp ? go_sigmoid(go_dot_dense(l->sh_gate_inp, x + t * E, E))
                                        : l->sh_gate_const;
            for (size_t i = 0; i < E; ++i) out[t * E + i] += sd[t * E + i] * gate;
        }
        free(sg);
        free(su);
        free(sd);
    }
    free(logits);
    free(ids);
    free(wts);
    free(xh);
    free(order);
    free(act);
    free(act_up);
    free(down);
    pthread_mutex_unlock(&g_pool_mu);
    return GO_OK;
}

/* ---------------------------------------------------------------- fp64 references */

void go_router_f64(const go_layer *l, const float *x, size_t n, double *logits) {
    for (size_t t = 0; t < n; ++t)
        for (size_t r = 0; r < l->n_expert; ++r) {
            double s = 0;
            for (size_t i = 0; i < l->E; ++i)
                s += (double)l->router[r * l->E + i] * (double)x[t * l->E + i];
            if (l->router_bias) s += (double)l->router_bias[r];
            logits[t * l->n_expert + r] = s;
        }
}

static double silu64(double v) { return v / (1.0 + exp(-v)); }

/* Same algebra as src/engine.zig:520-653, each product and sum in fp64, weights decoded
 * bit-exactly by the strict decoder. Routes are given, so top-k ties cannot diverge. */
int go_moe_dense_f64(const go_layer *l, const float *x, size_t n, const uint32_t *route_ids,
                     const float *route_w, double *out) {
    int rc = check_layer(l);
    if (rc) return rc;
    const size_t E = l->E, F = l->F, U = l->n_used;
    float *row = (float *)malloc((E > F ? E : F) * sizeof(float));
    double *xh = (double *)malloc(E * sizeof(double));
    double *g = (double *)malloc(F * sizeof(double));
    double *u = (double *)malloc(F * sizeof(double));
    double *a = (double *)malloc(F * sizeof(double));
    for (size_t t = 0; t < n; ++t) {
        double *o = out + t * E;
        for (size_t i = 0; i < E; ++i) o[i] = 0;
        /* xh = H (s . x) in fp64. */
        for (size_t i = 0; i < E; ++i) xh[i] = (double)x[t * E + i] * (l->gate_signs ? l->gate_signs[i] : 1.0);
        if (l->gate_signs)
            for (size_t b0 = 0; b0 < E; b0 += 128) {
                for (size_t w = 1; w < 128; w *= 2)
                    for (size_t s = 0; s < 128; s += 2 * w)
                        for (size_t j = 0; j < w; ++j) {
                            double p = xh[b0 + s + j], q = xh[b0 + s + j + w];
                            xh[b0 + s + j] = p + q;
                            xh[b0 + s + j + w] = p - q;
                        }
                for (size_t j = 0; j < 128; ++j) xh[b0 + j] /= sqrt(128.0);
            }
        for (size_t k = 0; k < U; ++k) {
            uint32_t e = route_ids[t * U + k];
            double w = route_w[t * U + k];
            uint32_t gt = l->gate_type[e], ut = l->up_type[e], dt = l->down_type[e];
            for (size_t r = 0; r < F; ++r) {
                go_decode_row(gt, 15, l->gate[e] + r * go_row_bytes(gt, E), go_row_bytes(gt, E), row, E);
                double s = 0;
                for (size_t i = 0; i < E; ++i) s += (double)row[i] * xh[i];
                g[r] = s;
                go_decode_row(ut, 15, l->up[e] + r * go_row_bytes(ut, E), go_row_bytes(ut, E), row, E);
                s = 0;
                for (size_t i = 0; i < E; ++i) s += (double)row[i] * xh[i];
                u[r] = s;
            }
            for (size_t r = 0; r < F; ++r) a[r] = silu64(g[r]) * u[r] * (l->down_signs ? l->down_signs[r] : 1.0);
            if (l->down_signs)
                for (size_t b0 = 0; b0 < F; b0 += 128) {
                    for (size_t wd = 1; wd < 128; wd *= 2)
                        for (size_t s = 0; s < 128; s += 2 * wd)
                            for (size_t j = 0; j < wd; ++j) {
                                double p = a[b0 + s + j], q = a[b0 + s + j + wd];
                                a[b0 + s + j] = p + q;
                                a[b0 + s + j + wd] = p - q;
                            }
                    for (size_t j = 0; j < 128; ++j) a[b0 + j] /= sqrt(128.0);
                }
            for (size_t r = 0; r < E; ++r) {
                go_decode_row(dt, 15, l->down[e] + r * go_row_bytes(dt, F), go_row_bytes(dt, F), row, F);
                double s = 0;
                for (size_t i = 0; i < F; ++i) s += (double)row[i] * a[i];
                o[r] += w * s;
            }
        }
        if (l->SF) {
            const size_t SF = l->SF;
            double *sg = (double *)malloc(SF * sizeof(double));
            const size_t rbe = go_dense_row_bytes(l->sh_type, E), rbf = go_dense_row_bytes(l->sh_type, SF);
            for (size_t r = 0; r < SF; ++r) {
                double s1 = 0, s2 = 0;
                const uint8_t *gr = (const uint8_t *)l->sh_gate + r * rbe, *ur = (const uint8_t *)l->sh_up + r * rbe;
                for (size_t i = 0; i < E; ++i) {
                    s1 += (double)dense_value(l->sh_type, gr, i) * (double)x[t * E + i];
                    s2 += (double)dense_value(l->sh_type, ur, i) * (double)x[t * E + i];
                }
                sg[r] = silu64(s1) * s2;
            }
            double gate;
            if (l->sh_gate_inp) {
                double s = 0;
                for (size_t i = 0; i < E; ++i) s += (double)l->sh_gate_inp[i] * (double)x[t * E + i];
                gate = 1.0 / (1.0 + exp(-s));
            } else {
                gate = l->sh_gate_const;
            }
            for (size_t r = 0; r < E; ++r) {
                double s = 0;
                const uint8_t *dr = (const uint8_t *)l->sh_down + r * rbf;
                for (size_t i = 0; i < SF; ++i) s += (double)dense_value(l->sh_type, dr, i) * sg[i];
                o[r] += gate * s;
            }
            free(sg);
        }
    }
    free(row);
    free(xh);
    free(g);
    free(u);
    free(a);
    return GO_OK;
}
