/*
 * fox_host.h -- the RustFox host API, kept, over the gfx950 device path.
 *
 * libfox.so exports the RustFox entry points a decode loop uses, with the
 * same names, argument meaning, status codes and ownership rules as
 * include/fox/fox.h of RustFox, so a caller of the reference switches by
 * opening the model with FOX_WEIGHTS_DEVICE.  Compute runs on the GPU through
 * include/fox_gpu.h; there are no CPU kernels in this library.
 *
 * Declarations below cite the RustFox interface each one keeps
 * (include/fox/fox.h:line).  Entries marked EXTENSION have no RustFox
 * counterpart.
 */
#ifndef FOX_HOST_H
#define FOX_HOST_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* include/fox/fox.h:17-30 */
typedef enum {
    FOX_OK = 0,
    FOX_ERR_ARG,
    FOX_ERR_IO,
    FOX_ERR_NOMEM,
    FOX_ERR_FORMAT,
    FOX_ERR_UNSUPPORTED,
    FOX_ERR_NOTFOUND,
    FOX_ERR_INTERNAL
} fox_status;

const char *fox_version(void);
const char *fox_status_str(fox_status s);
const char *fox_last_error(void);

#define FOX_NAME_MAX 128

/* include/fox/fox.h:213-224: the ggml type ids as GGUF files store them
 * (the device path computes F32, F16, Q4_K, Q6_K, TQ1_0 and TQ2_0 weights) */
typedef enum {
    FOX_GGML_F32 = 0, FOX_GGML_F16 = 1, FOX_GGML_Q4_0 = 2,
    FOX_GGML_Q4_1 = 3, FOX_GGML_Q5_0 = 6, FOX_GGML_Q5_1 = 7,
    FOX_GGML_Q8_0 = 8, FOX_GGML_Q2_K = 10, FOX_GGML_Q3_K = 11,
    FOX_GGML_Q4_K = 12, FOX_GGML_Q5_K = 13, FOX_GGML_Q6_K = 14,
    FOX_GGML_Q8_K = 15, FOX_GGML_IQ2_XXS = 16, FOX_GGML_IQ2_XS = 17,
    FOX_GGML_IQ3_XXS = 18, FOX_GGML_IQ1_S = 19, FOX_GGML_IQ4_NL = 20,
    FOX_GGML_IQ3_S = 21, FOX_GGML_IQ2_S = 22, FOX_GGML_IQ4_XS = 23,
    FOX_GGML_I8 = 24, FOX_GGML_I16 = 25, FOX_GGML_I32 = 26,
    FOX_GGML_I64 = 27, FOX_GGML_F64 = 28, FOX_GGML_IQ1_M = 29,
    FOX_GGML_BF16 = 30, FOX_GGML_TQ1_0 = 34, FOX_GGML_TQ2_0 = 35
} fox_ggml_type;

/* include/fox/fox.h:357-358: IEEE half <-> single.  f16 -> f32 is exact
 * (subnormals, infinities, NaN payloads kept); f32 -> f16 rounds to nearest
 * even into the normal range, half up into the subnormal range, flushes
 * below half the smallest subnormal to a signed zero, saturates to
 * infinity, and turns every NaN into the quiet NaN 0x7E00 with its sign. */
float    fox_f16_to_f32(uint16_t h);
uint16_t fox_f32_to_f16(float f);

/* --------------------------------------------------------------- gguf */

/* include/fox/fox.h:204-262: the GGUF reader the model loader uses.  Same
 * acceptance rules as RustFox src/gguf.c:348-466; metadata arrays are read
 * into memory.  Lookups by name return SIZE_MAX when absent; a getter on an
 * index past the table returns FOX_ERR_NOTFOUND, on a value of another type
 * FOX_ERR_FORMAT, with a NULL handle or output FOX_ERR_ARG. */
#define FOX_GGUF_MAX_DIMS 4

typedef enum {
    FOX_GGUF_UINT8 = 0, FOX_GGUF_INT8, FOX_GGUF_UINT16, FOX_GGUF_INT16,
    FOX_GGUF_UINT32, FOX_GGUF_INT32, FOX_GGUF_FLOAT32, FOX_GGUF_BOOL,
    FOX_GGUF_STRING, FOX_GGUF_ARRAY, FOX_GGUF_UINT64, FOX_GGUF_INT64,
    FOX_GGUF_FLOAT64
} fox_gguf_value_type;

typedef struct {
    const char   *name;
    uint32_t      n_dims;
    uint64_t      ne[FOX_GGUF_MAX_DIMS];
    fox_ggml_type type;
    uint64_t      offset;       /* from the start of the data section */
    uint64_t      size_bytes;
} fox_gguf_tensor;

typedef struct fox_gguf fox_gguf;

fox_status fox_gguf_open(const char *path, fox_gguf **out);
void       fox_gguf_close(fox_gguf *g);
uint32_t   fox_gguf_version(const fox_gguf *g);
size_t     fox_gguf_metadata_count(const fox_gguf *g);
size_t     fox_gguf_tensor_count(const fox_gguf *g);
size_t     fox_gguf_find(const fox_gguf *g, const char *key);
/* FOX_GGUF_ARRAY for an index past the table */
fox_gguf_value_type fox_gguf_metadata_type(const fox_gguf *g, size_t index);
/* 0 and FOX_GGUF_ARRAY when the value is not an array */
size_t     fox_gguf_metadata_array_count(const fox_gguf *g, size_t index);
fox_gguf_value_type fox_gguf_metadata_array_type(const fox_gguf *g, size_t index);
fox_status fox_gguf_get_u32(const fox_gguf *g, size_t index, uint32_t *out);
fox_status fox_gguf_get_bool(const fox_gguf *g, size_t index, int *out);
fox_status fox_gguf_get_f32(const fox_gguf *g, size_t index, float *out);
/* any integer or bool value, signed ones sign-extended */
fox_status fox_gguf_get_uint(const fox_gguf *g, size_t index, uint64_t *out);
fox_status fox_gguf_get_string(const fox_gguf *g, size_t index, const char **out);
fox_status fox_gguf_get_array_string(const fox_gguf *g, size_t index,
                                     size_t element, const char **out);
fox_status fox_gguf_get_array_i32(const fox_gguf *g, size_t index,
                                  size_t element, int32_t *out);
fox_status fox_gguf_get_array_f32(const fox_gguf *g, size_t index,
                                  size_t element, float *out);
fox_status fox_gguf_tensor_at(const fox_gguf *g, size_t index, fox_gguf_tensor *out);
size_t     fox_gguf_tensor_find(const fox_gguf *g, const char *name);
/* the tensor's bytes as stored in the file; FOX_ERR_ARG if capacity is
 * smaller than size_bytes */
fox_status fox_gguf_read_tensor(const fox_gguf *g, size_t index,
                                void *dst, size_t capacity);

const char *fox_ggml_type_name(fox_ggml_type type);
uint32_t    fox_ggml_type_block_size(fox_ggml_type type);
uint32_t    fox_ggml_type_block_bytes(fox_ggml_type type);
/* include/fox/fox.h:360-361: a type the device path has kernels for */
int         fox_gemv_supports(fox_ggml_type type);
size_t      fox_row_bytes(fox_ggml_type type, size_t n_cols);

/* ----------------------------------------------------------- operators */

/* The reference's operator entry points on host buffers, computed on the
 * GPU (rustfox_amd/host/operators.c): same arguments, results and status
 * codes; each call copies its operands to HBM and the result back, so the
 * decode path keeps weights resident instead.  The pool is accepted for
 * the ABI and not used; NULL is accepted. */
typedef struct fox_threadpool fox_threadpool;

/* include/fox/fox.h:331-333 (n <= 0: online cores, at most 256) */
fox_threadpool *fox_threadpool_create(int n_threads);
void            fox_threadpool_destroy(fox_threadpool *tp);
int             fox_threadpool_size(const fox_threadpool *tp);
/* include/fox/fox.h:335-338: fn(ctx, 0, 0, n) on the calling thread (no CPU
 * workers in this library; the reference's NULL-pool behaviour) */
typedef void (*fox_parallel_fn)(void *ctx, int worker, size_t begin, size_t end);
fox_status      fox_parallel_for(fox_threadpool *tp, size_t n, fox_parallel_fn fn, void *ctx);

/* include/fox/fox.h:322-329: *out = sum_b d_b * S_b over n/256 blocks */
fox_status fox_tq1_dot_i8(const int8_t *activations, const void *block_data,
                          size_t n, float *out);
fox_status fox_tq2_dot_i8(const int8_t *activations, const void *block_data,
                          size_t n, float *out);
fox_status fox_tq1_dot_i8_scalar(const int8_t *activations, const void *block_data,
                                 size_t n, float *out);
fox_status fox_tq2_dot_i8_scalar(const int8_t *activations, const void *block_data,
                                 size_t n, float *out);

/* include/fox/fox.h:342-343: per-vector int8 activations, scale amax/127 */
fox_status fox_quantize_activations_i8(const float *x, size_t n,
                                       int8_t *q, float *scale);

/* include/fox/fox.h:345-355 */
fox_status fox_gemv_tq1_f32(fox_threadpool *tp, const float *x, const void *weights,
                            size_t n_rows, size_t n_cols, float *out);
fox_status fox_gemv_tq2_f32(fox_threadpool *tp, const float *x, const void *weights,
                            size_t n_rows, size_t n_cols, float *out);
fox_status fox_gemv_tq1_i8(fox_threadpool *tp, const int8_t *q, float act_scale,
                           const void *weights, size_t n_rows, size_t n_cols,
                           float *out);
fox_status fox_gemv_tq2_i8(fox_threadpool *tp, const int8_t *q, float act_scale,
                           const void *weights, size_t n_rows, size_t n_cols,
                           float *out);

/* include/fox/fox.h:363-365: types of fox_gemv_supports; others
 * FOX_ERR_UNSUPPORTED */
fox_status fox_gemv(fox_threadpool *tp, fox_ggml_type type, const float *x,
                    const void *weights, size_t n_rows, size_t n_cols,
                    float *out);

/* include/fox/fox.h:367-368: F32, F16, Q8_0, Q4_0, Q4_K, Q5_K and Q6_K
 * rows (src/kernels.c:874-941) */
fox_status fox_dequant_row(fox_ggml_type type, const void *row, size_t n,
                           float *out);

/* ------------------------------------------------------------- weights */

/* include/fox/fox.h:370-403, plus the HBM-resident mode */
#define FOX_WEIGHTS_MAX_LIVE_LEASES 8

typedef enum {
    FOX_WEIGHTS_RESIDENT = 0,   /* host memory, loaded on first touch        */
    FOX_WEIGHTS_STREAM   = 1,   /* not provided by rustfox_amd               */
    FOX_WEIGHTS_DEVICE   = 2    /* HBM of the GPU, loaded once per tensor    */
} fox_weights_mode;

typedef struct fox_weights fox_weights;

/* For FOX_WEIGHTS_DEVICE, data is an opaque device tensor handle
 * (const fox_gpu_tensor *, include/fox_gpu.h) and bytes the GGUF size. */
typedef struct {
    const void *data;
    uint64_t    bytes;
    size_t      tensor_index;
    void       *slot;
} fox_weights_lease;

fox_status fox_weights_open(const char *gguf_path, fox_weights_mode mode,
                            uint64_t budget_bytes, fox_weights **out);
void       fox_weights_close(fox_weights *w);
/* include/fox/fox.h:390: the parsed file behind the handle (owned by w) */
const fox_gguf  *fox_weights_model(const fox_weights *w);
fox_weights_mode fox_weights_get_mode(const fox_weights *w);
size_t     fox_weights_tensor_count(const fox_weights *w);             /* EXTENSION */
size_t     fox_weights_tensor_find(const fox_weights *w, const char *name); /* EXTENSION */
fox_status fox_weights_acquire(fox_weights *w, size_t tensor_index,
                               fox_weights_lease *lease);
void       fox_weights_release(fox_weights *w, fox_weights_lease *lease);
fox_status fox_weights_prefetch(fox_weights *w, size_t tensor_index);
fox_status fox_weights_prefetch_async(fox_weights *w, size_t tensor_index);
fox_status fox_weights_prefetch_wait(fox_weights *w, size_t tensor_index);
size_t     fox_weights_live_leases(const fox_weights *w);
uint64_t   fox_weights_resident_bytes(const fox_weights *w);
uint64_t   fox_weights_reads(const fox_weights *w);
uint64_t   fox_weights_evictions(const fox_weights *w);

/* -------------------------------------------------------- model / eval */

/* include/fox/fox.h:405-420 */
typedef struct {
    char     arch[32];
    char     name[FOX_NAME_MAX];
    uint32_t n_layer;
    uint32_t n_embd;
    uint32_t n_head;
    uint32_t n_head_kv;
    uint32_t n_ff;
    uint32_t head_dim;
    uint32_t n_vocab;
    uint32_t n_ctx_train;
    float    rms_eps;
    float    rope_freq_base;
    uint64_t weight_bytes;
    int      tied_output;
} fox_model_info;

typedef struct fox_model   fox_model;
typedef struct fox_context fox_context;

/* include/fox/fox.h:425-431.  The GPU is HIP device FOX_DEVICE (environment,
 * default 0).  FOX_MAX_WORKGROUPS=n (environment) caps the fused GEMVs'
 * persistent grid (fox_gpu_set_max_workgroups); results do not change. */
fox_status fox_model_open(const char *gguf_path, fox_weights_mode mode,
                          uint64_t budget_bytes, fox_model **out);
void       fox_model_close(fox_model *m);
const fox_model_info *fox_model_get_info(const fox_model *m);
fox_weights          *fox_model_weights(fox_model *m);

/* include/fox/fox.h:433-451 */
typedef struct {
    uint32_t n_ctx;
    uint32_t n_batch;
    int      n_threads;   /* kept for the ABI; the GPU path ignores it */
} fox_context_config;

void       fox_context_config_default(fox_context_config *cfg, const fox_model *m);
fox_status fox_context_create(fox_model *m, const fox_context_config *cfg,
                              fox_context **out);
void       fox_context_destroy(fox_context *ctx);
void       fox_context_reset(fox_context *ctx);
/* logits of the last token, host memory owned by ctx, valid until the next
 * eval or destroy (src/forward.c:411-438) */
fox_status fox_eval(fox_context *ctx, const uint32_t *tokens, size_t n_tokens,
                    float **logits_out);
/* EXTENSION.  The logits of every one of the n_tokens positions, row i
 * those of token i (as fox_eval would return after tokens[0..i]), into
 * caller-owned host memory of n_tokens * n_vocab floats: speculative
 * verification checks all drafted positions in one pass.  RustFox computes
 * the last position's only (src/forward.c:401-408). */
fox_status fox_eval_all(fox_context *ctx, const uint32_t *tokens, size_t n_tokens,
                        float *logits);
uint32_t   fox_context_position(const fox_context *ctx);
double     fox_context_last_eval_seconds(const fox_context *ctx);
uint64_t   fox_context_weight_reads(const fox_context *ctx);

/* EXTENSION.  Greedy decode kept on the device: feed `token` at the current
 * position, then n_steps times take the first argmax of the logits
 * (src/sample.c:147-153, repeat penalty 1.0) as the next input.  out_ids
 * receives the n_steps chosen ids.  The step is one captured HIP graph, so
 * no logits cross PCIe.  Equivalent to fox_eval + argmax per step. */
fox_status fox_decode_greedy(fox_context *ctx, uint32_t token, size_t n_steps,
                             uint32_t *out_ids);

/* EXTENSION.  Write rows [p0, p0+n) of one layer's K and V cache (n_head_kv *
 * head_dim floats per row, host memory) and set the position: a pre-filled
 * cache without a prefill pass.  RustFox keeps its cache private. */
fox_status fox_context_set_kv(fox_context *ctx, uint32_t layer, uint32_t p0, uint32_t n,
                              const float *k, const float *v);
fox_status fox_context_set_position(fox_context *ctx, uint32_t pos);

/* EXTENSION.  Attention summation order.  exact != 0 (the default) sums in
 * the reference's order and reproduces its logits bit for bit; exact == 0
 * splits positions over workgroups (flash-decoding), logits equal within
 * float rounding.  The environment variable FOX_ATTENTION=split sets the
 * default of new contexts. */
fox_status fox_context_set_attention(fox_context *ctx, int exact);

/* ------------------------------------------------------------- sampler */

/* include/fox/fox.h:453-469 */
typedef struct {
    float    temperature;
    int      top_k;
    float    top_p;
    float    repeat_penalty;
    uint32_t repeat_last_n;
    uint64_t seed;
} fox_sampler_config;

typedef struct fox_sampler fox_sampler;

void         fox_sampler_config_default(fox_sampler_config *cfg);
fox_sampler *fox_sampler_create(const fox_sampler_config *cfg, size_t n_vocab);
void         fox_sampler_destroy(fox_sampler *s);
void         fox_sampler_accept(fox_sampler *s, uint32_t token);
fox_status   fox_sampler_pick(fox_sampler *s, const float *logits, uint32_t *out);

#ifdef __cplusplus
}
#endif
#endif
