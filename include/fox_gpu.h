/*
 * fox_gpu.h -- C ABI of the MI355X (gfx950) decode path for RustFox.
 *
 * The RustFox host code (forward.c, weights.c, model.c) keeps its own API and
 * calls this thin layer instead of its CPU kernels when a model is opened
 * with the HBM-resident backend.  Everything here is plain C: opaque
 * handles, device pointers as plain typed pointers, sizes as size_t, and the status
 * numbering of fox_status (include/fox/fox.h:17-26 in RustFox).
 *
 * Conventions (the reference's, src/gemv.c:74-97, src/kernels.c:809-872):
 *   - every call returns a fox_gpu_status; FOX_GPU_OK is 0;
 *   - NULL pointers, zero sizes and ragged K -> FOX_GPU_ERR_ARG;
 *     unknown tensor types -> FOX_GPU_ERR_UNSUPPORTED; allocation failures
 *     -> FOX_GPU_ERR_NOMEM; a failing HIP call -> FOX_GPU_ERR_INTERNAL;
 *     a message naming the problem is kept per thread, fox_gpu_last_error();
 *   - "device pointer" arguments point into memory from fox_gpu_malloc (or
 *     any HIP device allocation on the context's device);
 *   - compute calls are asynchronous on the context's stream and keep stream
 *     order; fox_gpu_sync() or a copy to the host waits for them;
 *   - a context is driven by one host thread at a time (the reference's
 *     pool contract, src/threadpool.c:151-178); contexts are independent.
 *
 * Matrices follow GGUF: ne0 = K = columns (elements per row), ne1 = N =
 * rows; gemv computes out[t][r] = sum_k W[r][k] * x[t][k] for M tokens.
 */
#ifndef FOX_GPU_H
#define FOX_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    FOX_GPU_OK = 0,
    FOX_GPU_ERR_ARG,
    FOX_GPU_ERR_IO,
    FOX_GPU_ERR_NOMEM,
    FOX_GPU_ERR_FORMAT,
    FOX_GPU_ERR_UNSUPPORTED,
    FOX_GPU_ERR_NOTFOUND,
    FOX_GPU_ERR_INTERNAL
} fox_gpu_status;

/* ggml type ids (include/fox/fox.h:213-224) understood by the device path
 * (Q4_0, Q8_0 and Q5_K by fox_gpu_dequant only) */
enum {
    FOX_GPU_F32 = 0, FOX_GPU_F16 = 1, FOX_GPU_Q4_0 = 2, FOX_GPU_Q8_0 = 8,
    FOX_GPU_Q4_K = 12, FOX_GPU_Q5_K = 13, FOX_GPU_Q6_K = 14,
    FOX_GPU_TQ1_0 = 34, FOX_GPU_TQ2_0 = 35
};

/* largest token count of one multi-token gemv / forward call */
#define FOX_GPU_MAX_TOKENS 8

typedef struct fox_gpu_ctx    fox_gpu_ctx;
typedef struct fox_gpu_tensor fox_gpu_tensor;

/* ---------------------------------------------------------- lifecycle */

/* Open device `device` (HIP ordinal) with one stream.  Replaces the CPU pool
 * of fox_threadpool_create (include/fox/fox.h:333). */
fox_gpu_status fox_gpu_init(int device, fox_gpu_ctx **out);
void           fox_gpu_shutdown(fox_gpu_ctx *ctx);
/* message of the last failure on this thread (src/log.c:40-57 analogue) */
const char    *fox_gpu_last_error(void);
const char    *fox_gpu_status_str(fox_gpu_status s);
fox_gpu_status fox_gpu_device_info(fox_gpu_ctx *ctx, char *name, size_t cap,
                                   int *compute_units, uint64_t *hbm_bytes);
/* Upper bound on the persistent grid of the fused GEMVs (fox_gpu_gemv,
 * _gemv_rmsnorm, _qkv_rope, _gate_up_silu on ternary weights); 0, the
 * default, means two workgroups per compute unit.  A small bound makes
 * every workgroup walk many row tiles in turn: results are unchanged
 * (each output row is combined by one workgroup in block order), only the
 * speed differs.  No counterpart in RustFox: the CPU pool's thread count
 * (src/threadpool.c:76) plays this role there. */
fox_gpu_status fox_gpu_set_max_workgroups(fox_gpu_ctx *ctx, int n);
/* Bytes of device memory the context's workspace holds now (it grows on
 * demand and never shrinks; earlier, smaller workspaces a captured graph may
 * still address are not counted).  No counterpart in RustFox, whose scratch
 * is per-thread stack and heap: a diagnostic for callers that must not let
 * a call allocate (fox_gpu_gemv_noalloc leaves it unchanged). */
size_t         fox_gpu_workspace_bytes(const fox_gpu_ctx *ctx);

/* ------------------------------------------------------------- memory */

fox_gpu_status fox_gpu_malloc(fox_gpu_ctx *ctx, size_t bytes, void **out);
fox_gpu_status fox_gpu_free(fox_gpu_ctx *ctx, void *ptr);
/* blocking copies; the device-to-host copy first waits for queued work */
fox_gpu_status fox_gpu_memcpy_h2d(fox_gpu_ctx *ctx, void *dst, const void *src, size_t n);
fox_gpu_status fox_gpu_memcpy_d2h(fox_gpu_ctx *ctx, void *dst, const void *src, size_t n);
/* stream-ordered device copy and byte fill (a kernel, safe under capture) */
fox_gpu_status fox_gpu_memcpy_d2d(fox_gpu_ctx *ctx, void *dst, const void *src, size_t n);
fox_gpu_status fox_gpu_memset(fox_gpu_ctx *ctx, void *dst, int value, size_t n);
fox_gpu_status fox_gpu_sync(fox_gpu_ctx *ctx);

/* ------------------------------------------------------------ weights */

/* Upload one GGUF tensor (`bytes` = its GGUF size, host pointer) into HBM.
 * Block types are repacked into the device layout (same byte count plus
 * padding of the row count to 16), except TQ1_0, which is held as TQ2_0
 * blocks of the same trits (66 B instead of 54 B per 256 weights: the GEMVs
 * then decode 2-bit fields; results are unchanged).  F16/F32 are laid out in
 * 256-row tiles of 128-byte row chunks (fox_gpu_tensor_download gives
 * row-major bytes back).
 * Backs the FOX_WEIGHTS_DEVICE mode of fox_weights_open
 * (include/fox/fox.h:372-387), loaded once per tensor like the resident
 * backend (src/weights.c:461-496). */
fox_gpu_status fox_gpu_tensor_upload(fox_gpu_ctx *ctx, int type, uint64_t ne0,
                                     uint64_t ne1, const void *host, uint64_t bytes,
                                     fox_gpu_tensor **out);
fox_gpu_status fox_gpu_tensor_info(const fox_gpu_tensor *t, int *type, uint64_t *ne0,
                                   uint64_t *ne1, uint64_t *gguf_bytes,
                                   uint64_t *device_bytes);
/* Copy the tensor back in its GGUF byte layout (inverse repack).  TQ1_0
 * bytes come back as the canonical encoding ceil(q * 256 / 243) of their
 * trits, the byte the reference's quantiser writes; a byte that decodes to
 * the same trits otherwise comes back as that canonical byte. */
fox_gpu_status fox_gpu_tensor_download(fox_gpu_ctx *ctx, const fox_gpu_tensor *t,
                                       void *host, uint64_t bytes);
void           fox_gpu_tensor_free(fox_gpu_ctx *ctx, fox_gpu_tensor *t);

/* ---------------------------------------------------- streamed weights */

/* The pieces of a streaming weight backend (the GPU form of RustFox's
 * storage-streamed slots, src/weights.c:248-459, with its layer-ahead
 * prefetch, src/forward.c:322-337): tensors allocated once and reloaded in
 * place, pinned host staging, and a second stream (the context's copy
 * stream) on which uploads run beside the compute stream.
 *
 * fox_gpu_tensor_alloc: a device tensor of the given type and shape, its
 * contents undefined until loaded.
 * fox_gpu_tensor_load_async: on the copy stream, copy `bytes` GGUF bytes
 * from `host` (pinned memory from fox_gpu_host_alloc, left untouched until
 * the copy stream has passed this call) into `dev_stage` (device memory of
 * at least `bytes`, reused only in copy-stream order) and repack them into
 * t's device layout; with `host` NULL the bytes are already in `dev_stage`
 * (fox_gpu_stage_async) and only the repack runs.  Nothing waits: order it
 * against compute-stream users of t with events.
 * fox_gpu_stage_async: on the copy stream, copy `bytes` from pinned `host`
 * memory to device memory `dev` (a streamed layer's tensors in one copy,
 * then one repack each; src/weights.c:314-459 reads a layer into its slot). */
fox_gpu_status fox_gpu_tensor_alloc(fox_gpu_ctx *ctx, int type, uint64_t ne0,
                                    uint64_t ne1, fox_gpu_tensor **out);
fox_gpu_status fox_gpu_tensor_load_async(fox_gpu_ctx *ctx, fox_gpu_tensor *t,
                                         const void *host, uint64_t bytes,
                                         void *dev_stage);
fox_gpu_status fox_gpu_stage_async(fox_gpu_ctx *ctx, void *dev, const void *host,
                                   uint64_t bytes);
fox_gpu_status fox_gpu_host_alloc(fox_gpu_ctx *ctx, size_t bytes, void **out);
fox_gpu_status fox_gpu_host_free(fox_gpu_ctx *ctx, void *p);

/* -------------------------------------------------------- activations */

typedef enum {
    FOX_GPU_ACT_PER_VECTOR = 0,  /* one scale per token: src/gemv.c:11-42   */
    FOX_GPU_ACT_PER_BLOCK  = 1   /* one per 256 values:  src/kernels.c:722-754 */
} fox_gpu_act_mode;

/* x: M rows of K floats (row stride x_stride floats) -> q: M x K int8,
 * scale: M floats (PER_VECTOR) or M x K/256 floats (PER_BLOCK).
 * Replaces fox_quantize_activations_i8 (include/fox/fox.h:342-343). */
fox_gpu_status fox_gpu_quantize(fox_gpu_ctx *ctx, int mode, const float *x,
                                size_t K, size_t M, size_t x_stride,
                                int8_t *q, float *scale);

/* ---------------------------------------------------------------- gemv */

/* out[t*out_stride + r] = W x[t] for t < M <= FOX_GPU_MAX_TOKENS.  Quantises
 * x the way fox_gemv does for the tensor's type (kernels.c:809-872) and
 * reproduces its per-row block-ordered float combine.
 * Replaces fox_gemv (include/fox/fox.h:363-365). */
#define FOX_GPU_GEMV_ACCUMULATE 1u  /* out = out + W x (the residual add,
                                        src/ops.c:50-54, fused) */
fox_gpu_status fox_gpu_gemv(fox_gpu_ctx *ctx, const fox_gpu_tensor *w,
                            const float *x, size_t x_stride, size_t M,
                            float *out, size_t out_stride, unsigned flags);

/* fox_gpu_gemv without any allocation.  No counterpart in RustFox: it is
 * for callers that cannot allocate device memory -- work under HIP graph
 * capture, tight serving loops, hosts that forbid allocation after start-up.
 * Same arguments and results as fox_gpu_gemv; where fox_gpu_gemv would grow
 * the context's workspace (K-quant weights, ternary rows wider than the
 * fused path takes), the activations go to a fixed 2 MiB scratch that the
 * library holds on each GPU until the process ends (its address resolved at
 * fox_gpu_init).  Inputs needing more scratch than that are refused with
 * FOX_GPU_ERR_ARG.  Every call on a GPU shares its scratch, so calls that
 * overlap in time on one GPU (two streams, two host threads) race. */
fox_gpu_status fox_gpu_gemv_noalloc(fox_gpu_ctx *ctx, const fox_gpu_tensor *w,
                                    const float *x, size_t x_stride, size_t M,
                                    float *out, size_t out_stride, unsigned flags);

/* Several matrices with the same K applied to one input (q/k/v, gate/up):
 * the input is quantised once.  outs[i] receives rows of ws[i]. */
fox_gpu_status fox_gpu_gemv_multi(fox_gpu_ctx *ctx, size_t n,
                                  const fox_gpu_tensor *const *ws,
                                  const float *x, size_t x_stride, size_t M,
                                  float *const *outs, const size_t *out_strides,
                                  unsigned flags);

/* Pre-quantised entry: q is M x K int8, scale as produced by
 * fox_gpu_quantize for the tensor's type.  Replaces fox_gemv_tq1_i8 /
 * fox_gemv_tq2_i8 (include/fox/fox.h:350-355) and gemv_qk_i8
 * (src/kernels.c:780-805). */
fox_gpu_status fox_gpu_gemv_i8(fox_gpu_ctx *ctx, const fox_gpu_tensor *w,
                               const int8_t *q, const float *scale, size_t M,
                               float *out, size_t out_stride);

/* Integer block sums, the bit-exact part of the contract: for token t, row r,
 * block b: TQ1_0/TQ2_0 one int32 (src/ternary.c:73-93, 177-188), Q4_K the
 * eight sub-block dots D_j (src/kernels.c:571-602), Q6_K the four scaled
 * group sums G (src/kernels.c:636-661).  sums is device memory of
 * M x N x K/256 x {1, 8, 4} int32. */
fox_gpu_status fox_gpu_block_sums(fox_gpu_ctx *ctx, const fox_gpu_tensor *w,
                                  const int8_t *q, size_t M, int32_t *sums);

/* One-launch stages of a decode layer (src/forward.c:318-397): the input
 * stage (RMSNorm, int8 quantisation) runs inside the GEMV's workgroups,
 * results bit-identical to the separate calls.  TQ1_0 / TQ2_0 weights for
 * 1 to FOX_GPU_MAX_TOKENS tokens, Q4_K / Q6_K weights for one token; other
 * cases return FOX_GPU_ERR_UNSUPPORTED (use the separate calls), and so do
 * activations too large for one workgroup's LDS.
 *
 * y_i = W_i rmsnorm(x, norm_w) for up to 4 matrices of one type and width
 * (flags as fox_gpu_gemv; the attn_norm / ffn_norm + project steps). */
fox_gpu_status fox_gpu_gemv_rmsnorm(fox_gpu_ctx *ctx, size_t n,
                                    const fox_gpu_tensor *const *ws, const float *x,
                                    size_t x_stride, size_t M, const float *norm_w,
                                    float eps, float *const *outs,
                                    const size_t *out_strides, unsigned flags);

/* xb = rmsnorm(x, norm_w); q, k, v = W xb; RoPE on q and k at pos[0] + t;
 * q -> q_out, k and v -> the layer's caches (layouts as fox_gpu_rope_store).
 * One launch when q and k share one type and v has it too, or when all three
 * are K-quants (Q4_K and Q6_K in any mix, one token); q and k of one type
 * and v of another otherwise run as two launches. */
fox_gpu_status fox_gpu_qkv_rope(fox_gpu_ctx *ctx, const fox_gpu_tensor *wq,
                                const fox_gpu_tensor *wk, const fox_gpu_tensor *wv,
                                const float *x, size_t x_stride, size_t M,
                                const float *norm_w, float eps, float *q_out,
                                size_t q_stride, const float *cos_t, const float *sin_t,
                                const uint32_t *pos, size_t n_ctx, float *k_cache,
                                float *v_cache, size_t head_dim);

/* xb = rmsnorm(x, norm_w); h = silu(W_gate xb) * (W_up xb). */
fox_gpu_status fox_gpu_gate_up_silu(fox_gpu_ctx *ctx, const fox_gpu_tensor *w_gate,
                                    const fox_gpu_tensor *w_up, const float *x,
                                    size_t x_stride, size_t M, const float *norm_w,
                                    float eps, float *h_out, size_t h_stride);

/* Prepared activations: x quantised once for one weight type and width, in
 * its own device buffer, then applied to any number of matrices of that
 * type and width with one kernel launch each (fox_gpu_gemv_act).  Block
 * types only; F16/F32 matrices read float activations directly. */
typedef struct fox_gpu_act fox_gpu_act;
fox_gpu_status fox_gpu_act_prepare(fox_gpu_ctx *ctx, int type, const float *x, size_t K,
                                   size_t M, size_t x_stride, fox_gpu_act **out);
fox_gpu_status fox_gpu_gemv_act(fox_gpu_ctx *ctx, const fox_gpu_tensor *w,
                                const fox_gpu_act *act, float *out, size_t out_stride,
                                unsigned flags);
void           fox_gpu_act_free(fox_gpu_ctx *ctx, fox_gpu_act *act);

/* ---------------------------------------------------------------- ops */

/* Rows of a tensor as f32 (fox_dequant_row, include/fox/fox.h:367-368):
 * out[i*out_stride ..] = row rows[i] for i < n; rows is device uint32.
 * A row index >= ne1 is not read: its output is left untouched and the
 * device flag *bad (if non-NULL) is set to 1.  Covers embed
 * (src/forward.c:259-293) and norm weights (src/forward.c:167-186). */
fox_gpu_status fox_gpu_get_rows(fox_gpu_ctx *ctx, const fox_gpu_tensor *t,
                                const uint32_t *rows, size_t n, float *out,
                                size_t out_stride, uint32_t *bad);

/* n elements of one row held in its GGUF bytes (device memory) as f32:
 * F32, F16, Q8_0, Q4_0, Q4_K, Q5_K and Q6_K with the reference's arithmetic
 * (src/kernels.c:874-941; NaN payloads kept as the reference's field
 * conversion keeps them).  Other types -> FOX_GPU_ERR_UNSUPPORTED, n not a
 * whole number of blocks -> FOX_GPU_ERR_ARG.  Backs fox_dequant_row
 * (include/fox/fox.h:367-368). */
fox_gpu_status fox_gpu_dequant(fox_gpu_ctx *ctx, int type, const void *row, size_t n,
                               float *out);

/* out = x * (1/sqrt(mean(x^2) + eps)) * w per row (src/ops.c:7-22). */
fox_gpu_status fox_gpu_rmsnorm(fox_gpu_ctx *ctx, float *out, size_t out_stride,
                               const float *x, size_t x_stride, const float *w,
                               size_t n, size_t M, float eps);

/* RoPE on q (n_head heads) and k (n_head_kv heads) of M tokens at positions
 * pos[0] + t, adjacent pairs (src/ops.c:56-73) with the host-built tables
 * (src/forward.c:104-118), then k and v rows stored into the layer's cache
 * rows pos[0] + t (src/forward.c:346-362).  A token whose position is not
 * below n_ctx is neither rotated nor stored.
 *
 * Cache layout: k_cache is f32 [n_ctx][kv_dim] (the reference's); v_cache is
 * position-quad interleaved, element (p, c) at ((p/4)*kv_dim + c)*4 + p%4,
 * and holds FOX_GPU_V_CACHE_FLOATS(n_ctx, kv_dim) floats.  Four consecutive
 * positions of a column are one 16-byte load for the value sums. */
#define FOX_GPU_V_CACHE_FLOATS(n_ctx, kv_dim) ((((size_t)(n_ctx) + 3) / 4) * 4 * (size_t)(kv_dim))
fox_gpu_status fox_gpu_rope_store(fox_gpu_ctx *ctx, float *q, size_t q_stride,
                                  float *k, size_t k_stride,
                                  const float *v, size_t v_stride,
                                  size_t n_head, size_t n_head_kv, size_t head_dim,
                                  size_t M, const float *cos_t, const float *sin_t,
                                  const uint32_t *pos, size_t n_ctx,
                                  float *k_cache, float *v_cache);

/* Rows p0 .. p0+n-1 of a layer's caches from device row-major k, v
 * [n][kv_dim] (pre-filling a cache; src/forward.c:346-362 stores rows one
 * token at a time). */
fox_gpu_status fox_gpu_kv_write(fox_gpu_ctx *ctx, float *k_cache, float *v_cache,
                                size_t kv_dim, size_t n_ctx, size_t p0, size_t n,
                                const float *k, const float *v);

/* Causal GQA attention of M tokens at positions pos[0] + t over cache rows
 * 0 .. pos[0] + t: softmax(q.k / sqrt(hd)) v (src/forward.c:222-257).
 * FOX_GPU_ATTN_EXACT computes every sum in the reference's order (scores in
 * head-dimension order, softmax and value sums in position order) and
 * reproduces it bit for bit; FOX_GPU_ATTN_SPLIT splits positions over
 * workgroups and merges the partial softmaxes (flash-decoding), equal to it
 * within float rounding. */
enum { FOX_GPU_ATTN_SPLIT = 0, FOX_GPU_ATTN_EXACT = 1 };
fox_gpu_status fox_gpu_attention(fox_gpu_ctx *ctx, float *out, size_t out_stride,
                                 const float *q, size_t q_stride,
                                 const float *k_cache, const float *v_cache,
                                 size_t n_head, size_t n_head_kv, size_t head_dim,
                                 size_t M, const uint32_t *pos, size_t n_ctx, int mode);


/* gate = silu(gate) * up (src/ops.c:41-48) and dst += src (src/ops.c:50-54)
 * on M rows of n. */
fox_gpu_status fox_gpu_silu_mul(fox_gpu_ctx *ctx, float *gate, const float *up,
                                size_t n, size_t M, size_t stride);
fox_gpu_status fox_gpu_add(fox_gpu_ctx *ctx, float *dst, const float *src,
                           size_t n, size_t M, size_t stride);

/* first index of the maximum (src/sample.c:147-153) -> *idx (device uint32).
 * With pos != NULL the device position is advanced by `advance` in the same
 * launch, and with history != NULL history[pos before the advance] = *idx:
 * the bookkeeping of a decode loop kept on the device. */
fox_gpu_status fox_gpu_argmax(fox_gpu_ctx *ctx, const float *logits, size_t n,
                              uint32_t *idx, uint32_t *pos, uint32_t advance,
                              uint32_t *history);

/* ------------------------------------------------------------- graphs */

/* Record the work queued on the context's stream between begin and end into
 * a replayable HIP graph (whole-token decode).  Kernels read the position
 * from device memory, so one graph serves every step. */
typedef struct fox_gpu_graph fox_gpu_graph;
fox_gpu_status fox_gpu_graph_begin(fox_gpu_ctx *ctx);
fox_gpu_status fox_gpu_graph_end(fox_gpu_ctx *ctx, fox_gpu_graph **out);
fox_gpu_status fox_gpu_graph_launch(fox_gpu_ctx *ctx, fox_gpu_graph *g);
void           fox_gpu_graph_free(fox_gpu_graph *g);

/* ------------------------------------------------------------- timing */

/* HIP events recorded on the context's stream (the stream the kernels run
 * on): elapsed milliseconds between two records. */
typedef struct fox_gpu_event fox_gpu_event;
fox_gpu_status fox_gpu_event_create(fox_gpu_ctx *ctx, fox_gpu_event **out);
fox_gpu_status fox_gpu_event_record(fox_gpu_ctx *ctx, fox_gpu_event *e);
fox_gpu_status fox_gpu_event_elapsed(fox_gpu_event *start, fox_gpu_event *stop,
                                     float *ms);
/* Ordering between the compute stream and the copy stream: record on the
 * copy stream; make the compute stream (on_copy = 0) or the copy stream
 * (on_copy = 1) wait for an event; wait on the host. */
fox_gpu_status fox_gpu_event_record_copy(fox_gpu_ctx *ctx, fox_gpu_event *e);
fox_gpu_status fox_gpu_event_wait(fox_gpu_ctx *ctx, fox_gpu_event *e, int on_copy);
fox_gpu_status fox_gpu_event_sync(fox_gpu_event *e);
void           fox_gpu_event_destroy(fox_gpu_event *e);

#ifdef __cplusplus
}
#endif
#endif
