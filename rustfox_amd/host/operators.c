/* operators.c -- RustFox's operator entry points on host buffers
 * (include/fox/fox.h:322-368), computed on the GPU.
 *
 * Same names, arguments, status codes and results as the reference: the
 * caller owns every buffer, nothing is retained, a call blocks until its
 * result is in the caller's memory.  Each call copies its operands into
 * HBM, runs the device kernels of include/fox_gpu.h (the weights go
 * through the same upload and repack as a FOX_WEIGHTS_DEVICE model) and
 * copies the result back; that PCIe round trip makes these entries a
 * compatibility path, not the decode path, which keeps weights resident.
 *
 * The calls share one device context per process (HIP device FOX_DEVICE),
 * created on first use and serialised by a lock: the operators are
 * thread-safe like the reference's.  The pool argument is accepted for the
 * ABI and not used (the launch grid replaces the CPU pool;
 * src/threadpool.c:151-178), and NULL is accepted as in the reference.
 */
#include "fox_host_internal.h"

#include <stdlib.h>
#include <string.h>
#include <unistd.h>

struct fox_threadpool {
    int n_threads;
};

/* src/threadpool.c:71-78: n <= 0 means the online core count, at most 256 */
fox_threadpool *fox_threadpool_create(int n_threads)
{
    fox_threadpool *tp;
    if (n_threads <= 0) n_threads = (int)sysconf(_SC_NPROCESSORS_ONLN);
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 256) n_threads = 256;
    tp = (fox_threadpool *)calloc(1, sizeof(*tp));
    if (!tp) {
        fox_fail(FOX_ERR_NOMEM, "threadpool: handle");
        return NULL;
    }
    tp->n_threads = n_threads;
    return tp;
}

void fox_threadpool_destroy(fox_threadpool *tp) { free(tp); }

int fox_threadpool_size(const fox_threadpool *tp) { return tp ? tp->n_threads : 1; }

/* include/fox/fox.h:337-338.  A caller's own host callback runs on the
 * calling thread over the whole range, every index once (the reference's
 * NULL-pool behaviour, src/threadpool.c:157-160): this library has no CPU
 * worker threads; its kernels spread work over the launch grid instead. */
fox_status fox_parallel_for(fox_threadpool *tp, size_t n, fox_parallel_fn fn, void *ctx)
{
    (void)tp;
    if (!fn) return FOX_ERR_ARG;
    if (n == 0) return FOX_OK;
    fn(ctx, 0, 0, n);
    return FOX_OK;
}

/* ------------------------------------------------------ shared device */

static pthread_mutex_t g_lock = PTHREAD_MUTEX_INITIALIZER;
static fox_gpu_ctx *g_gpu;

static fox_status device(fox_gpu_ctx **out)
{
    if (!g_gpu) {
        const char *e = getenv("FOX_DEVICE");
        fox_gpu_status gs = fox_gpu_init(e && *e ? atoi(e) : 0, &g_gpu);
        if (gs != FOX_GPU_OK) {
            g_gpu = NULL;
            return fox_gpu_failed(gs, "operators: no usable GPU");
        }
    }
    *out = g_gpu;
    return FOX_OK;
}

/* device buffers of one call, freed together */
typedef struct {
    fox_gpu_ctx *gpu;
    void *buf[4];
    int n;
    fox_gpu_tensor *t;
} call_mem;

static fox_status cm_alloc(call_mem *m, size_t bytes, const void *host, void **out)
{
    fox_gpu_status gs = fox_gpu_malloc(m->gpu, bytes ? bytes : 4, out);
    if (gs != FOX_GPU_OK) return fox_gpu_failed(gs, "operators: device buffer");
    m->buf[m->n++] = *out;
    if (host && bytes) {
        gs = fox_gpu_memcpy_h2d(m->gpu, *out, host, bytes);
        if (gs != FOX_GPU_OK) return fox_gpu_failed(gs, "operators: copy to the device");
    }
    return FOX_OK;
}

static void cm_free(call_mem *m)
{
    int i;
    if (m->gpu) fox_gpu_sync(m->gpu);
    for (i = 0; i < m->n; i++) fox_gpu_free(m->gpu, m->buf[i]);
    if (m->t) fox_gpu_tensor_free(m->gpu, m->t);
}

static fox_status cm_begin(call_mem *m)
{
    memset(m, 0, sizeof(*m));
    pthread_mutex_lock(&g_lock);
    return device(&m->gpu);
}

static fox_status cm_end(call_mem *m, fox_status st)
{
    cm_free(m);
    pthread_mutex_unlock(&g_lock);
    return st;
}

static fox_status cm_weights(call_mem *m, int type, const void *w, size_t rows, size_t cols)
{
    const size_t rb = fox_row_bytes((fox_ggml_type)type, cols);
    fox_gpu_status gs = fox_gpu_tensor_upload(m->gpu, type, cols, rows, w, (uint64_t)rb * rows,
                                              &m->t);
    if (gs != FOX_GPU_OK) {
        m->t = NULL;
        return fox_gpu_failed(gs, "operators: weights");
    }
    return FOX_OK;
}

#define TRY(x)                                \
    do {                                      \
        if ((st = (x)) != FOX_OK) return cm_end(&m, st); \
    } while (0)
#define GTRY(x, what)                                                     \
    do {                                                                  \
        fox_gpu_status gs_ = (x);                                         \
        if (gs_ != FOX_GPU_OK) return cm_end(&m, fox_gpu_failed(gs_, what)); \
    } while (0)

/* --------------------------------------------------------- quantiser */

/* include/fox/fox.h:342-343, src/gemv.c:11-42 */
fox_status fox_quantize_activations_i8(const float *x, size_t n, int8_t *q, float *scale)
{
    call_mem m;
    fox_status st;
    void *dx, *dq, *ds;
    if (!x || !q || !scale || n == 0) return FOX_ERR_ARG;
    TRY(cm_begin(&m));
    TRY(cm_alloc(&m, n * sizeof(float), x, &dx));
    TRY(cm_alloc(&m, n, NULL, &dq));
    TRY(cm_alloc(&m, sizeof(float), NULL, &ds));
    GTRY(fox_gpu_quantize(m.gpu, FOX_GPU_ACT_PER_VECTOR, (const float *)dx, n, 1, n,
                          (int8_t *)dq, (float *)ds), "quantize");
    GTRY(fox_gpu_memcpy_d2h(m.gpu, q, dq, n), "quantize: result");
    GTRY(fox_gpu_memcpy_d2h(m.gpu, scale, ds, sizeof(float)), "quantize: result");
    return cm_end(&m, FOX_OK);
}

/* ------------------------------------------------------------- gemv */

static fox_status check_gemv(const void *in, const void *w, size_t rows, size_t cols,
                             const float *out)
{
    if (!in || !w || !out) return FOX_ERR_ARG;
    if (rows == 0 || cols == 0) return FOX_ERR_ARG;
    return FOX_OK;
}

static fox_status ragged(size_t cols, fox_ggml_type type)
{
    return fox_fail(FOX_ERR_ARG, "gemv: %llu columns is not a whole number of %s blocks",
                    (unsigned long long)cols, fox_ggml_type_name(type));
}

/* out[r] = W_r . x with x quantised as fox_gemv quantises it for `type`
 * (src/kernels.c:809-872) */
static fox_status gemv_f32(fox_ggml_type type, const float *x, const void *w, size_t rows,
                           size_t cols, float *out)
{
    call_mem m;
    fox_status st;
    void *dx, *dout;
    if ((st = check_gemv(x, w, rows, cols, out)) != FOX_OK) return st;
    if (!fox_gemv_supports(type))
        return fox_fail(FOX_ERR_UNSUPPORTED, "gemv: no device kernel for %s; this library "
                        "handles F32, F16, Q4_K, Q6_K, TQ1_0 and TQ2_0",
                        fox_ggml_type_name(type));
    if (fox_row_bytes(type, cols) == 0) return ragged(cols, type);
    TRY(cm_begin(&m));
    TRY(cm_weights(&m, (int)type, w, rows, cols));
    TRY(cm_alloc(&m, cols * sizeof(float), x, &dx));
    TRY(cm_alloc(&m, rows * sizeof(float), NULL, &dout));
    GTRY(fox_gpu_gemv(m.gpu, m.t, (const float *)dx, cols, 1, (float *)dout, rows, 0), "gemv");
    GTRY(fox_gpu_memcpy_d2h(m.gpu, out, dout, rows * sizeof(float)), "gemv: result");
    return cm_end(&m, FOX_OK);
}

/* include/fox/fox.h:363-365 */
fox_status fox_gemv(fox_threadpool *tp, fox_ggml_type type, const float *x, const void *weights,
                    size_t n_rows, size_t n_cols, float *out)
{
    (void)tp;
    return gemv_f32(type, x, weights, n_rows, n_cols, out);
}

/* include/fox/fox.h:345-348, src/gemv.c:120-144 */
fox_status fox_gemv_tq1_f32(fox_threadpool *tp, const float *x, const void *weights,
                            size_t n_rows, size_t n_cols, float *out)
{
    (void)tp;
    if (!x || !weights || !out || n_rows == 0 || n_cols == 0) return FOX_ERR_ARG;
    if (n_cols % 256) return ragged(n_cols, FOX_GGML_TQ1_0);
    return gemv_f32(FOX_GGML_TQ1_0, x, weights, n_rows, n_cols, out);
}

fox_status fox_gemv_tq2_f32(fox_threadpool *tp, const float *x, const void *weights,
                            size_t n_rows, size_t n_cols, float *out)
{
    (void)tp;
    if (!x || !weights || !out || n_rows == 0 || n_cols == 0) return FOX_ERR_ARG;
    if (n_cols % 256) return ragged(n_cols, FOX_GGML_TQ2_0);
    return gemv_f32(FOX_GGML_TQ2_0, x, weights, n_rows, n_cols, out);
}

/* out[r] = (sum_b d_rb * (float)S_rb) * act_scale (src/gemv.c:54-97) */
static fox_status gemv_i8(fox_ggml_type type, const int8_t *q, float act_scale,
                          const void *w, size_t rows, size_t cols, float *out)
{
    call_mem m;
    fox_status st;
    void *dq, *ds, *dout;
    if ((st = check_gemv(q, w, rows, cols, out)) != FOX_OK) return st;
    if (cols % 256) return ragged(cols, type);
    TRY(cm_begin(&m));
    TRY(cm_weights(&m, (int)type, w, rows, cols));
    TRY(cm_alloc(&m, cols, q, &dq));
    TRY(cm_alloc(&m, sizeof(float), &act_scale, &ds));
    TRY(cm_alloc(&m, rows * sizeof(float), NULL, &dout));
    GTRY(fox_gpu_gemv_i8(m.gpu, m.t, (const int8_t *)dq, (const float *)ds, 1, (float *)dout,
                         rows), "gemv");
    GTRY(fox_gpu_memcpy_d2h(m.gpu, out, dout, rows * sizeof(float)), "gemv: result");
    return cm_end(&m, FOX_OK);
}

/* include/fox/fox.h:350-355 */
fox_status fox_gemv_tq1_i8(fox_threadpool *tp, const int8_t *q, float act_scale,
                           const void *weights, size_t n_rows, size_t n_cols, float *out)
{
    (void)tp;
    return gemv_i8(FOX_GGML_TQ1_0, q, act_scale, weights, n_rows, n_cols, out);
}

fox_status fox_gemv_tq2_i8(fox_threadpool *tp, const int8_t *q, float act_scale,
                           const void *weights, size_t n_rows, size_t n_cols, float *out)
{
    (void)tp;
    return gemv_i8(FOX_GGML_TQ2_0, q, act_scale, weights, n_rows, n_cols, out);
}

/* ---------------------------------------------------- block-row dots */

/* *out = sum over the n/256 blocks, in order from 0.0f, of d_b * (float)S_b
 * (src/ternary.c:190-246): one row of the i8 GEMV with activation scale
 * 1.0f, which multiplies exactly */
static fox_status tq_dot(fox_ggml_type type, const int8_t *x, const void *blk, size_t n,
                         float *out)
{
    if (!x || !blk || !out) return FOX_ERR_ARG;
    if (n == 0 || n % 256) return FOX_ERR_ARG;
    return gemv_i8(type, x, 1.0f, blk, 1, n, out);
}

/* include/fox/fox.h:322-329 */
fox_status fox_tq1_dot_i8(const int8_t *activations, const void *block_data, size_t n,
                          float *out)
{
    return tq_dot(FOX_GGML_TQ1_0, activations, block_data, n, out);
}

fox_status fox_tq2_dot_i8(const int8_t *activations, const void *block_data, size_t n,
                          float *out)
{
    return tq_dot(FOX_GGML_TQ2_0, activations, block_data, n, out);
}

/* the reference's portable variants compute the same sums
 * (tests/test_ternary.c checks scalar == SIMD) */
fox_status fox_tq1_dot_i8_scalar(const int8_t *activations, const void *block_data, size_t n,
                                 float *out)
{
    return tq_dot(FOX_GGML_TQ1_0, activations, block_data, n, out);
}

fox_status fox_tq2_dot_i8_scalar(const int8_t *activations, const void *block_data, size_t n,
                                 float *out)
{
    return tq_dot(FOX_GGML_TQ2_0, activations, block_data, n, out);
}

/* ---------------------------------------------------------- dequant */

/* include/fox/fox.h:367-368, src/kernels.c:874-941 */
fox_status fox_dequant_row(fox_ggml_type type, const void *row, size_t n, float *out)
{
    call_mem m;
    fox_status st;
    size_t rb;
    void *dw, *dout;
    if (!row || !out || n == 0) return FOX_ERR_ARG;
    rb = fox_row_bytes(type, n);
    if (rb == 0)
        return fox_fail(FOX_ERR_ARG, "dequant: %llu elements is not a whole number of %s blocks",
                        (unsigned long long)n, fox_ggml_type_name(type));
    if (type != FOX_GGML_F32 && type != FOX_GGML_F16 && type != FOX_GGML_Q8_0 &&
        type != FOX_GGML_Q4_0 && type != FOX_GGML_Q4_K && type != FOX_GGML_Q5_K &&
        type != FOX_GGML_Q6_K)
        return fox_fail(FOX_ERR_UNSUPPORTED, "dequant: %s is not implemented yet",
                        fox_ggml_type_name(type));
    TRY(cm_begin(&m));
    TRY(cm_alloc(&m, rb, row, &dw));
    TRY(cm_alloc(&m, n * sizeof(float), NULL, &dout));
    GTRY(fox_gpu_dequant(m.gpu, (int)type, dw, n, (float *)dout), "dequant");
    GTRY(fox_gpu_memcpy_d2h(m.gpu, out, dout, n * sizeof(float)), "dequant: result");
    return cm_end(&m, FOX_OK);
}
