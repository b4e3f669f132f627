/* forward.c -- fox_eval on the GPU (RustFox src/forward.c:56-132, 295-438 semantics).
 *
 * One decode pass, per layer (src/forward.c:318-397):
 *   xb = rmsnorm(x, attn_norm); q, k, v = W xb; rope(q, k) at pos + t and
 *   store k, v in the layer's cache (one launch for ternary weights);
 *   xb = attention; x += W_o xb (residual fused into the gemv);
 *   xb = rmsnorm(x, ffn_norm); hb = silu(W_gate xb) * (W_up xb) (one launch
 *   for ternary weights); x += W_down hb.
 * then xb = rmsnorm(x_last, output_norm) and logits = W_out xb.
 *
 * The K cache is f32 [n_layer][n_ctx][n_head_kv * head_dim] as in the
 * reference, the V cache the device's position-quad interleaved layout
 * (fox_gpu.h) per layer; the RoPE tables are built on the host in double exactly as
 * src/forward.c:104-118 and uploaded.  A pass takes at most
 * FOX_GPU_MAX_TOKENS tokens; fox_eval cuts its input into such passes, which
 * gives the same result as the reference's n_batch chunks because a token
 * depends only on the cache rows before it (batched == stepped,
 * tests/test_forward.c:258-272).
 */
#include "fox_host_internal.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

typedef struct {
    const fox_gpu_tensor *attn_q, *attn_k, *attn_v, *attn_out, *ffn_gate, *ffn_up, *ffn_down;
    float *attn_norm, *ffn_norm;   /* device f32 [n_embd] */
} dev_layer;

struct fox_context {
    fox_model          *m;
    fox_context_config  cfg;
    fox_gpu_ctx        *gpu;
    uint32_t            pos;
    size_t              d, nq, nkv, wide, ff, hd, vocab;
    dev_layer          *L;
    const fox_gpu_tensor *embd, *out;
    float              *out_norm;
    /* device activations */
    float *x, *xb, *q, *k, *v, *hb, *hb2, *dlogits;
    float *kc, *vc, *rc, *rs;
    uint32_t *dtok, *dpos, *dhist, *dzero;
    float *norms;                  /* all norm vectors, n_embd floats each */
    float *logits;                 /* host */
    double last_seconds;
    uint64_t reads_at_start;
    fox_gpu_graph *greedy;
    int attn_mode;                 /* FOX_GPU_ATTN_EXACT or FOX_GPU_ATTN_SPLIT */
    void *allocs[32];
    int n_allocs;
};

static double now_s(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + (double)ts.tv_nsec * 1e-9;
}

#define GPU(call, what)                                       \
    do {                                                      \
        fox_gpu_status gs_ = (call);                          \
        if (gs_ != FOX_GPU_OK) return fox_gpu_failed(gs_, what); \
    } while (0)

static fox_status dalloc(fox_context *c, size_t bytes, void **out)
{
    fox_gpu_status gs;
    if (c->n_allocs == (int)(sizeof(c->allocs) / sizeof(c->allocs[0])))
        return fox_fail(FOX_ERR_INTERNAL, "context: too many buffers");
    gs = fox_gpu_malloc(c->gpu, bytes ? bytes : 4, out);
    if (gs != FOX_GPU_OK)
        return fox_gpu_failed(gs, "context: cannot allocate working memory; try a smaller n_ctx");
    c->allocs[c->n_allocs++] = *out;
    return FOX_OK;
}

static const fox_gpu_tensor *dev_tensor(fox_model *m, size_t idx)
{
    return m->weights->dev[idx];
}

static int streaming(const fox_context *c)
{
    return c->m->weights->mode == FOX_WEIGHTS_STREAM;
}

void fox_context_config_default(fox_context_config *cfg, const fox_model *m)
{
    if (!cfg) return;
    memset(cfg, 0, sizeof(*cfg));
    cfg->n_ctx = m ? m->info.n_ctx_train : 2048;
    cfg->n_batch = 32;
    cfg->n_threads = 0;
    if (cfg->n_ctx == 0) cfg->n_ctx = 2048;
}

void fox_context_destroy(fox_context *c)
{
    int i;
    if (!c) return;
    if (c->greedy) fox_gpu_graph_free(c->greedy);
    if (c->gpu) {
        fox_gpu_sync(c->gpu);
        for (i = 0; i < c->n_allocs; i++) fox_gpu_free(c->gpu, c->allocs[i]);
    }
    free(c->L);
    free(c->logits);
    free(c);
}

/* device f32 copy of a norm vector into `dst` (src/forward.c:167-186
 * dequantises it per use; it never changes, so it is dequantised once) */
static fox_status norm_vector(fox_context *c, const fox_gpu_tensor *t, float *dst)
{
    GPU(fox_gpu_get_rows(c->gpu, t, c->dzero, 1, dst, c->d, NULL), "context: norm weights");
    return FOX_OK;
}

fox_status fox_context_create(fox_model *m, const fox_context_config *cfg, fox_context **out)
{
    fox_context *c;
    fox_context_config k;
    const fox_model_info *mi;
    fox_status st;
    size_t nb, half, p, i;
    float *tc, *ts;
    uint32_t l, zero = 0;

    if (!m || !out) return fox_fail(FOX_ERR_ARG, "context: null argument");
    *out = NULL;
    if (m->weights->mode == FOX_WEIGHTS_RESIDENT)
        return fox_fail(FOX_ERR_UNSUPPORTED,
                        "context: rustfox_amd computes on the GPU; open the model with "
                        "FOX_WEIGHTS_DEVICE or FOX_WEIGHTS_STREAM");
    if (cfg) k = *cfg;
    else fox_context_config_default(&k, m);
    if (k.n_ctx == 0) k.n_ctx = m->info.n_ctx_train;
    if (k.n_ctx == 0) k.n_ctx = 2048;
    if (k.n_batch == 0) k.n_batch = 32;
    if (k.n_batch > k.n_ctx) k.n_batch = k.n_ctx;
    mi = &m->info;

    c = (fox_context *)calloc(1, sizeof(*c));
    if (!c) return fox_fail(FOX_ERR_NOMEM, "context: handle");
    c->m = m;
    c->cfg = k;
    c->gpu = m->weights->gpu;
    c->d = mi->n_embd;
    c->hd = mi->head_dim;
    c->nq = (size_t)mi->n_head * mi->head_dim;
    c->nkv = (size_t)mi->n_head_kv * mi->head_dim;
    c->wide = c->nq > c->d ? c->nq : c->d;
    c->ff = mi->n_ff;
    c->vocab = mi->n_vocab;
    c->attn_mode = FOX_GPU_ATTN_EXACT;
    {
        const char *e = getenv("FOX_ATTENTION");
        if (e && strcmp(e, "split") == 0) c->attn_mode = FOX_GPU_ATTN_SPLIT;
    }
    nb = FOX_GPU_MAX_TOKENS;

    c->logits = (float *)calloc(c->vocab, sizeof(float));
    c->L = (dev_layer *)calloc(mi->n_layer, sizeof(dev_layer));
    if (!c->logits || !c->L) { fox_context_destroy(c); return fox_fail(FOX_ERR_NOMEM, "context: tables"); }

#define ALLOC(ptr, bytes) \
    if ((st = dalloc(c, (bytes), (void **)&(ptr))) != FOX_OK) { fox_context_destroy(c); return st; }
    ALLOC(c->x, nb * c->d * 4)
    ALLOC(c->xb, nb * c->wide * 4)
    ALLOC(c->q, nb * c->nq * 4)
    ALLOC(c->k, nb * c->nkv * 4)
    ALLOC(c->v, nb * c->nkv * 4)
    ALLOC(c->hb, nb * c->ff * 4)
    ALLOC(c->hb2, nb * c->ff * 4)
    ALLOC(c->dlogits, nb * c->vocab * 4)          /* nb rows for fox_eval_all */
    ALLOC(c->kc, (size_t)mi->n_layer * k.n_ctx * c->nkv * 4)
    ALLOC(c->vc, (size_t)mi->n_layer * FOX_GPU_V_CACHE_FLOATS(k.n_ctx, c->nkv) * 4)
    ALLOC(c->rc, (size_t)k.n_ctx * (c->hd / 2) * 4)
    ALLOC(c->rs, (size_t)k.n_ctx * (c->hd / 2) * 4)
    ALLOC(c->dtok, nb * 4)
    ALLOC(c->dpos, 4)
    ALLOC(c->dhist, (size_t)k.n_ctx * 4)
    ALLOC(c->dzero, 4)
    ALLOC(c->norms, (2 * (size_t)mi->n_layer + 1) * c->d * 4)
#undef ALLOC
    if (fox_gpu_memcpy_h2d(c->gpu, c->dzero, &zero, 4) != FOX_GPU_OK ||
        fox_gpu_memset(c->gpu, c->kc, 0, (size_t)mi->n_layer * k.n_ctx * c->nkv * 4) != FOX_GPU_OK ||
        fox_gpu_memset(c->gpu, c->vc, 0,
                       (size_t)mi->n_layer * FOX_GPU_V_CACHE_FLOATS(k.n_ctx, c->nkv) * 4) !=
            FOX_GPU_OK) {
        st = fox_gpu_failed(FOX_GPU_ERR_INTERNAL, "context: initialise buffers");
        fox_context_destroy(c);
        return st;
    }

    /* RoPE tables, src/forward.c:104-118 */
    half = c->hd / 2;
    tc = (float *)malloc((size_t)k.n_ctx * half * 4);
    ts = (float *)malloc((size_t)k.n_ctx * half * 4);
    if (!tc || !ts) {
        free(tc); free(ts);
        fox_context_destroy(c);
        return fox_fail(FOX_ERR_NOMEM, "context: rope tables");
    }
    for (p = 0; p < k.n_ctx; p++)
        for (i = 0; i < half; i++) {
            double ex = -2.0 * (double)i / (double)c->hd;
            double th = (double)p * pow((double)mi->rope_freq_base, ex);
            tc[p * half + i] = (float)cos(th);
            ts[p * half + i] = (float)sin(th);
        }
    st = FOX_OK;
    if (fox_gpu_memcpy_h2d(c->gpu, c->rc, tc, (size_t)k.n_ctx * half * 4) != FOX_GPU_OK ||
        fox_gpu_memcpy_h2d(c->gpu, c->rs, ts, (size_t)k.n_ctx * half * 4) != FOX_GPU_OK)
        st = fox_gpu_failed(FOX_GPU_ERR_INTERNAL, "context: upload rope tables");
    free(tc);
    free(ts);
    if (st != FOX_OK) { fox_context_destroy(c); return st; }

    if ((st = fox_weights_use(m->weights, m->token_embd, &c->embd)) != FOX_OK ||
        (st = fox_weights_use(m->weights, m->output, &c->out)) != FOX_OK) {
        fox_context_destroy(c);
        return st;
    }
    for (l = 0; l < mi->n_layer; l++) {
        const fox_layer_tensors *t = &m->layers[l];
        dev_layer *D = &c->L[l];
        const fox_gpu_tensor *an, *fn;
        D->attn_norm = c->norms + (2 * (size_t)l) * c->d;
        D->ffn_norm = c->norms + (2 * (size_t)l + 1) * c->d;
        if (streaming(c)) {
            /* the layer's matrices are taken from its slot at every pass;
             * its norm vectors are copied out once here */
            const fox_gpu_tensor *lt[FOX_LAYER_ROLES];
            st = fox_weights_use_layer(m->weights, l, lt);
            an = lt[FOX_ROLE_ATTN_NORM];
            fn = lt[FOX_ROLE_FFN_NORM];
        } else {
            D->attn_q = dev_tensor(m, t->attn_q);
            D->attn_k = dev_tensor(m, t->attn_k);
            D->attn_v = dev_tensor(m, t->attn_v);
            D->attn_out = dev_tensor(m, t->attn_out);
            D->ffn_gate = dev_tensor(m, t->ffn_gate);
            D->ffn_up = dev_tensor(m, t->ffn_up);
            D->ffn_down = dev_tensor(m, t->ffn_down);
            an = dev_tensor(m, t->attn_norm);
            fn = dev_tensor(m, t->ffn_norm);
            st = FOX_OK;
        }
        if (st == FOX_OK) st = norm_vector(c, an, D->attn_norm);
        if (st == FOX_OK) st = norm_vector(c, fn, D->ffn_norm);
        if (streaming(c)) fox_weights_done_layer(m->weights, l);
        if (st != FOX_OK) {
            fox_context_destroy(c);
            return st;
        }
    }
    c->out_norm = c->norms + 2 * (size_t)mi->n_layer * c->d;
    {
        const fox_gpu_tensor *on;
        if ((st = fox_weights_use(m->weights, m->output_norm, &on)) != FOX_OK ||
            (st = norm_vector(c, on, c->out_norm)) != FOX_OK) {
            fox_context_destroy(c);
            return st;
        }
    }
    if (fox_gpu_sync(c->gpu) != FOX_GPU_OK) {
        st = fox_gpu_failed(FOX_GPU_ERR_INTERNAL, "context: setup");
        fox_context_destroy(c);
        return st;
    }
    *out = c;
    return FOX_OK;
}

void fox_context_reset(fox_context *c)
{
    if (c) c->pos = 0;
}

uint32_t fox_context_position(const fox_context *c) { return c ? c->pos : 0; }
double fox_context_last_eval_seconds(const fox_context *c) { return c ? c->last_seconds : 0.0; }
uint64_t fox_context_weight_reads(const fox_context *c)
{
    return c ? fox_weights_reads(c->m->weights) : 0;
}

static int same_type(const fox_gpu_tensor *a, const fox_gpu_tensor *b)
{
    int ta, tb;
    uint64_t ka, kb;
    fox_gpu_tensor_info(a, &ta, &ka, NULL, NULL, NULL);
    fox_gpu_tensor_info(b, &tb, &kb, NULL, NULL, NULL);
    return ta == tb && ka == kb;
}

/* y_i = W_i x for matrices sharing the input: one launch for each run of
 * equal types (q/k/v, gate/up) */
static fox_status project_group(fox_context *c, size_t n, const fox_gpu_tensor *const *ws,
                                const float *x, size_t x_stride, size_t M, float *const *outs,
                                const size_t *strides)
{
    size_t i = 0;
    while (i < n) {
        size_t j = i + 1;
        while (j < n && same_type(ws[i], ws[j])) j++;
        GPU(fox_gpu_gemv_multi(c->gpu, j - i, ws + i, x, x_stride, M, outs + i, strides + i, 0),
            "forward: projection");
        i = j;
    }
    return FOX_OK;
}

/* one pass over all layers for M <= FOX_GPU_MAX_TOKENS tokens already in
 * dtok, at the position held in dpos; queued on the stream, no host sync.
 * want_logits: 0 none, 1 the last token's (dlogits row 0), 2 every token's
 * (dlogits rows 0 .. M-1) */
static fox_status forward_pass(fox_context *c, size_t M, int want_logits)
{
    const fox_model_info *mi = &c->m->info;
    const size_t kvl = (size_t)c->cfg.n_ctx * c->nkv;
    const size_t vl = FOX_GPU_V_CACHE_FLOATS(c->cfg.n_ctx, c->nkv);
    uint32_t l;
    fox_status st;
    fox_gpu_status gs;

    GPU(fox_gpu_get_rows(c->gpu, c->embd, c->dtok, M, c->x, c->d, NULL), "forward: embed");
    for (l = 0; l < mi->n_layer; l++) {
        dev_layer SD;
        const dev_layer *D = &c->L[l];
        if (streaming(c)) {
            /* this layer from its slot (loaded now if the prefetch did not
             * reach it); the compute stream waits for its upload */
            const fox_gpu_tensor *lt[FOX_LAYER_ROLES];
            if ((st = fox_weights_use_layer(c->m->weights, l, lt)) != FOX_OK) return st;
            SD = *D;
            SD.attn_q = lt[FOX_ROLE_ATTN_Q];
            SD.attn_k = lt[FOX_ROLE_ATTN_K];
            SD.attn_v = lt[FOX_ROLE_ATTN_V];
            SD.attn_out = lt[FOX_ROLE_ATTN_OUT];
            SD.ffn_gate = lt[FOX_ROLE_FFN_GATE];
            SD.ffn_up = lt[FOX_ROLE_FFN_UP];
            SD.ffn_down = lt[FOX_ROLE_FFN_DOWN];
            D = &SD;
        }
        const fox_gpu_tensor *qkv[3] = { D->attn_q, D->attn_k, D->attn_v };
        float *qkv_out[3] = { c->q, c->k, c->v };
        size_t qkv_str[3] = { c->nq, c->nkv, c->nkv };
        const fox_gpu_tensor *gu[2] = { D->ffn_gate, D->ffn_up };
        float *gu_out[2] = { c->hb, c->hb2 };
        size_t gu_str[2] = { c->ff, c->ff };

        /* ternary layers: norm, quantisation, q/k/v and RoPE + cache store in
         * one launch; other types (or activations too wide for one
         * workgroup) take the separate steps */
        gs = fox_gpu_qkv_rope(c->gpu, D->attn_q, D->attn_k, D->attn_v, c->x, c->d, M,
                              D->attn_norm, mi->rms_eps, c->q, c->nq, c->rc, c->rs, c->dpos,
                              c->cfg.n_ctx, c->kc + l * kvl, c->vc + l * vl, c->hd);
        if (gs == FOX_GPU_ERR_UNSUPPORTED) {
            GPU(fox_gpu_rmsnorm(c->gpu, c->xb, c->wide, c->x, c->d, D->attn_norm, c->d, M,
                                mi->rms_eps), "forward: attn_norm");
            if ((st = project_group(c, 3, qkv, c->xb, c->wide, M, qkv_out, qkv_str)) != FOX_OK)
                return st;
            GPU(fox_gpu_rope_store(c->gpu, c->q, c->nq, c->k, c->nkv, c->v, c->nkv, mi->n_head,
                                   mi->n_head_kv, c->hd, M, c->rc, c->rs, c->dpos, c->cfg.n_ctx,
                                   c->kc + l * kvl, c->vc + l * vl), "forward: rope");
        } else if (gs != FOX_GPU_OK) {
            return fox_gpu_failed(gs, "forward: q/k/v");
        }
        GPU(fox_gpu_attention(c->gpu, c->xb, c->wide, c->q, c->nq, c->kc + l * kvl,
                              c->vc + l * vl, mi->n_head, mi->n_head_kv, c->hd, M, c->dpos,
                              c->cfg.n_ctx, c->attn_mode), "forward: attention");
        GPU(fox_gpu_gemv(c->gpu, D->attn_out, c->xb, c->wide, M, c->x, c->d,
                         FOX_GPU_GEMV_ACCUMULATE), "forward: attn_output");
        gs = fox_gpu_gate_up_silu(c->gpu, D->ffn_gate, D->ffn_up, c->x, c->d, M, D->ffn_norm,
                                  mi->rms_eps, c->hb, c->ff);
        if (gs == FOX_GPU_ERR_UNSUPPORTED) {
            GPU(fox_gpu_rmsnorm(c->gpu, c->xb, c->wide, c->x, c->d, D->ffn_norm, c->d, M,
                                mi->rms_eps), "forward: ffn_norm");
            if ((st = project_group(c, 2, gu, c->xb, c->wide, M, gu_out, gu_str)) != FOX_OK)
                return st;
            GPU(fox_gpu_silu_mul(c->gpu, c->hb, c->hb2, c->ff, M, c->ff), "forward: swiglu");
        } else if (gs != FOX_GPU_OK) {
            return fox_gpu_failed(gs, "forward: gate/up");
        }
        GPU(fox_gpu_gemv(c->gpu, D->ffn_down, c->hb, c->ff, M, c->x, c->d,
                         FOX_GPU_GEMV_ACCUMULATE), "forward: ffn_down");
        if (streaming(c)) {
            /* the layer-ahead load (src/forward.c:333-337): the next layer,
             * or the first one of the next pass, goes up on the copy stream
             * while this one computes */
            fox_weights_done_layer(c->m->weights, l);
            if ((st = fox_weights_prefetch_layer(c->m->weights, (l + 1) % mi->n_layer)) != FOX_OK)
                return st;
        }
    }
    if (!want_logits) return FOX_OK;
    {
        /* src/forward.c:401-408 on the last row, or on every row: each row's
         * norm and head product are independent of the others */
        const size_t rows = want_logits == 2 ? M : 1;
        GPU(fox_gpu_rmsnorm(c->gpu, c->xb, c->wide, c->x + (M - rows) * c->d, c->d, c->out_norm,
                            c->d, rows, mi->rms_eps), "forward: output_norm");
        GPU(fox_gpu_gemv(c->gpu, c->out, c->xb, c->wide, rows, c->dlogits, c->vocab, 0),
            "forward: output");
    }
    return FOX_OK;
}

static fox_status check_tokens(const fox_context *c, const uint32_t *t, size_t n)
{
    size_t i;
    for (i = 0; i < n; i++)
        if (t[i] >= c->vocab)
            return fox_fail(FOX_ERR_ARG, "forward: token %u is outside the %zu entry vocabulary",
                            t[i], c->vocab);
    return FOX_OK;
}

/* tokens in chunks of at most n_batch (and FOX_GPU_MAX_TOKENS); all == NULL:
 * the last token's logits into c->logits, else every token's into all */
static fox_status eval_chunks(fox_context *c, const uint32_t *tokens, size_t n, float *all)
{
    size_t done = 0;
    double t0;
    fox_status st;

    t0 = now_s();
    c->reads_at_start = fox_weights_reads(c->m->weights);
    while (done < n) {
        size_t chunk = n - done, cap = c->cfg.n_batch;
        int last;
        if (cap > FOX_GPU_MAX_TOKENS) cap = FOX_GPU_MAX_TOKENS;
        if (chunk > cap) chunk = cap;
        last = done + chunk == n;
        if ((size_t)c->pos + chunk > c->cfg.n_ctx)
            return fox_fail(FOX_ERR_ARG, "forward: %zu tokens past position %u would overrun the "
                            "%u token context", chunk, c->pos, c->cfg.n_ctx);
        if ((st = check_tokens(c, tokens + done, chunk)) != FOX_OK) return st;
        GPU(fox_gpu_memcpy_h2d(c->gpu, c->dtok, tokens + done, chunk * 4), "eval: tokens");
        GPU(fox_gpu_memcpy_h2d(c->gpu, c->dpos, &c->pos, 4), "eval: position");
        if ((st = forward_pass(c, chunk, all ? 2 : last)) != FOX_OK) return st;
        if (all)
            GPU(fox_gpu_memcpy_d2h(c->gpu, all + done * c->vocab, c->dlogits,
                                   chunk * c->vocab * 4), "eval: logits");
        c->pos += (uint32_t)chunk;
        done += chunk;
    }
    if (!all) GPU(fox_gpu_memcpy_d2h(c->gpu, c->logits, c->dlogits, c->vocab * 4), "eval: logits");
    c->last_seconds = now_s() - t0;
    return FOX_OK;
}

fox_status fox_eval(fox_context *c, const uint32_t *tokens, size_t n, float **logits_out)
{
    fox_status st;
    if (!c || !tokens || n == 0) return fox_fail(FOX_ERR_ARG, "eval: nothing to evaluate");
    if ((st = eval_chunks(c, tokens, n, NULL)) != FOX_OK) return st;
    if (logits_out) *logits_out = c->logits;
    return FOX_OK;
}

fox_status fox_eval_all(fox_context *c, const uint32_t *tokens, size_t n, float *logits)
{
    if (!c || !tokens || n == 0 || !logits)
        return fox_fail(FOX_ERR_ARG, "eval_all: nothing to evaluate");
    return eval_chunks(c, tokens, n, logits);
}

/* one greedy step: forward at dpos with the token in dtok[0], then
 * dtok[0] = argmax, dhist[dpos] = argmax, dpos += 1 */
static fox_status greedy_step(fox_context *c)
{
    fox_status st = forward_pass(c, 1, 1);
    if (st != FOX_OK) return st;
    GPU(fox_gpu_argmax(c->gpu, c->dlogits, c->vocab, c->dtok, c->dpos, 1, c->dhist),
        "decode: argmax");
    return FOX_OK;
}

fox_status fox_decode_greedy(fox_context *c, uint32_t token, size_t n_steps, uint32_t *out_ids)
{
    double t0;
    size_t s;
    fox_status st;

    if (!c || (!out_ids && n_steps)) return fox_fail(FOX_ERR_ARG, "decode: null argument");
    if (n_steps == 0) return FOX_OK;
    if ((size_t)c->pos + n_steps > c->cfg.n_ctx)
        return fox_fail(FOX_ERR_ARG, "decode: %zu steps past position %u would overrun the %u "
                        "token context", n_steps, c->pos, c->cfg.n_ctx);
    if ((st = check_tokens(c, &token, 1)) != FOX_OK) return st;
    t0 = now_s();
    GPU(fox_gpu_memcpy_h2d(c->gpu, c->dtok, &token, 4), "decode: token");
    GPU(fox_gpu_memcpy_h2d(c->gpu, c->dpos, &c->pos, 4), "decode: position");
    /* the first step runs eagerly (it also sizes every workspace), the rest
     * replay one captured graph; FOX_GRAPHS=0 keeps every step eager (for
     * profilers that cannot follow graph launches), and so does streaming
     * (each step reloads layer slots from the host) */
    if ((st = greedy_step(c)) != FOX_OK) return st;
    {
        const char *e = getenv("FOX_GRAPHS");
        if ((e && strcmp(e, "0") == 0) || streaming(c)) {
            for (s = 1; s < n_steps; s++)
                if ((st = greedy_step(c)) != FOX_OK) return st;
            GPU(fox_gpu_memcpy_d2h(c->gpu, out_ids, c->dhist + c->pos, n_steps * 4), "decode: ids");
            c->pos += (uint32_t)n_steps;
            c->last_seconds = now_s() - t0;
            return FOX_OK;
        }
    }
    if (n_steps > 1 && !c->greedy) {
        GPU(fox_gpu_graph_begin(c->gpu), "decode: capture");
        st = greedy_step(c);
        {
            fox_gpu_status gs = fox_gpu_graph_end(c->gpu, &c->greedy);
            if (st != FOX_OK) return st;
            if (gs != FOX_GPU_OK) return fox_gpu_failed(gs, "decode: capture");
        }
    }
    for (s = 1; s < n_steps; s++) GPU(fox_gpu_graph_launch(c->gpu, c->greedy), "decode: replay");
    GPU(fox_gpu_memcpy_d2h(c->gpu, out_ids, c->dhist + c->pos, n_steps * 4), "decode: ids");
    c->pos += (uint32_t)n_steps;
    c->last_seconds = now_s() - t0;
    return FOX_OK;
}

fox_status fox_context_set_kv(fox_context *c, uint32_t layer, uint32_t p0, uint32_t n,
                              const float *k, const float *v)
{
    size_t bytes;
    float *tmp;
    fox_gpu_status gs;
    if (!c || !k || !v) return fox_fail(FOX_ERR_ARG, "set_kv: null argument");
    if (layer >= c->m->info.n_layer || (size_t)p0 + n > c->cfg.n_ctx)
        return fox_fail(FOX_ERR_ARG, "set_kv: rows %u..%u of layer %u are outside the cache",
                        p0, p0 + n, layer);
    if (n == 0) return FOX_OK;
    bytes = (size_t)n * c->nkv * 4;
    GPU(fox_gpu_malloc(c->gpu, 2 * bytes, (void **)&tmp), "set_kv: staging");
    gs = fox_gpu_memcpy_h2d(c->gpu, tmp, k, bytes);
    if (gs == FOX_GPU_OK) gs = fox_gpu_memcpy_h2d(c->gpu, tmp + (size_t)n * c->nkv, v, bytes);
    if (gs == FOX_GPU_OK)
        gs = fox_gpu_kv_write(c->gpu, c->kc + (size_t)layer * c->cfg.n_ctx * c->nkv,
                              c->vc + (size_t)layer * FOX_GPU_V_CACHE_FLOATS(c->cfg.n_ctx, c->nkv),
                              c->nkv, c->cfg.n_ctx, p0, n, tmp, tmp + (size_t)n * c->nkv);
    if (gs == FOX_GPU_OK) gs = fox_gpu_sync(c->gpu);
    fox_gpu_free(c->gpu, tmp);
    if (gs != FOX_GPU_OK) return fox_gpu_failed(gs, "set_kv");
    return FOX_OK;
}

fox_status fox_context_set_position(fox_context *c, uint32_t pos)
{
    if (!c) return fox_fail(FOX_ERR_ARG, "set_position: null context");
    if (pos > c->cfg.n_ctx) return fox_fail(FOX_ERR_ARG, "set_position: %u > n_ctx", pos);
    c->pos = pos;
    return FOX_OK;
}

fox_status fox_context_set_attention(fox_context *c, int exact)
{
    if (!c) return fox_fail(FOX_ERR_ARG, "set_attention: null context");
    c->attn_mode = exact ? FOX_GPU_ATTN_EXACT : FOX_GPU_ATTN_SPLIT;
    if (c->greedy) {
        fox_gpu_sync(c->gpu);
        fox_gpu_graph_free(c->greedy);
        c->greedy = NULL;
    }
    return FOX_OK;
}
