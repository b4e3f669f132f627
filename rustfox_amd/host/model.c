/* model.c -- llama-shaped model over the weights backend.
 *
 * Metadata keys and defaults follow RustFox src/model.c:146-303:
 * <arch>.block_count, embedding_length, attention.head_count and
 * feed_forward_length are required; head_count_kv defaults to head_count,
 * context_length to 2048, attention.key_length to n_embd / n_head,
 * layer_norm_rms_epsilon to 1e-5, rope.freq_base to 10000; the head
 * dimension must be even and the heads divide evenly over the kv heads;
 * output.weight falls back to token_embd.weight (tied).  Every tensor must
 * have a kernel (src/model.c:85-99), here a device kernel.
 */
#include "fox_host_internal.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static fox_status meta_u(const fox_gguf *g, const char *arch, const char *suffix,
                         uint64_t *out, uint64_t fallback, int required)
{
    char key[160];
    size_t idx;
    snprintf(key, sizeof(key), "%s.%s", arch, suffix);
    idx = fox_gguf_find(g, key);
    if (idx == FOX_TENSOR_ABSENT) {
        if (required) return fox_fail(FOX_ERR_NOTFOUND, "model: the file has no '%s' key", key);
        *out = fallback;
        return FOX_OK;
    }
    if (fox_gguf_get_uint(g, idx, out) != FOX_OK)
        return fox_fail(FOX_ERR_FORMAT, "model: '%s' holds no integer", key);
    return FOX_OK;
}

static void meta_f(const fox_gguf *g, const char *arch, const char *suffix, float *out,
                   float fallback)
{
    char key[160];
    size_t idx;
    snprintf(key, sizeof(key), "%s.%s", arch, suffix);
    idx = fox_gguf_find(g, key);
    if (idx == FOX_TENSOR_ABSENT || fox_gguf_get_f32(g, idx, out) != FOX_OK) *out = fallback;
}

static size_t need(const fox_gguf *g, const char *name, fox_status *st)
{
    size_t idx = fox_gguf_tensor_find(g, name);
    if (idx == FOX_TENSOR_ABSENT && *st == FOX_OK)
        *st = fox_fail(FOX_ERR_NOTFOUND, "model: the file has no tensor '%s'", name);
    return idx;
}

const char *fox_ggml_type_name(fox_ggml_type type)
{
    switch ((int)type) {
    case 0: return "F32";
    case 1: return "F16";
    case 2: return "Q4_0";
    case 3: return "Q4_1";
    case 6: return "Q5_0";
    case 7: return "Q5_1";
    case 8: return "Q8_0";
    case 10: return "Q2_K";
    case 11: return "Q3_K";
    case 12: return "Q4_K";
    case 13: return "Q5_K";
    case 14: return "Q6_K";
    case 15: return "Q8_K";
    case 30: return "BF16";
    case 34: return "TQ1_0";
    case 35: return "TQ2_0";
    default: return "unknown";
    }
}

uint32_t fox_ggml_type_block_size(fox_ggml_type type)
{
    uint32_t b, n;
    return fox_type_layout((uint32_t)type, &b, &n) ? b : 0;
}

uint32_t fox_ggml_type_block_bytes(fox_ggml_type type)
{
    uint32_t b, n;
    return fox_type_layout((uint32_t)type, &b, &n) ? n : 0;
}

int fox_gemv_supports(fox_ggml_type type)
{
    switch ((int)type) {
    case FOX_GGML_F32: case FOX_GGML_F16: case FOX_GGML_Q4_K: case FOX_GGML_Q6_K:
    case FOX_GGML_TQ1_0: case FOX_GGML_TQ2_0:
        return 1;
    default:
        return 0;
    }
}

size_t fox_row_bytes(fox_ggml_type type, size_t n_cols)
{
    uint32_t b, n;
    if (!fox_type_layout((uint32_t)type, &b, &n) || n_cols % b) return 0;
    return n_cols / b * n;
}

/* the llama metadata a model needs: key suffix, destination, default, and
 * whether the key must be present */
typedef struct {
    const char *key;
    uint32_t *dst;
    uint32_t fallback;
    int required;
} meta_want;

static fox_status read_shape(fox_model *m, const fox_gguf *g, const char *arch)
{
    fox_model_info *mi = &m->info;
    const meta_want want[] = {
        {"block_count", &mi->n_layer, 0, 1},
        {"embedding_length", &mi->n_embd, 0, 1},
        {"attention.head_count", &mi->n_head, 0, 1},
        {"feed_forward_length", &mi->n_ff, 0, 1},
        {"context_length", &mi->n_ctx_train, 2048, 0},
        {"attention.key_length", &mi->head_dim, 0, 0},
    };
    size_t k;
    uint64_t v;
    fox_status st;

    for (k = 0; k < sizeof(want) / sizeof(want[0]); k++) {
        if ((st = meta_u(g, arch, want[k].key, &v, want[k].fallback, want[k].required)))
            return st;
        *want[k].dst = (uint32_t)v;
    }
    /* the kv head count defaults to the query head count, read above */
    if ((st = meta_u(g, arch, "attention.head_count_kv", &v, mi->n_head, 0))) return st;
    mi->n_head_kv = (uint32_t)v;
    if (mi->n_layer == 0 || mi->n_embd == 0 || mi->n_head == 0 || mi->n_head_kv == 0 ||
        mi->n_ff == 0)
        return fox_fail(FOX_ERR_FORMAT, "model: %s metadata gives a zero layer, width, head or "
                        "feed-forward count", arch);
    if (mi->head_dim == 0) mi->head_dim = mi->n_embd / mi->n_head;
    if (mi->head_dim == 0 || (mi->head_dim & 1))
        return fox_fail(FOX_ERR_UNSUPPORTED, "model: RoPE rotates pairs of values; a head of %u "
                        "values has no such pairing", mi->head_dim);
    if (mi->n_head % mi->n_head_kv)
        return fox_fail(FOX_ERR_FORMAT, "model: grouped attention needs the %u query heads to "
                        "be a multiple of the %u key/value heads", mi->n_head, mi->n_head_kv);
    meta_f(g, arch, "attention.layer_norm_rms_epsilon", &mi->rms_eps, 1e-5f);
    meta_f(g, arch, "rope.freq_base", &mi->rope_freq_base, 10000.0f);
    return FOX_OK;
}

/* a tensor's columns (ne0) and rows (ne1; 0 for a vector) must be the
 * ones the forward pass sizes its buffers and caches by: the kernels read
 * and write as many as the tensor holds */
static fox_status check_dims(const fox_gguf *g, size_t idx, uint64_t cols, uint64_t rows)
{
    const fox_tensor_desc *t = &g->tensors[idx];
    uint64_t r = 1;
    uint32_t d;
    for (d = 1; d < t->n_dims; d++) r *= t->ne[d];
    if (t->ne[0] != cols || (rows ? r != rows : r != 1))
        return fox_fail(FOX_ERR_FORMAT, "model: tensor '%s' is %llu x %llu where the metadata "
                        "implies %llu x %llu", t->name, (unsigned long long)t->ne[0],
                        (unsigned long long)r, (unsigned long long)cols,
                        (unsigned long long)(rows ? rows : 1));
    return FOX_OK;
}

/* rows the device reads as floats (the embedding gather, norm vectors) */
static fox_status check_float(const fox_gguf *g, size_t idx)
{
    const fox_tensor_desc *t = &g->tensors[idx];
    if (t->type != FOX_GGML_F32 && t->type != FOX_GGML_F16)
        return fox_fail(FOX_ERR_UNSUPPORTED, "model: tensor '%s' is %s; the device path reads "
                        "embeddings and norm vectors as F16 or F32", t->name,
                        fox_ggml_type_name((fox_ggml_type)t->type));
    return FOX_OK;
}

static fox_status find_layers(fox_model *m, const fox_gguf *g)
{
    const fox_model_info *mi = &m->info;
    const uint64_t d = mi->n_embd, q = (uint64_t)mi->n_head * mi->head_dim,
                   kv = (uint64_t)mi->n_head_kv * mi->head_dim, ff = mi->n_ff;
    uint32_t l;
    fox_status st = FOX_OK;
    char name[FOX_NAME_MAX];

    m->layers = (fox_layer_tensors *)calloc(mi->n_layer, sizeof(*m->layers));
    if (!m->layers) return fox_fail(FOX_ERR_NOMEM, "model: table of %u layers", mi->n_layer);
    for (l = 0; l < mi->n_layer && st == FOX_OK; l++) {
        fox_layer_tensors *t = &m->layers[l];
        const struct {
            const char *suffix;
            size_t *slot;
            uint64_t cols, rows;
            int is_norm;
        } parts[] = {
            {"attn_norm", &t->attn_norm, d, 0, 1}, {"attn_q", &t->attn_q, d, q, 0},
            {"attn_k", &t->attn_k, d, kv, 0},      {"attn_v", &t->attn_v, d, kv, 0},
            {"attn_output", &t->attn_out, q, d, 0}, {"ffn_norm", &t->ffn_norm, d, 0, 1},
            {"ffn_gate", &t->ffn_gate, d, ff, 0},  {"ffn_up", &t->ffn_up, d, ff, 0},
            {"ffn_down", &t->ffn_down, ff, d, 0},
        };
        size_t k;
        for (k = 0; k < sizeof(parts) / sizeof(parts[0]) && st == FOX_OK; k++) {
            snprintf(name, sizeof(name), "blk.%u.%s.weight", l, parts[k].suffix);
            *parts[k].slot = need(g, name, &st);
            if (st == FOX_OK) st = check_dims(g, *parts[k].slot, parts[k].cols, parts[k].rows);
            if (st == FOX_OK && parts[k].is_norm) st = check_float(g, *parts[k].slot);
        }
    }
    return st;
}

fox_status fox_model_open(const char *gguf_path, fox_weights_mode mode,
                          uint64_t budget_bytes, fox_model **out)
{
    fox_model *m;
    const fox_gguf *g;
    const char *arch = "llama", *str;
    fox_status st;
    size_t i;

    if (!gguf_path || !out) return fox_fail(FOX_ERR_ARG, "model: a path and an output are needed");
    *out = NULL;
    m = (fox_model *)calloc(1, sizeof(*m));
    if (!m) return fox_fail(FOX_ERR_NOMEM, "model: no memory for the handle");
    m->token_embd = m->output_norm = m->output = FOX_TENSOR_ABSENT;
    if ((st = fox_weights_open(gguf_path, mode, budget_bytes, &m->weights)) != FOX_OK) {
        free(m);
        return st;
    }
    g = m->weights->g;

    i = fox_gguf_find(g, "general.architecture");
    if (i != FOX_TENSOR_ABSENT && fox_gguf_get_string(g, i, &str) == FOX_OK && str) arch = str;
    snprintf(m->info.arch, sizeof(m->info.arch), "%s", arch);
    str = NULL;
    i = fox_gguf_find(g, "general.name");
    if (i != FOX_TENSOR_ABSENT) fox_gguf_get_string(g, i, &str);
    snprintf(m->info.name, sizeof(m->info.name), "%s", str && *str ? str : "unnamed");

    if ((st = read_shape(m, g, arch)) != FOX_OK) goto fail;
    for (i = 0; i < g->n_tensors; i++) {
        if (!fox_gemv_supports((fox_ggml_type)g->tensors[i].type)) {
            st = fox_fail(FOX_ERR_UNSUPPORTED, "model: no device kernel reads %s, the type of "
                          "tensor '%s'", fox_ggml_type_name((fox_ggml_type)g->tensors[i].type),
                          g->tensors[i].name);
            goto fail;
        }
    }

    /* the embedding fixes the vocabulary; a missing output head is tied to it */
    m->token_embd = need(g, "token_embd.weight", &st);
    if (st == FOX_OK) m->output_norm = need(g, "output_norm.weight", &st);
    if (st != FOX_OK) goto fail;
    {
        const fox_tensor_desc *e = &g->tensors[m->token_embd];
        if (e->n_dims != 2 || e->ne[1] == 0 || e->ne[1] > 0xFFFFFFFFull) {
            st = fox_fail(FOX_ERR_FORMAT, "model: token_embd.weight must be a matrix of one "
                          "row per token");
            goto fail;
        }
        m->info.n_vocab = (uint32_t)e->ne[1];
    }
    m->output = fox_gguf_tensor_find(g, "output.weight");
    m->info.tied_output = m->output == FOX_TENSOR_ABSENT;
    if (m->info.tied_output) m->output = m->token_embd;
    if ((st = check_dims(g, m->token_embd, m->info.n_embd, m->info.n_vocab)) != FOX_OK ||
        (st = check_float(g, m->token_embd)) != FOX_OK ||
        (st = check_dims(g, m->output_norm, m->info.n_embd, 0)) != FOX_OK ||
        (st = check_float(g, m->output_norm)) != FOX_OK ||
        (st = check_dims(g, m->output, m->info.n_embd, m->info.n_vocab)) != FOX_OK)
        goto fail;
    if ((st = find_layers(m, g)) != FOX_OK) goto fail;

    if (strcmp(m->info.arch, "llama") != 0)
        fox_warn("model: '%s' is run with the llama layer structure", m->info.arch);
    for (i = 0; i < g->n_tensors; i++) m->info.weight_bytes += g->tensors[i].size_bytes;
    /* HBM residency: every tensor is read and uploaded once, before the
     * first evaluation */
    if (mode == FOX_WEIGHTS_DEVICE)
        for (i = 0; i < g->n_tensors && st == FOX_OK; i++) st = fox_weights_prefetch(m->weights, i);
    /* streaming: the tensors outside the layers stay resident from the start */
    if (mode == FOX_WEIGHTS_STREAM) {
        const size_t keep[3] = {m->token_embd, m->output_norm, m->output};
        for (i = 0; i < 3 && st == FOX_OK; i++) st = fox_weights_prefetch(m->weights, keep[i]);
    }
    if (st != FOX_OK) goto fail;
    *out = m;
    return FOX_OK;

fail:
    fox_model_close(m);
    return st;
}

void fox_model_close(fox_model *m)
{
    if (!m) return;
    free(m->layers);
    fox_weights_close(m->weights);
    free(m);
}

const fox_model_info *fox_model_get_info(const fox_model *m) { return m ? &m->info : NULL; }
fox_weights *fox_model_weights(fox_model *m) { return m ? m->weights : NULL; }
