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
        if (required) return fox_fail(FOX_ERR_NOTFOUND, "model: '%s' is missing", key);
        *out = fallback;
        return FOX_OK;
    }
    if (fox_gguf_get_uint(g, idx, out) != FOX_OK)
        return fox_fail(FOX_ERR_FORMAT, "model: '%s' is not an integer", key);
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
        *st = fox_fail(FOX_ERR_NOTFOUND, "model: tensor '%s' is missing", name);
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

fox_status fox_model_open(const char *gguf_path, fox_weights_mode mode,
                          uint64_t budget_bytes, fox_model **out)
{
    fox_model *m;
    const fox_gguf *g;
    const char *arch = "llama";
    fox_status st;
    uint64_t v;
    size_t idx, i;
    uint32_t l;
    char name[FOX_NAME_MAX];

    if (!gguf_path || !out) return fox_fail(FOX_ERR_ARG, "model: null argument");
    *out = NULL;
    m = (fox_model *)calloc(1, sizeof(*m));
    if (!m) return fox_fail(FOX_ERR_NOMEM, "model: handle");
    m->token_embd = m->output_norm = m->output = FOX_TENSOR_ABSENT;

    st = fox_weights_open(gguf_path, mode, budget_bytes, &m->weights);
    if (st != FOX_OK) { free(m); return st; }
    g = m->weights->g;

    idx = fox_gguf_find(g, "general.architecture");
    if (idx != FOX_TENSOR_ABSENT) {
        const char *s = NULL;
        if (fox_gguf_get_string(g, idx, &s) == FOX_OK && s) arch = s;
    }
    snprintf(m->info.arch, sizeof(m->info.arch), "%s", arch);
    idx = fox_gguf_find(g, "general.name");
    if (idx != FOX_TENSOR_ABSENT) {
        const char *s = NULL;
        if (fox_gguf_get_string(g, idx, &s) == FOX_OK && s)
            snprintf(m->info.name, sizeof(m->info.name), "%s", s);
    }
    if (!m->info.name[0]) snprintf(m->info.name, sizeof(m->info.name), "unnamed");

    if ((st = meta_u(g, arch, "block_count", &v, 0, 1))) goto fail;
    m->info.n_layer = (uint32_t)v;
    if ((st = meta_u(g, arch, "embedding_length", &v, 0, 1))) goto fail;
    m->info.n_embd = (uint32_t)v;
    if ((st = meta_u(g, arch, "attention.head_count", &v, 0, 1))) goto fail;
    m->info.n_head = (uint32_t)v;
    if ((st = meta_u(g, arch, "attention.head_count_kv", &v, m->info.n_head, 0))) goto fail;
    m->info.n_head_kv = (uint32_t)v;
    if ((st = meta_u(g, arch, "feed_forward_length", &v, 0, 1))) goto fail;
    m->info.n_ff = (uint32_t)v;
    if ((st = meta_u(g, arch, "context_length", &v, 2048, 0))) goto fail;
    m->info.n_ctx_train = (uint32_t)v;
    if ((st = meta_u(g, arch, "attention.key_length", &v, 0, 0))) goto fail;
    m->info.head_dim = (uint32_t)v;

    if (!m->info.n_layer || !m->info.n_embd || !m->info.n_head || !m->info.n_ff ||
        !m->info.n_head_kv) {
        st = fox_fail(FOX_ERR_FORMAT, "model: architecture metadata is incomplete");
        goto fail;
    }
    if (!m->info.head_dim) m->info.head_dim = m->info.n_embd / m->info.n_head;
    if (!m->info.head_dim || m->info.head_dim % 2) {
        st = fox_fail(FOX_ERR_UNSUPPORTED, "model: head dimension %u is not usable by rope on "
                      "adjacent pairs", m->info.head_dim);
        goto fail;
    }
    if (m->info.n_head % m->info.n_head_kv) {
        st = fox_fail(FOX_ERR_FORMAT, "model: %u query heads do not divide evenly into %u kv "
                      "heads", m->info.n_head, m->info.n_head_kv);
        goto fail;
    }
    meta_f(g, arch, "attention.layer_norm_rms_epsilon", &m->info.rms_eps, 1e-5f);
    meta_f(g, arch, "rope.freq_base", &m->info.rope_freq_base, 10000.0f);

    for (i = 0; i < g->n_tensors; i++) {
        if (!fox_gemv_supports((fox_ggml_type)g->tensors[i].type)) {
            st = fox_fail(FOX_ERR_UNSUPPORTED, "model: tensor '%s' is %s and rustfox_amd has no "
                          "device kernel for it", g->tensors[i].name,
                          fox_ggml_type_name((fox_ggml_type)g->tensors[i].type));
            goto fail;
        }
    }

    st = FOX_OK;
    m->token_embd = need(g, "token_embd.weight", &st);
    m->output_norm = need(g, "output_norm.weight", &st);
    if (st != FOX_OK) goto fail;
    m->output = fox_gguf_tensor_find(g, "output.weight");
    if (m->output == FOX_TENSOR_ABSENT) {
        m->output = m->token_embd;
        m->info.tied_output = 1;
    }
    {
        const fox_tensor_desc *t = &g->tensors[m->token_embd];
        if (t->n_dims < 2) {
            st = fox_fail(FOX_ERR_FORMAT, "model: token_embd.weight is malformed");
            goto fail;
        }
        m->info.n_vocab = (uint32_t)t->ne[1];
        if (t->ne[0] != m->info.n_embd) {
            st = fox_fail(FOX_ERR_FORMAT, "model: token_embd rows are %llu wide but the model "
                          "says the embedding is %u", (unsigned long long)t->ne[0],
                          m->info.n_embd);
            goto fail;
        }
    }

    m->layers = (fox_layer_tensors *)calloc(m->info.n_layer, sizeof(*m->layers));
    if (!m->layers) { st = fox_fail(FOX_ERR_NOMEM, "model: layer table"); goto fail; }
    for (l = 0; l < m->info.n_layer && st == FOX_OK; l++) {
        fox_layer_tensors *t = &m->layers[l];
#define LAYER_T(field, suffix) \
        snprintf(name, sizeof(name), "blk.%u." suffix, l); \
        t->field = need(g, name, &st);
        LAYER_T(attn_norm, "attn_norm.weight")
        LAYER_T(attn_q, "attn_q.weight")
        LAYER_T(attn_k, "attn_k.weight")
        LAYER_T(attn_v, "attn_v.weight")
        LAYER_T(attn_out, "attn_output.weight")
        LAYER_T(ffn_norm, "ffn_norm.weight")
        LAYER_T(ffn_gate, "ffn_gate.weight")
        LAYER_T(ffn_up, "ffn_up.weight")
        LAYER_T(ffn_down, "ffn_down.weight")
#undef LAYER_T
    }
    if (st != FOX_OK) goto fail;
    if (strcmp(m->info.arch, "llama") != 0)
        fox_warn("model: architecture is '%s'; the forward pass implements the llama shape",
                 m->info.arch);
    for (i = 0; i < g->n_tensors; i++) m->info.weight_bytes += g->tensors[i].size_bytes;

    /* HBM residency: every tensor read and uploaded once, up front */
    if (mode == FOX_WEIGHTS_DEVICE) {
        for (i = 0; i < g->n_tensors; i++) {
            st = fox_weights_prefetch(m->weights, i);
            if (st != FOX_OK) goto fail;
        }
    }
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
