/* sample.c -- token choice on the host (RustFox src/sample.c semantics).
 *
 * Greedy (temperature <= 0): repeat penalty over the last repeat_last_n
 * accepted tokens (a positive logit is divided, a non-positive one
 * multiplied), then the first index of the maximum (src/sample.c:135-153).
 * Otherwise: the top_k best logits in descending order (ties keep the lower
 * id first), softmax at the temperature, optional top_p cut and
 * renormalisation, and one uniform draw from xorshift64* (Marsaglia/Vigna:
 * shifts 12, 25, 27, multiplier 0x2545F4914F6CDD1D; the top 24 bits make a
 * float in [0, 1)) walked along the cumulative sum (src/sample.c:155-194).
 */
#include "fox_host_internal.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define TOPK_MAX 512

struct fox_sampler {
    fox_sampler_config cfg;
    size_t n_vocab;
    uint64_t rng;
    float *work;
    uint32_t *hist;
    size_t hist_cap, hist_len, hist_head;
};

void fox_sampler_config_default(fox_sampler_config *cfg)
{
    if (!cfg) return;
    cfg->temperature = 0.8f;
    cfg->top_k = 40;
    cfg->top_p = 0.95f;
    cfg->repeat_penalty = 1.1f;
    cfg->repeat_last_n = 64;
    cfg->seed = 0;
}

static uint64_t xs64(uint64_t *s)
{
    uint64_t x = *s;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *s = x;
    return x * 0x2545F4914F6CDD1Dull;
}

static float uniform01(uint64_t *s)
{
    return (float)((double)(xs64(s) >> 40) / 16777216.0);
}

fox_sampler *fox_sampler_create(const fox_sampler_config *cfg, size_t n_vocab)
{
    fox_sampler *s;
    if (n_vocab == 0) { fox_fail(FOX_ERR_ARG, "sampler: empty vocabulary"); return NULL; }
    s = (fox_sampler *)calloc(1, sizeof(*s));
    if (!s) { fox_fail(FOX_ERR_NOMEM, "sampler: handle"); return NULL; }
    if (cfg) s->cfg = *cfg;
    else fox_sampler_config_default(&s->cfg);
    if (s->cfg.top_k < 0) s->cfg.top_k = 0;
    if (s->cfg.top_k > TOPK_MAX) s->cfg.top_k = TOPK_MAX;
    if (s->cfg.top_p <= 0.0f || s->cfg.top_p > 1.0f) s->cfg.top_p = 1.0f;
    if (s->cfg.repeat_penalty < 1.0f) s->cfg.repeat_penalty = 1.0f;
    s->n_vocab = n_vocab;
    s->rng = s->cfg.seed ? s->cfg.seed : 0x9E3779B97F4A7C15ull;
    s->hist_cap = s->cfg.repeat_last_n ? s->cfg.repeat_last_n : 1;
    s->work = (float *)calloc(n_vocab, sizeof(float));
    s->hist = (uint32_t *)calloc(s->hist_cap, sizeof(uint32_t));
    if (!s->work || !s->hist) {
        fox_sampler_destroy(s);
        fox_fail(FOX_ERR_NOMEM, "sampler: buffers");
        return NULL;
    }
    return s;
}

void fox_sampler_destroy(fox_sampler *s)
{
    if (!s) return;
    free(s->work);
    free(s->hist);
    free(s);
}

void fox_sampler_accept(fox_sampler *s, uint32_t token)
{
    if (!s) return;
    s->hist[s->hist_head] = token;
    s->hist_head = (s->hist_head + 1) % s->hist_cap;
    if (s->hist_len < s->hist_cap) s->hist_len++;
}

typedef struct { float v; uint32_t id; } cand;

fox_status fox_sampler_pick(fox_sampler *s, const float *logits, uint32_t *out)
{
    cand top[TOPK_MAX];
    size_t i, n = 0, k;
    float mx, sum, cum, r;

    if (!s || !logits || !out) return FOX_ERR_ARG;
    memcpy(s->work, logits, s->n_vocab * sizeof(float));
    if (s->cfg.repeat_penalty > 1.0f) {
        for (i = 0; i < s->hist_len; i++) {
            uint32_t t = s->hist[i];
            if (t >= s->n_vocab) continue;
            if (s->work[t] > 0.0f) s->work[t] /= s->cfg.repeat_penalty;
            else s->work[t] *= s->cfg.repeat_penalty;
        }
    }
    if (s->cfg.temperature <= 0.0f) {
        size_t best = 0;
        for (i = 1; i < s->n_vocab; i++) if (s->work[i] > s->work[best]) best = i;
        *out = (uint32_t)best;
        return FOX_OK;
    }

    k = (s->cfg.top_k > 0 && (size_t)s->cfg.top_k <= s->n_vocab) ? (size_t)s->cfg.top_k
        : (s->n_vocab < TOPK_MAX ? s->n_vocab : TOPK_MAX);
    for (i = 0; i < s->n_vocab; i++) {
        float v = s->work[i];
        size_t j;
        if (n < k) {
            j = n++;
        } else {
            if (v <= top[n - 1].v) continue;
            j = n - 1;
        }
        while (j > 0 && top[j - 1].v < v) { top[j] = top[j - 1]; j--; }
        top[j].v = v;
        top[j].id = (uint32_t)i;
    }
    if (n == 0) return fox_fail(FOX_ERR_INTERNAL, "sampler: no candidates");

    mx = top[0].v;
    sum = 0.0f;
    for (i = 0; i < n; i++) {
        top[i].v = expf((top[i].v - mx) / s->cfg.temperature);
        sum += top[i].v;
    }
    if (!(sum > 0.0f)) { *out = top[0].id; return FOX_OK; }
    for (i = 0; i < n; i++) top[i].v /= sum;
    if (s->cfg.top_p < 1.0f) {
        cum = 0.0f;
        for (i = 0; i < n; i++) {
            cum += top[i].v;
            if (cum >= s->cfg.top_p) { n = i + 1; break; }
        }
        sum = 0.0f;
        for (i = 0; i < n; i++) sum += top[i].v;
        if (sum > 0.0f) for (i = 0; i < n; i++) top[i].v /= sum;
    }
    r = uniform01(&s->rng);
    cum = 0.0f;
    for (i = 0; i < n; i++) {
        cum += top[i].v;
        if (r <= cum) { *out = top[i].id; return FOX_OK; }
    }
    *out = top[n - 1].id;
    return FOX_OK;
}
