/* sample.c -- the greedy token choice of fox_sampler_pick.
 *
 * In scope is greedy decoding (temperature <= 0): each logit of a token
 * accepted k times among the last W accepted tokens (W = repeat_last_n, or
 * 1 when that is 0) is penalised k times -- divided by repeat_penalty while
 * positive, else multiplied -- and the pick is the lowest index holding the
 * largest penalised value (src/sample.c:95-107, 135-153).  A penalty at or
 * below 1.0 leaves the logits as they are.
 *
 * The handle keeps, per vocabulary entry, how often it occurs in the
 * window, and the window's ids in arrival order so that the oldest one can
 * be retired; a pick scans the logits once, penalising only counted ids on
 * the fly, without copying them.
 *
 * Stochastic sampling (temperature > 0: top-k, top-p, a seeded draw) is not
 * part of the decode path this library provides: such a pick fails with
 * FOX_ERR_UNSUPPORTED.  The configuration's defaults are the reference's
 * (include/fox/fox.h:453-469), so that a caller's configuration code is
 * unchanged.
 */
#include "fox_host_internal.h"

#include <stdlib.h>
#include <string.h>

struct fox_sampler {
    float penalty;        /* > 1.0f, or 1.0f for none */
    int greedy;
    size_t vocab;
    uint32_t *count;      /* occurrences of each id in the window */
    uint32_t *window;     /* ids, oldest at window[first] */
    size_t cap, used, first;
};

void fox_sampler_config_default(fox_sampler_config *cfg)
{
    if (!cfg) return;
    memset(cfg, 0, sizeof(*cfg));
    cfg->temperature = 0.8f;
    cfg->top_k = 40;
    cfg->top_p = 0.95f;
    cfg->repeat_penalty = 1.1f;
    cfg->repeat_last_n = 64;
}

fox_sampler *fox_sampler_create(const fox_sampler_config *cfg, size_t n_vocab)
{
    fox_sampler_config c;
    fox_sampler *s;

    if (n_vocab == 0) {
        fox_fail(FOX_ERR_ARG, "sampler: the vocabulary has no entries");
        return NULL;
    }
    if (cfg) c = *cfg;
    else fox_sampler_config_default(&c);
    s = (fox_sampler *)calloc(1, sizeof(*s));
    if (s) {
        s->vocab = n_vocab;
        s->greedy = !(c.temperature > 0.0f);
        s->penalty = c.repeat_penalty > 1.0f ? c.repeat_penalty : 1.0f;
        s->cap = c.repeat_last_n ? c.repeat_last_n : 1;
        s->count = (uint32_t *)calloc(n_vocab, sizeof(uint32_t));
        s->window = (uint32_t *)calloc(s->cap, sizeof(uint32_t));
    }
    if (!s || !s->count || !s->window) {
        fox_sampler_destroy(s);
        fox_fail(FOX_ERR_NOMEM, "sampler: cannot allocate its %zu-entry tables", n_vocab);
        return NULL;
    }
    return s;
}

void fox_sampler_destroy(fox_sampler *s)
{
    if (!s) return;
    free(s->count);
    free(s->window);
    free(s);
}

void fox_sampler_accept(fox_sampler *s, uint32_t token)
{
    size_t slot;
    if (!s) return;
    if (s->used == s->cap) {               /* the oldest id leaves the window */
        uint32_t old = s->window[s->first];
        if (old < s->vocab) s->count[old]--;
        s->first = (s->first + 1) % s->cap;
        s->used--;
    }
    slot = (s->first + s->used) % s->cap;
    s->window[slot] = token;
    s->used++;
    if (token < s->vocab) s->count[token]++;
}

/* x penalised k times: each application rounds, as the reference's
 * repeated in-place update does */
static float penalised(float x, uint32_t k, float p)
{
    while (k--) x = x > 0.0f ? x / p : x * p;
    return x;
}

fox_status fox_sampler_pick(fox_sampler *s, const float *logits, uint32_t *out)
{
    size_t i, best = 0;
    float top;

    if (!s || !logits || !out) return FOX_ERR_ARG;
    if (!s->greedy)
        return fox_fail(FOX_ERR_UNSUPPORTED, "sampler: this library decodes greedily; set "
                        "temperature <= 0 (stochastic sampling is not provided)");
    top = s->penalty > 1.0f && s->count[0] ? penalised(logits[0], s->count[0], s->penalty)
                                           : logits[0];
    for (i = 1; i < s->vocab; i++) {
        float v = logits[i];
        if (s->penalty > 1.0f && s->count[i]) v = penalised(v, s->count[i], s->penalty);
        if (v > top) {                     /* strict: the first maximum stays */
            top = v;
            best = i;
        }
    }
    *out = (uint32_t)best;
    return FOX_OK;
}
