/*
 * fox_oracle.c -- CPU restatement of RustFox's decode path (test oracle only).
 * See fox_oracle.h for scope, provenance and how each part is pinned.
 * Citations are file:line into the RustFox sources.
 */
#include "fox_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ f16 */

/* src/kernels.c:14-39: exact widening, subnormals renormalised, inf/nan kept */
float or_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    uint32_t bits;
    float f;

    if (e == 0x1F) {
        bits = sign | 0x7F800000u | (m << 13);
    } else if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            int shift = 0;
            while (!(m & 0x400u)) { m <<= 1; shift++; }
            m &= 0x3FFu;
            bits = sign | ((uint32_t)(113 - shift) << 23) | (m << 13);
        }
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    memcpy(&f, &bits, 4);
    return f;
}

/* src/kernels.c:41-74: round half up on the dropped mantissa bits in the
 * normal range, truncating shift with a half-bias for subnormals */
uint16_t or_f32_to_f16(float f)
{
    uint32_t u, sign, mant;
    int exp;

    memcpy(&u, &f, 4);
    sign = (u >> 16) & 0x8000u;
    mant = u & 0x7FFFFFu;
    if (((u >> 23) & 0xFFu) == 0xFFu)
        return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0u));
    exp = (int)((u >> 23) & 0xFFu) - 112;
    if (exp >= 31) return (uint16_t)(sign | 0x7C00u);
    if (exp <= 0) {
        int shift;
        if (exp < -10) return (uint16_t)sign;
        shift = 14 - exp;
        mant |= 0x800000u;
        return (uint16_t)(sign | ((mant + (1u << (shift - 1))) >> shift));
    }
    return (uint16_t)(sign | (((uint32_t)exp << 10) +
                              ((mant + 0x0FFFu + ((mant >> 13) & 1u)) >> 13)));
}

static float half_at(const uint8_t *p)
{
    return or_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
}

/* --------------------------------------------------------- block table */

/* src/gguf.c:160-195 (the subset on the path) */
size_t or_block_elems(int type)
{
    switch (type) {
    case OR_F32: case OR_F16: return 1;
    case OR_Q4_0: case OR_Q8_0: return 32;
    case OR_Q4_K: case OR_Q5_K: case OR_Q6_K: case OR_TQ1_0: case OR_TQ2_0: return 256;
    default: return 0;
    }
}

size_t or_block_bytes(int type)
{
    switch (type) {
    case OR_F32: return 4;
    case OR_F16: return 2;
    case OR_Q4_0: return 18;
    case OR_Q8_0: return 34;
    case OR_Q4_K: return 144;
    case OR_Q5_K: return 176;
    case OR_Q6_K: return 210;
    case OR_TQ1_0: return 54;
    case OR_TQ2_0: return 66;
    default: return 0;
    }
}

/* src/kernels.c:690-698 */
size_t or_row_bytes(int type, size_t n_cols)
{
    size_t be = or_block_elems(type), bb = or_block_bytes(type);
    if (!be || !bb || n_cols % be) return 0;
    return n_cols / be * bb;
}

/* ---------------------------------------------------- activation quant */

/* One scale over n values: amax by strict '>' (NaN never wins), q rounded
 * half away from zero by truncating v +/- 0.5f, clamped to +/-127.
 * Shared by src/gemv.c:11-42 (whole vector) and src/kernels.c:722-754
 * (per 256-element block). */
static float quantize_run(const float *x, size_t n, int8_t *q)
{
    float amax = 0.0f, inv;
    size_t i;

    for (i = 0; i < n; i++) {
        float a = fabsf(x[i]);
        if (a > amax) amax = a;
    }
    if (!(amax > 0.0f)) {
        memset(q, 0, n);
        return 0.0f;
    }
    inv = 127.0f / amax;
    for (i = 0; i < n; i++) {
        float v = x[i] * inv;
        float t = v < 0.0f ? v - 0.5f : v + 0.5f;
        int r = (int)t;
        q[i] = (int8_t)(r > 127 ? 127 : r < -127 ? -127 : r);
    }
    return amax / 127.0f;
}

/* src/gemv.c:11-42 */
int or_quantize_act_i8(const float *x, size_t n, int8_t *q, float *scale)
{
    if (!x || !q || !scale || n == 0) return OR_ERR_ARG;
    *scale = quantize_run(x, n, q);
    return OR_OK;
}

/* src/kernels.c:722-754 */
void or_quantize_act_k(const float *x, size_t n, int8_t *q, float *scales)
{
    size_t b;
    for (b = 0; b < n / 256; b++)
        scales[b] = quantize_run(x + b * 256, 256, q + b * 256);
}

/* ---------------------------------------------------------- block sums */

/* src/ternary.c:59-63: trit at base-3 level l of a TQ1_0 byte */
static int tq1_trit(uint8_t code, int level)
{
    static const uint8_t p3[5] = { 1, 3, 9, 27, 81 };
    uint8_t scaled = (uint8_t)(code * p3[level]);
    return (int)(((unsigned)scaled * 3u) >> 8) - 1;
}

/* src/ternary.c:73-93 (element order; the SSE2 path in ternary.c:97-173
 * computes the same integer) */
int32_t or_tq1_block_sum(const int8_t *x, const uint8_t *blk)
{
    int32_t s = 0;
    int l, m;

    for (l = 0; l < 5; l++)
        for (m = 0; m < 32; m++) s += tq1_trit(blk[m], l) * x[l * 32 + m];
    for (l = 0; l < 5; l++)
        for (m = 0; m < 16; m++) s += tq1_trit(blk[32 + m], l) * x[160 + l * 16 + m];
    for (l = 0; l < 4; l++)
        for (m = 0; m < 4; m++) s += tq1_trit(blk[48 + m], l) * x[240 + l * 4 + m];
    return s;
}

/* src/ternary.c:177-188: code 3 decodes to +2 and is not clamped */
int32_t or_tq2_block_sum(const int8_t *x, const uint8_t *blk)
{
    int32_t s = 0;
    int half, l, m;

    for (half = 0; half < 2; half++)
        for (l = 0; l < 4; l++)
            for (m = 0; m < 32; m++) {
                int code = (blk[half * 32 + m] >> (2 * l)) & 3;
                s += (code - 1) * x[half * 128 + l * 32 + m];
            }
    return s;
}

/* src/kernels.c:246-255: 6-bit scale and min of sub-block j */
static void q4k_scale_min(const uint8_t *s, int j, int *sc, int *mn)
{
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* src/kernels.c:571-602 with kernel_dot_u4_i8 / kernel_sum_i8 (450-500):
 * sub-block j = 2p (low nibbles of qs[32p..32p+31]) and 2p+1 (high nibbles)
 * against x[64p .. 64p+31] and x[64p+32 .. 64p+63] */
void or_q4k_block_sums(const int8_t *x, const uint8_t *blk,
                       int32_t dots[8], int32_t sums[8])
{
    const uint8_t *qs = blk + 16;
    int p, l;

    for (p = 0; p < 4; p++) {
        int32_t dlo = 0, dhi = 0, slo = 0, shi = 0;
        for (l = 0; l < 32; l++) {
            int8_t a = x[64 * p + l], c = x[64 * p + 32 + l];
            dlo += (qs[32 * p + l] & 0x0F) * a;
            dhi += (qs[32 * p + l] >> 4) * c;
            slo += a;
            shi += c;
        }
        dots[2 * p] = dlo;  dots[2 * p + 1] = dhi;
        sums[2 * p] = slo;  sums[2 * p + 1] = shi;
    }
}

/* src/kernels.c:531-569 and 636-661: for half h and sub s, the integer
 * G = sum_g sc[8h + s + 2g] * sum_{l<16} (q6 - 32) * x[128h + 32g + 16s + l] */
void or_q6k_block_sums(const int8_t *x, const uint8_t *blk, int32_t g[4])
{
    int h, s, grp, l;

    for (h = 0; h < 2; h++) {
        const uint8_t *ql = blk + 64 * h;
        const uint8_t *qh = blk + 128 + 32 * h;
        const int8_t *sc = (const int8_t *)(blk + 192) + 8 * h;
        for (s = 0; s < 2; s++) {
            int32_t total = 0;
            for (grp = 0; grp < 4; grp++) {
                int32_t d = 0;
                for (l = 16 * s; l < 16 * s + 16; l++) {
                    int lo = grp & 1 ? ql[l + 32] : ql[l];
                    int nib = grp < 2 ? lo & 0x0F : lo >> 4;
                    int hi = (qh[l] >> (2 * grp)) & 3;
                    d += ((nib | (hi << 4)) - 32) * x[128 * h + 32 * grp + l];
                }
                total += sc[s + 2 * grp] * d;
            }
            g[2 * h + s] = total;
        }
    }
}

int or_block_sums(int type, const int8_t *q, const void *w, size_t rows,
                  size_t cols, int32_t *out)
{
    size_t rb = or_row_bytes(type, cols), nb = cols / 256, r, b;
    const uint8_t *wb = (const uint8_t *)w;

    if (!rb || !q || !w || !out) return OR_ERR_ARG;
    for (r = 0; r < rows; r++) {
        for (b = 0; b < nb; b++) {
            const uint8_t *blk = wb + r * rb + b * or_block_bytes(type);
            const int8_t *xb = q + b * 256;
            switch (type) {
            case OR_TQ1_0: out[r * nb + b] = or_tq1_block_sum(xb, blk); break;
            case OR_TQ2_0: out[r * nb + b] = or_tq2_block_sum(xb, blk); break;
            case OR_Q4_K: {
                int32_t d[8], s[8];
                or_q4k_block_sums(xb, blk, d, s);
                memcpy(out + (r * nb + b) * 8, d, sizeof(d));
                break;
            }
            case OR_Q6_K: or_q6k_block_sums(xb, blk, out + (r * nb + b) * 4); break;
            default: return OR_ERR_UNSUPPORTED;
            }
        }
    }
    return OR_OK;
}

/* ---------------------------------------------------------- row dots */

/* src/ternary.c:226-246 / 303-325 and src/gemv.c:62-70: acc starts at 0.0f and adds
 * f16(d) * (float)S block by block (two roundings per block) */
static float tq_row(int type, const int8_t *q, const uint8_t *row, size_t cols)
{
    size_t nb = cols / 256, b, bb = or_block_bytes(type);
    float acc = 0.0f;

    for (b = 0; b < nb; b++) {
        const uint8_t *blk = row + b * bb;
        int32_t s = type == OR_TQ1_0 ? or_tq1_block_sum(q + b * 256, blk)
                                     : or_tq2_block_sum(q + b * 256, blk);
        float p = half_at(blk + bb - 2) * (float)s;
        acc = acc + p;
    }
    return acc;
}

/* src/kernels.c:571-602 float combine, evaluated left to right */
static float q4k_row(const uint8_t *row, const int8_t *q, size_t cols,
                     const float *ascale)
{
    size_t nb = cols / 256, b;
    float sum = 0.0f;

    for (b = 0; b < nb; b++) {
        const uint8_t *blk = row + b * 144;
        float d = half_at(blk), dmin = half_at(blk + 2);
        int32_t dots[8], sums[8];
        int j;
        or_q4k_block_sums(q + b * 256, blk, dots, sums);
        for (j = 0; j < 8; j++) {
            int sc, mn;
            float t;
            q4k_scale_min(blk + 4, j, &sc, &mn);
            t = d * (float)sc * (float)dots[j] - dmin * (float)mn * (float)sums[j];
            sum = sum + ascale[b] * t;
        }
    }
    return sum;
}

/* src/kernels.c:636-661: sum += (ascale * d) * (float)G, half 0 sub 0..1,
 * then half 1 */
static float q6k_row(const uint8_t *row, const int8_t *q, size_t cols,
                     const float *ascale)
{
    size_t nb = cols / 256, b;
    float sum = 0.0f;

    for (b = 0; b < nb; b++) {
        const uint8_t *blk = row + b * 210;
        float d = half_at(blk + 208);
        int32_t g[4];
        int k;
        or_q6k_block_sums(q + b * 256, blk, g);
        for (k = 0; k < 4; k++) sum = sum + ascale[b] * d * (float)g[k];
    }
    return sum;
}

/* src/kernels.c:81-96: sequential f32 sum of products */
static float float_row(int type, const uint8_t *row, const float *x, size_t n)
{
    float sum = 0.0f;
    size_t i;
    if (type == OR_F32) {
        for (i = 0; i < n; i++) {
            float w;
            memcpy(&w, row + 4 * i, 4);
            sum = sum + w * x[i];
        }
    } else {
        for (i = 0; i < n; i++) sum = sum + half_at(row + 2 * i) * x[i];
    }
    return sum;
}

/* -------------------------------------------------------- parallel rows */

/* src/threadpool.c:29-40: static contiguous split, the first n % T
 * workers take one extra item; worker 0 runs on the calling thread */
typedef struct {
    void (*fn)(void *ctx, size_t begin, size_t end);
    void *ctx;
    size_t begin, end;
} or_slice;

static void *slice_main(void *p)
{
    or_slice *s = (or_slice *)p;
    if (s->end > s->begin) s->fn(s->ctx, s->begin, s->end);
    return NULL;
}

static void parallel_rows(size_t n, int n_threads,
                          void (*fn)(void *, size_t, size_t), void *ctx)
{
    or_slice sl[256];
    pthread_t th[256];
    size_t per, rem, t, at = 0;

    if (n_threads < 1) n_threads = 1;
    if (n_threads > 256) n_threads = 256;
    if (n_threads == 1) { fn(ctx, 0, n); return; }
    per = n / (size_t)n_threads;
    rem = n % (size_t)n_threads;
    for (t = 0; t < (size_t)n_threads; t++) {
        size_t cnt = per + (t < rem ? 1 : 0);
        sl[t].fn = fn; sl[t].ctx = ctx; sl[t].begin = at; sl[t].end = at + cnt;
        at += cnt;
    }
    for (t = 1; t < (size_t)n_threads; t++)
        pthread_create(&th[t], NULL, slice_main, &sl[t]);
    slice_main(&sl[0]);
    for (t = 1; t < (size_t)n_threads; t++) pthread_join(th[t], NULL);
}

typedef struct {
    int type;
    const uint8_t *w;
    size_t rb, cols;
    const int8_t *q;
    const float *ascale;
    float act_scale;
    const float *x;
    float *out;
} gemv_job;

static void gemv_slice(void *vj, size_t begin, size_t end)
{
    gemv_job *j = (gemv_job *)vj;
    size_t r;
    for (r = begin; r < end; r++) {
        const uint8_t *row = j->w + r * j->rb;
        switch (j->type) {
        case OR_TQ1_0: case OR_TQ2_0:
            /* src/gemv.c:54-72 */
            j->out[r] = tq_row(j->type, j->q, row, j->cols) * j->act_scale;
            break;
        case OR_Q4_K: j->out[r] = q4k_row(row, j->q, j->cols, j->ascale); break;
        case OR_Q6_K: j->out[r] = q6k_row(row, j->q, j->cols, j->ascale); break;
        default: j->out[r] = float_row(j->type, row, j->x, j->cols); break;
        }
    }
}

/* src/gemv.c:74-111 */
int or_gemv_tq_i8(int type, const int8_t *q, float act_scale, const void *w,
                  size_t rows, size_t cols, float *out)
{
    gemv_job j;
    if (!q || !w || !out || rows == 0 || cols == 0) return OR_ERR_ARG;
    if (cols % 256 || (type != OR_TQ1_0 && type != OR_TQ2_0)) return OR_ERR_ARG;
    memset(&j, 0, sizeof(j));
    j.type = type; j.w = (const uint8_t *)w; j.rb = or_row_bytes(type, cols);
    j.cols = cols; j.q = q; j.act_scale = act_scale; j.out = out;
    gemv_slice(&j, 0, rows);
    return OR_OK;
}

/* src/kernels.c:780-805 */
int or_gemv_qk_i8(int type, const int8_t *q, const float *ascale,
                  const void *w, size_t rows, size_t cols, float *out)
{
    gemv_job j;
    if (!q || !ascale || !w || !out || rows == 0 || cols == 0) return OR_ERR_ARG;
    if (cols % 256 || (type != OR_Q4_K && type != OR_Q6_K)) return OR_ERR_ARG;
    memset(&j, 0, sizeof(j));
    j.type = type; j.w = (const uint8_t *)w; j.rb = or_row_bytes(type, cols);
    j.cols = cols; j.q = q; j.ascale = ascale; j.out = out;
    gemv_slice(&j, 0, rows);
    return OR_OK;
}

/* src/kernels.c:809-872 (the x86 dispatch: K-quants go through per-block
 * int8 activations, TQ through one per-vector scale, F16/F32 stay float) */
int or_gemv(int type, const float *x, const void *w, size_t rows, size_t cols,
            float *out, int n_threads)
{
    gemv_job j;
    int8_t *q = NULL;
    float *asc = NULL;

    if (!x || !w || !out || rows == 0 || cols == 0) return OR_ERR_ARG;
    if (!or_block_elems(type)) return OR_ERR_UNSUPPORTED;
    if (!or_row_bytes(type, cols)) return OR_ERR_ARG;

    memset(&j, 0, sizeof(j));
    j.type = type; j.w = (const uint8_t *)w; j.rb = or_row_bytes(type, cols);
    j.cols = cols; j.x = x; j.out = out;

    if (type == OR_TQ1_0 || type == OR_TQ2_0 || type == OR_Q4_K || type == OR_Q6_K) {
        q = (int8_t *)malloc(cols);
        if (!q) return OR_ERR_NOMEM;
        if (type == OR_Q4_K || type == OR_Q6_K) {
            asc = (float *)malloc(cols / 256 * sizeof(float));
            if (!asc) { free(q); return OR_ERR_NOMEM; }
            or_quantize_act_k(x, cols, q, asc);
        } else {
            j.act_scale = quantize_run(x, cols, q);
        }
        j.q = q;
        j.ascale = asc;
    }
    parallel_rows(rows, n_threads, gemv_slice, &j);
    free(q);
    free(asc);
    return OR_OK;
}

/* src/kernels.c:874-941 with the block decoders of src/kernels.c:217-306
 * (Q8_0, Q4_0: 32-element blocks, d f16 first; Q5_K: d, dmin, 12 scale
 * bytes, qh[32], qs[128]) */
int or_dequant_row(int type, const void *row, size_t n, float *out)
{
    const uint8_t *w = (const uint8_t *)row;
    size_t i, b;

    if (!row || !out || n == 0) return OR_ERR_ARG;
    if (!or_row_bytes(type, n)) return OR_ERR_ARG;
    switch (type) {
    case OR_F32:
        memcpy(out, w, n * 4);
        return OR_OK;
    case OR_F16:
        for (i = 0; i < n; i++) out[i] = half_at(w + 2 * i);
        return OR_OK;
    case OR_Q6_K:
        for (b = 0; b < n / 256; b++) {
            const uint8_t *blk = w + b * 210;
            float d = half_at(blk + 208);
            for (i = 0; i < 256; i++) {
                int h = (int)i / 128, grp = ((int)i % 128) / 32, l = (int)i % 32;
                const uint8_t *ql = blk + 64 * h, *qh = blk + 128 + 32 * h;
                const int8_t *sc = (const int8_t *)(blk + 192) + 8 * h;
                int lo = grp & 1 ? ql[l + 32] : ql[l];
                int nib = grp < 2 ? lo & 0x0F : lo >> 4;
                int q6 = (nib | (((qh[l] >> (2 * grp)) & 3) << 4)) - 32;
                out[b * 256 + i] = d * (float)sc[l / 16 + 2 * grp] * (float)q6;
            }
        }
        return OR_OK;
    case OR_Q4_K:
        for (b = 0; b < n / 256; b++) {
            const uint8_t *blk = w + b * 144;
            float d = half_at(blk), dmin = half_at(blk + 2);
            for (i = 0; i < 256; i++) {
                int j = (int)i / 32, sc, mn;
                uint8_t byte = blk[16 + 32 * (j / 2) + i % 32];
                int nib = j & 1 ? byte >> 4 : byte & 0x0F;
                q4k_scale_min(blk + 4, j, &sc, &mn);
                out[b * 256 + i] = d * (float)sc * (float)nib - dmin * (float)mn;
            }
        }
        return OR_OK;
    case OR_Q8_0:
        for (b = 0; b < n / 32; b++) {
            const uint8_t *blk = w + b * 34;
            float d = half_at(blk);
            for (i = 0; i < 32; i++) out[b * 32 + i] = (float)(int8_t)blk[2 + i] * d;
        }
        return OR_OK;
    case OR_Q4_0:
        for (b = 0; b < n / 32; b++) {
            const uint8_t *blk = w + b * 18;
            float d = half_at(blk);
            for (i = 0; i < 32; i++) {
                uint8_t byte = blk[2 + i % 16];
                int nib = i < 16 ? byte & 0x0F : byte >> 4;
                out[b * 32 + i] = (float)(nib - 8) * d;
            }
        }
        return OR_OK;
    case OR_Q5_K:
        for (b = 0; b < n / 256; b++) {
            const uint8_t *blk = w + b * 176;
            float d = half_at(blk), dmin = half_at(blk + 2);
            for (i = 0; i < 256; i++) {
                int grp = (int)i / 32, l = (int)i % 32, sc, mn;
                uint8_t byte = blk[48 + 32 * (grp % 4) + l];
                int v = (grp < 4 ? byte & 0x0F : byte >> 4) | (((blk[16 + l] >> grp) & 1) << 4);
                q4k_scale_min(blk + 4, grp, &sc, &mn);
                out[b * 256 + i] = d * (float)sc * (float)v - dmin * (float)mn;
            }
        }
        return OR_OK;
    default:
        return OR_ERR_UNSUPPORTED;
    }
}

/* ------------------------------------------------------------------ ops */

/* src/ops.c:7-22: squares summed in double, scale rounded to float once */
void or_rmsnorm(float *out, const float *x, const float *w, size_t n, float eps)
{
    double ss = 0.0;
    float scale;
    size_t i;
    for (i = 0; i < n; i++) ss += (double)x[i] * (double)x[i];
    scale = (float)(1.0 / sqrt(ss / (double)n + (double)eps));
    for (i = 0; i < n; i++) out[i] = w ? x[i] * scale * w[i] : x[i] * scale;
}

/* src/ops.c:24-39 */
void or_softmax(float *x, size_t n)
{
    float mx = x[0], sum = 0.0f;
    size_t i;
    for (i = 1; i < n; i++) if (x[i] > mx) mx = x[i];
    for (i = 0; i < n; i++) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    if (sum > 0.0f) {
        float inv = 1.0f / sum;
        for (i = 0; i < n; i++) x[i] *= inv;
    }
}

/* src/ops.c:41-48 */
void or_silu_mul(float *gate, const float *up, size_t n)
{
    size_t i;
    for (i = 0; i < n; i++) {
        float g = gate[i];
        gate[i] = g / (1.0f + expf(-g)) * up[i];
    }
}

/* src/ops.c:50-54 */
void or_add(float *dst, const float *src, size_t n)
{
    size_t i;
    for (i = 0; i < n; i++) dst[i] += src[i];
}

/* src/ops.c:56-73: adjacent pairs (2i, 2i+1) rotate by table entry i */
void or_rope(float *vec, size_t n_heads, size_t head_dim,
             const float *cos_row, const float *sin_row)
{
    size_t h, i;
    for (h = 0; h < n_heads; h++) {
        float *v = vec + h * head_dim;
        for (i = 0; i < head_dim / 2; i++) {
            float a = v[2 * i], b = v[2 * i + 1];
            v[2 * i]     = a * cos_row[i] - b * sin_row[i];
            v[2 * i + 1] = a * sin_row[i] + b * cos_row[i];
        }
    }
}

/* src/ops.c:75-81 */
float or_dot_f32(const float *a, const float *b, size_t n)
{
    float s = 0.0f;
    size_t i;
    for (i = 0; i < n; i++) s += a[i] * b[i];
    return s;
}

/* src/forward.c:104-118: angle p * base^(-2i/hd) in double, cast per entry */
void or_rope_tables(float *cos_t, float *sin_t, size_t n_ctx, size_t head_dim,
                    float freq_base)
{
    size_t half = head_dim / 2, p, i;
    for (p = 0; p < n_ctx; p++)
        for (i = 0; i < half; i++) {
            double ex = -2.0 * (double)i / (double)head_dim;
            double th = (double)p * pow((double)freq_base, ex);
            cos_t[p * half + i] = (float)cos(th);
            sin_t[p * half + i] = (float)sin(th);
        }
}

/* src/sample.c:147-153: first maximum wins (strict '>') */
uint32_t or_argmax(const float *logits, size_t n)
{
    size_t i, best = 0;
    for (i = 1; i < n; i++) if (logits[i] > logits[best]) best = i;
    return (uint32_t)best;
}

/* -------------------------------------------------------------- forward */

struct or_context {
    const or_model *m;
    uint32_t n_ctx, n_batch, pos;
    int n_threads;
    size_t nq, nkv, wide, gqa;
    float *kc, *vc, *x, *xb, *xb2, *q, *kb, *vb, *hb, *hb2, *att, *norm;
    float *logits, *rc, *rs;
};

int or_context_create(const or_model *m, uint32_t n_ctx, uint32_t n_batch,
                      int n_threads, or_context **out)
{
    or_context *c;
    size_t nb;

    if (!m || !out || !n_ctx) return OR_ERR_ARG;
    c = (or_context *)calloc(1, sizeof(*c));
    if (!c) return OR_ERR_NOMEM;
    /* src/forward.c:67-72 */
    if (n_batch == 0) n_batch = 32;
    if (n_batch > n_ctx) n_batch = n_ctx;
    c->m = m; c->n_ctx = n_ctx; c->n_batch = n_batch; c->n_threads = n_threads;
    c->nq = (size_t)m->n_head * m->head_dim;
    c->nkv = (size_t)m->n_head_kv * m->head_dim;
    c->gqa = m->n_head / m->n_head_kv;
    c->wide = c->nq > m->n_embd ? c->nq : m->n_embd;
    nb = n_batch;
    c->kc = (float *)calloc((size_t)m->n_layer * n_ctx * c->nkv, 4);
    c->vc = (float *)calloc((size_t)m->n_layer * n_ctx * c->nkv, 4);
    c->x = (float *)calloc(nb * m->n_embd, 4);
    c->xb = (float *)calloc(nb * c->wide, 4);
    c->xb2 = (float *)calloc(nb * c->wide, 4);
    c->q = (float *)calloc(nb * c->nq, 4);
    c->kb = (float *)calloc(nb * c->nkv, 4);
    c->vb = (float *)calloc(nb * c->nkv, 4);
    c->hb = (float *)calloc(nb * m->n_ff, 4);
    c->hb2 = (float *)calloc(nb * m->n_ff, 4);
    c->att = (float *)calloc(n_ctx, 4);
    c->norm = (float *)calloc(c->wide, 4);
    c->logits = (float *)calloc(m->n_vocab, 4);
    c->rc = (float *)calloc((size_t)n_ctx * (m->head_dim / 2), 4);
    c->rs = (float *)calloc((size_t)n_ctx * (m->head_dim / 2), 4);
    if (!c->kc || !c->vc || !c->x || !c->xb || !c->xb2 || !c->q || !c->kb ||
        !c->vb || !c->hb || !c->hb2 || !c->att || !c->norm || !c->logits ||
        !c->rc || !c->rs) {
        or_context_destroy(c);
        return OR_ERR_NOMEM;
    }
    or_rope_tables(c->rc, c->rs, n_ctx, m->head_dim, m->rope_base);
    *out = c;
    return OR_OK;
}

void or_context_destroy(or_context *c)
{
    if (!c) return;
    free(c->kc); free(c->vc); free(c->x); free(c->xb); free(c->xb2);
    free(c->q); free(c->kb); free(c->vb); free(c->hb); free(c->hb2);
    free(c->att); free(c->norm); free(c->logits); free(c->rc); free(c->rs);
    free(c);
}

void or_context_reset(or_context *c) { if (c) c->pos = 0; }
uint32_t or_context_pos(const or_context *c) { return c ? c->pos : 0; }

int or_context_set_kv(or_context *c, uint32_t layer, uint32_t p0, uint32_t n,
                      const float *k, const float *v)
{
    size_t base;
    if (!c || layer >= c->m->n_layer || (size_t)p0 + n > c->n_ctx) return OR_ERR_ARG;
    base = ((size_t)layer * c->n_ctx + p0) * c->nkv;
    memcpy(c->kc + base, k, (size_t)n * c->nkv * 4);
    memcpy(c->vc + base, v, (size_t)n * c->nkv * 4);
    return OR_OK;
}

int or_context_set_pos(or_context *c, uint32_t pos)
{
    if (!c || pos > c->n_ctx) return OR_ERR_ARG;
    c->pos = pos;
    return OR_OK;
}

/* src/forward.c:167-186: a norm vector is the dequantised tensor */
static const float *norm_vec(or_context *c, const or_tensor *t, size_t n)
{
    or_dequant_row(t->type, t->data, n, c->norm);
    return c->norm;
}

/* src/forward.c:188-213: one gemv per token */
static void project(or_context *c, const or_tensor *t, size_t rows, size_t cols,
                    size_t ntok, const float *in, size_t in_stride,
                    float *out, size_t out_stride)
{
    size_t i;
    for (i = 0; i < ntok; i++)
        or_gemv(t->type, in + i * in_stride, t->data, rows, cols,
                out + i * out_stride, c->n_threads);
}

/* src/forward.c:222-257 for one head: scores, softmax, j-ordered V sum;
 * att is n_ctx floats of scratch */
static void attend_head(or_context *c, size_t layer, size_t tok, size_t h,
                        uint32_t seq_pos, float *att)
{
    const or_model *m = c->m;
    size_t hd = m->head_dim, kvh = h / c->gqa, j, d;
    size_t base = layer * c->n_ctx * c->nkv;
    const float *qh = c->q + tok * c->nq + h * hd;
    float *dst = c->xb + tok * c->wide + h * hd;
    float scale = 1.0f / sqrtf((float)hd);
    size_t upto = (size_t)seq_pos + 1;

    for (j = 0; j < upto; j++)
        att[j] = or_dot_f32(qh, c->kc + base + j * c->nkv + kvh * hd, hd) * scale;
    or_softmax(att, upto);
    for (d = 0; d < hd; d++) dst[d] = 0.0f;
    for (j = 0; j < upto; j++) {
        const float *vj = c->vc + base + j * c->nkv + kvh * hd;
        for (d = 0; d < hd; d++) dst[d] += att[j] * vj[d];
    }
}

/* the heads of one token split over the pool like the reference's
 * attention (src/forward.c:364-371): heads are independent, so the split
 * changes no result */
typedef struct {
    or_context *c;
    size_t layer, tok;
    uint32_t seq_pos;
} attn_job;

static void attend_slice(void *p, size_t begin, size_t end)
{
    attn_job *j = (attn_job *)p;
    float *att = begin == 0 ? j->c->att : (float *)malloc((size_t)j->c->n_ctx * 4);
    size_t h;
    if (!att) return;
    for (h = begin; h < end; h++) attend_head(j->c, j->layer, j->tok, h, j->seq_pos, att);
    if (att != j->c->att) free(att);
}

/* src/forward.c:295-409 */
static int forward_batch(or_context *c, const uint32_t *tok, size_t n, int want_logits)
{
    const or_model *m = c->m;
    size_t d = m->n_embd, i;
    uint32_t l;
    const float *w;
    size_t erow = or_row_bytes(m->token_embd.type, d);

    if ((size_t)c->pos + n > c->n_ctx) return OR_ERR_ARG;
    for (i = 0; i < n; i++) {
        if (tok[i] >= m->n_vocab) return OR_ERR_ARG;
        or_dequant_row(m->token_embd.type,
                       (const uint8_t *)m->token_embd.data + (size_t)tok[i] * erow,
                       d, c->x + i * d);
    }

    for (l = 0; l < m->n_layer; l++) {
        const or_layer *L = &m->layers[l];
        size_t base = (size_t)l * c->n_ctx * c->nkv;

        w = norm_vec(c, &L->attn_norm, d);
        for (i = 0; i < n; i++)
            or_rmsnorm(c->xb + i * c->wide, c->x + i * d, w, d, m->rms_eps);

        project(c, &L->attn_q, c->nq, d, n, c->xb, c->wide, c->q, c->nq);
        project(c, &L->attn_k, c->nkv, d, n, c->xb, c->wide, c->kb, c->nkv);
        project(c, &L->attn_v, c->nkv, d, n, c->xb, c->wide, c->vb, c->nkv);

        for (i = 0; i < n; i++) {
            uint32_t p = c->pos + (uint32_t)i;
            const float *rc = c->rc + (size_t)p * (m->head_dim / 2);
            const float *rs = c->rs + (size_t)p * (m->head_dim / 2);
            or_rope(c->q + i * c->nq, m->n_head, m->head_dim, rc, rs);
            or_rope(c->kb + i * c->nkv, m->n_head_kv, m->head_dim, rc, rs);
            memcpy(c->kc + base + (size_t)p * c->nkv, c->kb + i * c->nkv, c->nkv * 4);
            memcpy(c->vc + base + (size_t)p * c->nkv, c->vb + i * c->nkv, c->nkv * 4);
        }
        for (i = 0; i < n; i++) {
            attn_job job;
            job.c = c; job.layer = l; job.tok = i; job.seq_pos = c->pos + (uint32_t)i;
            parallel_rows(m->n_head, c->n_threads, attend_slice, &job);
        }

        project(c, &L->attn_out, d, c->nq, n, c->xb, c->wide, c->xb2, c->wide);
        for (i = 0; i < n; i++) or_add(c->x + i * d, c->xb2 + i * c->wide, d);

        w = norm_vec(c, &L->ffn_norm, d);
        for (i = 0; i < n; i++)
            or_rmsnorm(c->xb + i * c->wide, c->x + i * d, w, d, m->rms_eps);
        project(c, &L->ffn_gate, m->n_ff, d, n, c->xb, c->wide, c->hb, m->n_ff);
        project(c, &L->ffn_up, m->n_ff, d, n, c->xb, c->wide, c->hb2, m->n_ff);
        for (i = 0; i < n; i++)
            or_silu_mul(c->hb + i * m->n_ff, c->hb2 + i * m->n_ff, m->n_ff);
        project(c, &L->ffn_down, d, m->n_ff, n, c->hb, m->n_ff, c->xb2, c->wide);
        for (i = 0; i < n; i++) or_add(c->x + i * d, c->xb2 + i * c->wide, d);
    }
    c->pos += (uint32_t)n;
    if (!want_logits) return OR_OK;

    w = norm_vec(c, &m->output_norm, d);
    or_rmsnorm(c->xb, c->x + (n - 1) * d, w, d, m->rms_eps);
    project(c, &m->output, m->n_vocab, d, 1, c->xb, c->wide, c->logits, m->n_vocab);
    return OR_OK;
}

/* src/forward.c:411-438: chunks of n_batch tokens, logits for the last */
int or_eval(or_context *c, const uint32_t *tokens, size_t n, float **logits)
{
    size_t done = 0;
    if (!c || !tokens || n == 0) return OR_ERR_ARG;
    while (done < n) {
        size_t chunk = n - done;
        int st;
        if (chunk > c->n_batch) chunk = c->n_batch;
        st = forward_batch(c, tokens + done, chunk, done + chunk == n);
        if (st != OR_OK) return st;
        done += chunk;
    }
    if (logits) *logits = c->logits;
    return OR_OK;
}
