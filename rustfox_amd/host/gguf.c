/* gguf.c -- bounded GGUF v2/v3 reader: header, metadata, tensor table.
 *
 * Same acceptance rules as RustFox src/gguf.c:348-466: magic "GGUF", version
 * 2 or 3, plausible counts, unique keys and tensor names, 1..4 non-zero
 * dimensions, a known block layout whose block divides the element count,
 * general.alignment a power of two <= 4096 (default 32), data section
 * aligned after the tensor table, every tensor inside the file.  Array
 * metadata is skipped (nothing on the decode path reads it).
 */
#include "fox_host_internal.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define MAX_TENSORS 1000000u
#define MAX_META    65536u
#define MAX_STRING  (16u << 20)
#define MAX_ALIGN   4096u

typedef struct {
    FILE    *f;
    uint64_t pos, size;
} rd;

static int take(rd *r, void *p, size_t n)
{
    if ((uint64_t)n > r->size - r->pos) return 0;
    if (n && fread(p, 1, n, r->f) != n) return 0;
    r->pos += n;
    return 1;
}

static int skip(rd *r, uint64_t n)
{
    if (n > r->size - r->pos) return 0;
    if (fseeko(r->f, (off_t)(r->pos + n), SEEK_SET) != 0) return 0;
    r->pos += n;
    return 1;
}

static int le(rd *r, uint64_t *v, int n)
{
    uint8_t b[8];
    int i;
    if (!take(r, b, (size_t)n)) return 0;
    *v = 0;
    for (i = 0; i < n; i++) *v |= (uint64_t)b[i] << (8 * i);
    return 1;
}

static int scalar_size(uint32_t t)
{
    static const int sz[] = { 1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8 };
    return t <= GGUF_F64 ? sz[t] : 0;
}

static int read_str(rd *r, char **out)
{
    uint64_t n;
    char *s;
    if (!le(r, &n, 8) || n > MAX_STRING || n > r->size - r->pos) return 0;
    s = (char *)malloc((size_t)n + 1);
    if (!s) return 0;
    if (!take(r, s, (size_t)n)) { free(s); return 0; }
    s[n] = '\0';
    *out = s;
    return 1;
}

static int skip_array(rd *r)
{
    uint64_t et, count, i, n;
    if (!le(r, &et, 4) || et > GGUF_F64 || et == GGUF_ARRAY) return 0;
    if (!le(r, &count, 8) || count > MAX_TENSORS * 16ull) return 0;
    if (et == GGUF_STRING) {
        for (i = 0; i < count; i++)
            if (!le(r, &n, 8) || n > MAX_STRING || !skip(r, n)) return 0;
        return 1;
    }
    return skip(r, count * (uint64_t)scalar_size((uint32_t)et));
}

/* block elements and bytes of each ggml type (RustFox src/gguf.c:160-195) */
int fox_type_layout(uint32_t t, uint32_t *block, uint32_t *bytes)
{
    static const struct { uint32_t t, block, bytes; } tab[] = {
        { 0, 1, 4 }, { 1, 1, 2 }, { 30, 1, 2 }, { 24, 1, 1 }, { 25, 1, 2 },
        { 26, 1, 4 }, { 27, 1, 8 }, { 28, 1, 8 }, { 2, 32, 18 }, { 3, 32, 20 },
        { 6, 32, 22 }, { 7, 32, 24 }, { 8, 32, 34 }, { 15, 256, 292 },
        { 10, 256, 84 }, { 11, 256, 110 }, { 12, 256, 144 }, { 13, 256, 176 },
        { 14, 256, 210 }, { 16, 256, 66 }, { 17, 256, 74 }, { 18, 256, 98 },
        { 19, 256, 50 }, { 20, 32, 18 }, { 21, 256, 110 }, { 22, 256, 82 },
        { 23, 256, 136 }, { 29, 256, 56 }, { 34, 256, 54 }, { 35, 256, 66 },
    };
    size_t i;
    for (i = 0; i < sizeof(tab) / sizeof(tab[0]); i++)
        if (tab[i].t == t) { *block = tab[i].block; *bytes = tab[i].bytes; return 1; }
    return 0;
}

void fox_gguf_close(fox_gguf *g)
{
    size_t i;
    if (!g) return;
    for (i = 0; i < g->n_meta; i++) { free(g->meta[i].key); free(g->meta[i].str); }
    for (i = 0; i < g->n_tensors; i++) free(g->tensors[i].name);
    free(g->meta);
    free(g->tensors);
    free(g);
}

fox_status fox_gguf_open(const char *path, fox_gguf **out)
{
    rd r;
    fox_gguf *g;
    char magic[4];
    uint64_t v, n_tensors, n_meta, i, j;
    fox_status st = FOX_ERR_FORMAT;

    if (!path || !out) return fox_fail(FOX_ERR_ARG, "gguf: null path or output");
    *out = NULL;
    r.f = fopen(path, "rb");
    if (!r.f) return fox_fail(FOX_ERR_IO, "gguf: cannot open %s", path);
    if (fseeko(r.f, 0, SEEK_END) != 0) { fclose(r.f); return fox_fail(FOX_ERR_IO, "gguf: seek"); }
    r.size = (uint64_t)ftello(r.f);
    r.pos = 0;
    rewind(r.f);

    g = (fox_gguf *)calloc(1, sizeof(*g));
    if (!g) { fclose(r.f); return fox_fail(FOX_ERR_NOMEM, "gguf: header"); }
    g->file_size = r.size;
    g->alignment = 32;

    if (!take(&r, magic, 4) || memcmp(magic, "GGUF", 4) != 0) {
        st = fox_fail(FOX_ERR_FORMAT, "gguf: %s is not a GGUF file", path);
        goto fail;
    }
    if (!le(&r, &v, 4) || !le(&r, &n_tensors, 8) || !le(&r, &n_meta, 8)) {
        st = fox_fail(FOX_ERR_FORMAT, "gguf: truncated header in %s", path);
        goto fail;
    }
    if (v < 2 || v > 3) {
        st = fox_fail(FOX_ERR_UNSUPPORTED, "gguf: file format version %llu is not supported",
                      (unsigned long long)v);
        goto fail;
    }
    if (n_tensors > MAX_TENSORS || n_meta > MAX_META) {
        st = fox_fail(FOX_ERR_FORMAT, "gguf: implausible header counts");
        goto fail;
    }
    g->version = (uint32_t)v;
    g->meta = (fox_meta *)calloc(n_meta ? n_meta : 1, sizeof(fox_meta));
    g->tensors = (fox_tensor_desc *)calloc(n_tensors ? n_tensors : 1, sizeof(fox_tensor_desc));
    if (!g->meta || !g->tensors) { st = fox_fail(FOX_ERR_NOMEM, "gguf: tables"); goto fail; }

    for (i = 0; i < n_meta; i++) {
        fox_meta *m = &g->meta[i];
        uint64_t t;
        if (!read_str(&r, &m->key)) { st = fox_fail(FOX_ERR_FORMAT, "gguf: bad metadata key"); goto fail; }
        g->n_meta = i + 1;
        for (j = 0; j < i; j++)
            if (strcmp(g->meta[j].key, m->key) == 0) {
                st = fox_fail(FOX_ERR_FORMAT, "gguf: duplicate metadata key '%s'", m->key);
                goto fail;
            }
        if (!le(&r, &t, 4) || t > GGUF_F64) {
            st = fox_fail(FOX_ERR_FORMAT, "gguf: bad value type for key '%s'", m->key);
            goto fail;
        }
        m->type = (uint32_t)t;
        if (t == GGUF_STRING) {
            if (!read_str(&r, &m->str)) {
                st = fox_fail(FOX_ERR_FORMAT, "gguf: bad string for key '%s'", m->key);
                goto fail;
            }
        } else if (t == GGUF_ARRAY) {
            if (!skip_array(&r)) {
                st = fox_fail(FOX_ERR_FORMAT, "gguf: bad array for key '%s'", m->key);
                goto fail;
            }
        } else if (!le(&r, &m->raw, scalar_size(m->type))) {
            st = fox_fail(FOX_ERR_FORMAT, "gguf: bad scalar for key '%s'", m->key);
            goto fail;
        }
        if (t == GGUF_U32 && strcmp(m->key, "general.alignment") == 0)
            g->alignment = (uint32_t)m->raw;
    }
    if (g->alignment == 0 || (g->alignment & (g->alignment - 1)) || g->alignment > MAX_ALIGN) {
        st = fox_fail(FOX_ERR_FORMAT, "gguf: bad general.alignment %u", g->alignment);
        goto fail;
    }

    for (i = 0; i < n_tensors; i++) {
        fox_tensor_desc *t = &g->tensors[i];
        uint64_t dims, type, elems = 1, d;
        uint32_t block, bytes;
        if (!read_str(&r, &t->name)) { st = fox_fail(FOX_ERR_FORMAT, "gguf: bad tensor name"); goto fail; }
        g->n_tensors = i + 1;
        for (j = 0; j < i; j++)
            if (strcmp(g->tensors[j].name, t->name) == 0) {
                st = fox_fail(FOX_ERR_FORMAT, "gguf: duplicate tensor name '%s'", t->name);
                goto fail;
            }
        if (!le(&r, &dims, 4) || dims == 0 || dims > 4) {
            st = fox_fail(FOX_ERR_FORMAT, "gguf: tensor '%s' declares %llu dimensions", t->name,
                          (unsigned long long)dims);
            goto fail;
        }
        t->n_dims = (uint32_t)dims;
        for (j = 0; j < dims; j++) {
            if (!le(&r, &d, 8) || d == 0 || (elems && d > UINT64_MAX / elems)) {
                st = fox_fail(FOX_ERR_FORMAT, "gguf: tensor '%s' has a bad dimension", t->name);
                goto fail;
            }
            t->ne[j] = d;
            elems *= d;
        }
        if (!le(&r, &type, 4) || !le(&r, &t->offset, 8)) {
            st = fox_fail(FOX_ERR_FORMAT, "gguf: truncated descriptor for '%s'", t->name);
            goto fail;
        }
        if (!fox_type_layout((uint32_t)type, &block, &bytes)) {
            st = fox_fail(FOX_ERR_UNSUPPORTED, "gguf: tensor '%s' uses quantisation type %llu, "
                          "which rustfox_amd cannot lay out", t->name, (unsigned long long)type);
            goto fail;
        }
        if (elems % block) {
            st = fox_fail(FOX_ERR_FORMAT, "gguf: tensor '%s' holds %llu elements, not a multiple "
                          "of its %u-element block", t->name, (unsigned long long)elems, block);
            goto fail;
        }
        t->type = (uint32_t)type;
        t->size_bytes = elems / block * bytes;
    }
    g->data_offset = (r.pos + g->alignment - 1) / g->alignment * g->alignment;
    if (g->data_offset > r.size) { st = fox_fail(FOX_ERR_FORMAT, "gguf: data section starts past the end"); goto fail; }
    for (i = 0; i < g->n_tensors; i++) {
        uint64_t end = g->data_offset + g->tensors[i].offset;
        if (end < g->data_offset || end + g->tensors[i].size_bytes < end ||
            end + g->tensors[i].size_bytes > r.size) {
            st = fox_fail(FOX_ERR_FORMAT, "gguf: tensor '%s' extends past the end of the file",
                          g->tensors[i].name);
            goto fail;
        }
    }
    fclose(r.f);
    *out = g;
    return FOX_OK;

fail:
    fclose(r.f);
    fox_gguf_close(g);
    return st;
}

size_t fox_gguf_find(const fox_gguf *g, const char *key)
{
    size_t i;
    if (!g || !key) return FOX_TENSOR_ABSENT;
    for (i = 0; i < g->n_meta; i++) if (strcmp(g->meta[i].key, key) == 0) return i;
    return FOX_TENSOR_ABSENT;
}

fox_status fox_gguf_get_uint(const fox_gguf *g, size_t idx, uint64_t *out)
{
    const fox_meta *m;
    if (!g || idx >= g->n_meta || !out) return FOX_ERR_ARG;
    m = &g->meta[idx];
    switch (m->type) {
    case GGUF_U8: case GGUF_U16: case GGUF_U32: case GGUF_U64: case GGUF_BOOL:
        *out = m->raw; return FOX_OK;
    case GGUF_I8: *out = (uint64_t)(int64_t)(int8_t)m->raw; return FOX_OK;
    case GGUF_I16: *out = (uint64_t)(int64_t)(int16_t)m->raw; return FOX_OK;
    case GGUF_I32: *out = (uint64_t)(int64_t)(int32_t)m->raw; return FOX_OK;
    case GGUF_I64: *out = m->raw; return FOX_OK;
    default: return FOX_ERR_FORMAT;
    }
}

fox_status fox_gguf_get_f32(const fox_gguf *g, size_t idx, float *out)
{
    uint32_t u;
    if (!g || idx >= g->n_meta || !out) return FOX_ERR_ARG;
    if (g->meta[idx].type != GGUF_F32) return FOX_ERR_FORMAT;
    u = (uint32_t)g->meta[idx].raw;
    memcpy(out, &u, 4);
    return FOX_OK;
}

fox_status fox_gguf_get_string(const fox_gguf *g, size_t idx, const char **out)
{
    if (!g || idx >= g->n_meta || !out) return FOX_ERR_ARG;
    if (g->meta[idx].type != GGUF_STRING) return FOX_ERR_FORMAT;
    *out = g->meta[idx].str;
    return FOX_OK;
}

size_t fox_gguf_tensor_find(const fox_gguf *g, const char *name)
{
    size_t i;
    if (!g || !name) return FOX_TENSOR_ABSENT;
    for (i = 0; i < g->n_tensors; i++) if (strcmp(g->tensors[i].name, name) == 0) return i;
    return FOX_TENSOR_ABSENT;
}
