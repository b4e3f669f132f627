/* gguf.c -- bounded GGUF v2/v3 reader: header, metadata, tensor table.
 *
 * Same acceptance rules as RustFox src/gguf.c:348-466: magic "GGUF", version
 * 2 or 3, plausible counts, unique keys and tensor names, 1..4 non-zero
 * dimensions, a known block layout whose block divides the element count,
 * general.alignment a power of two <= 4096 (default 32), data section
 * aligned after the tensor table, every tensor inside the file.  Array
 * metadata is read into memory (scalar elements as their bits, strings as
 * strings) for the fox_gguf_get_array_* accessors.
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

/* an array value: element type, count, then the elements (nested arrays
 * are refused, as RustFox src/gguf.c:128-175 refuses them) */
static int read_array(rd *r, fox_meta *m)
{
    uint64_t et, count, i;
    if (!le(r, &et, 4) || et > GGUF_F64 || et == GGUF_ARRAY) return 0;
    if (!le(r, &count, 8) || count > MAX_TENSORS * 16ull) return 0;
    m->atype = (uint32_t)et;
    if (et == GGUF_STRING) {
        /* each string takes at least its 8-byte length */
        if (count > (r->size - r->pos) / 8) return 0;
        m->astrs = (char **)calloc(count ? count : 1, sizeof(char *));
        if (!m->astrs) return 0;
        for (i = 0; i < count; i++) {
            if (!read_str(r, &m->astrs[i])) return 0;
            m->acount = i + 1;
        }
        return 1;
    }
    {
        const int sz = scalar_size((uint32_t)et);
        if (count > (r->size - r->pos) / (uint64_t)sz) return 0;
        m->avals = (uint64_t *)malloc((count ? count : 1) * sizeof(uint64_t));
        if (!m->avals) return 0;
        for (i = 0; i < count; i++)
            if (!le(r, &m->avals[i], sz)) return 0;
        m->acount = count;
    }
    return 1;
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
    for (i = 0; i < g->n_meta; i++) {
        fox_meta *m = &g->meta[i];
        uint64_t j;
        free(m->key);
        free(m->str);
        if (m->astrs)
            for (j = 0; j < m->acount; j++) free(m->astrs[j]);
        free(m->astrs);
        free(m->avals);
    }
    for (i = 0; i < g->n_tensors; i++) free(g->tensors[i].name);
    free(g->meta);
    free(g->tensors);
    free(g->path);
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
    g->path = strdup(path);
    if (!g->path) { fclose(r.f); free(g); return fox_fail(FOX_ERR_NOMEM, "gguf: path"); }

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
            if (!read_array(&r, m)) {
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

uint32_t fox_gguf_version(const fox_gguf *g) { return g ? g->version : 0; }
size_t fox_gguf_metadata_count(const fox_gguf *g) { return g ? g->n_meta : 0; }
size_t fox_gguf_tensor_count(const fox_gguf *g) { return g ? g->n_tensors : 0; }

size_t fox_gguf_find(const fox_gguf *g, const char *key)
{
    size_t i;
    if (!g || !key) return FOX_TENSOR_ABSENT;
    for (i = 0; i < g->n_meta; i++) if (strcmp(g->meta[i].key, key) == 0) return i;
    return FOX_TENSOR_ABSENT;
}

/* the metadata entry idx of type `want` (any type with want < 0) */
static fox_status meta_of(const fox_gguf *g, size_t idx, const void *out, int want,
                          const fox_meta **m)
{
    if (!g || !out) return FOX_ERR_ARG;
    if (idx >= g->n_meta) return FOX_ERR_NOTFOUND;
    *m = &g->meta[idx];
    if (want >= 0 && (*m)->type != (uint32_t)want) return FOX_ERR_FORMAT;
    return FOX_OK;
}

fox_gguf_value_type fox_gguf_metadata_type(const fox_gguf *g, size_t idx)
{
    if (!g || idx >= g->n_meta) return FOX_GGUF_ARRAY;
    return (fox_gguf_value_type)g->meta[idx].type;
}

size_t fox_gguf_metadata_array_count(const fox_gguf *g, size_t idx)
{
    if (!g || idx >= g->n_meta || g->meta[idx].type != GGUF_ARRAY) return 0;
    return (size_t)g->meta[idx].acount;
}

fox_gguf_value_type fox_gguf_metadata_array_type(const fox_gguf *g, size_t idx)
{
    if (!g || idx >= g->n_meta || g->meta[idx].type != GGUF_ARRAY) return FOX_GGUF_ARRAY;
    return (fox_gguf_value_type)g->meta[idx].atype;
}

fox_status fox_gguf_get_u32(const fox_gguf *g, size_t idx, uint32_t *out)
{
    const fox_meta *m;
    fox_status st = meta_of(g, idx, out, GGUF_U32, &m);
    if (st == FOX_OK) *out = (uint32_t)m->raw;
    return st;
}

fox_status fox_gguf_get_bool(const fox_gguf *g, size_t idx, int *out)
{
    const fox_meta *m;
    fox_status st = meta_of(g, idx, out, GGUF_BOOL, &m);
    if (st == FOX_OK) *out = m->raw != 0;
    return st;
}

fox_status fox_gguf_get_uint(const fox_gguf *g, size_t idx, uint64_t *out)
{
    const fox_meta *m;
    fox_status st = meta_of(g, idx, out, -1, &m);
    if (st != FOX_OK) return st;
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
    const fox_meta *m;
    uint32_t u;
    fox_status st = meta_of(g, idx, out, GGUF_F32, &m);
    if (st != FOX_OK) return st;
    u = (uint32_t)m->raw;
    memcpy(out, &u, 4);
    return FOX_OK;
}

fox_status fox_gguf_get_string(const fox_gguf *g, size_t idx, const char **out)
{
    const fox_meta *m;
    fox_status st = meta_of(g, idx, out, GGUF_STRING, &m);
    if (st == FOX_OK) *out = m->str;
    return st;
}

/* element `el` of an array of `want` elements */
static fox_status elem_of(const fox_gguf *g, size_t idx, size_t el, const void *out,
                          uint32_t want, const fox_meta **m)
{
    fox_status st = meta_of(g, idx, out, GGUF_ARRAY, m);
    if (st != FOX_OK) return st;
    if ((*m)->atype != want) return FOX_ERR_FORMAT;
    if (el >= (*m)->acount) return FOX_ERR_NOTFOUND;
    return FOX_OK;
}

fox_status fox_gguf_get_array_string(const fox_gguf *g, size_t idx, size_t el, const char **out)
{
    const fox_meta *m;
    fox_status st = elem_of(g, idx, el, out, GGUF_STRING, &m);
    if (st == FOX_OK) *out = m->astrs[el];
    return st;
}

fox_status fox_gguf_get_array_i32(const fox_gguf *g, size_t idx, size_t el, int32_t *out)
{
    const fox_meta *m;
    fox_status st = elem_of(g, idx, el, out, GGUF_I32, &m);
    if (st == FOX_OK) *out = (int32_t)(uint32_t)m->avals[el];
    return st;
}

fox_status fox_gguf_get_array_f32(const fox_gguf *g, size_t idx, size_t el, float *out)
{
    const fox_meta *m;
    uint32_t u;
    fox_status st = elem_of(g, idx, el, out, GGUF_F32, &m);
    if (st != FOX_OK) return st;
    u = (uint32_t)m->avals[el];
    memcpy(out, &u, 4);
    return FOX_OK;
}

fox_status fox_gguf_tensor_at(const fox_gguf *g, size_t idx, fox_gguf_tensor *out)
{
    const fox_tensor_desc *t;
    uint32_t d;
    if (!g || !out) return FOX_ERR_ARG;
    if (idx >= g->n_tensors) return FOX_ERR_NOTFOUND;
    t = &g->tensors[idx];
    memset(out, 0, sizeof(*out));
    out->name = t->name;
    out->n_dims = t->n_dims;
    for (d = 0; d < t->n_dims && d < FOX_GGUF_MAX_DIMS; d++) out->ne[d] = t->ne[d];
    out->type = (fox_ggml_type)t->type;
    out->offset = t->offset;
    out->size_bytes = t->size_bytes;
    return FOX_OK;
}

size_t fox_gguf_tensor_find(const fox_gguf *g, const char *name)
{
    size_t i;
    if (!g || !name) return FOX_TENSOR_ABSENT;
    for (i = 0; i < g->n_tensors; i++) if (strcmp(g->tensors[i].name, name) == 0) return i;
    return FOX_TENSOR_ABSENT;
}

fox_status fox_gguf_read_tensor(const fox_gguf *g, size_t idx, void *dst, size_t capacity)
{
    const fox_tensor_desc *t;
    FILE *f;
    int ok;
    if (!g || !dst) return FOX_ERR_ARG;
    if (idx >= g->n_tensors) return FOX_ERR_NOTFOUND;
    t = &g->tensors[idx];
    if (t->size_bytes > capacity) return FOX_ERR_ARG;
    f = fopen(g->path, "rb");
    if (!f) return FOX_ERR_IO;
    ok = fseeko(f, (off_t)(g->data_offset + t->offset), SEEK_SET) == 0 &&
         fread(dst, 1, (size_t)t->size_bytes, f) == (size_t)t->size_bytes;
    fclose(f);
    return ok ? FOX_OK : FOX_ERR_IO;
}
