/* fox_host_internal.h -- shared state of the C host library (libfox.so). */
#ifndef FOX_HOST_INTERNAL_H
#define FOX_HOST_INTERNAL_H

#include "../../include/fox_gpu.h"
#include "../../include/fox_host.h"

#include <pthread.h>
#include <stddef.h>
#include <stdint.h>

#define FOX_TENSOR_ABSENT ((size_t)-1)

/* internal to libfox.so: not exported */
#pragma GCC visibility push(hidden)

/* errors and logging (log.c) */
fox_status fox_fail(fox_status st, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void       fox_warn(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
/* map a device-library failure to fox_status, keeping its message */
fox_status fox_gpu_failed(fox_gpu_status st, const char *what);

/* ------------------------------------------------------------------ gguf */

enum {
    GGUF_U8 = 0, GGUF_I8, GGUF_U16, GGUF_I16, GGUF_U32, GGUF_I32, GGUF_F32,
    GGUF_BOOL, GGUF_STRING, GGUF_ARRAY, GGUF_U64, GGUF_I64, GGUF_F64
};

typedef struct {
    char    *key;
    uint32_t type;
    uint64_t raw;        /* scalar bits, little endian */
    char    *str;        /* GGUF_STRING */
} fox_meta;

typedef struct {
    char    *name;
    uint32_t n_dims;
    uint64_t ne[4];
    uint32_t type;
    uint64_t offset;     /* from the start of the data section */
    uint64_t size_bytes;
} fox_tensor_desc;

typedef struct {
    uint32_t         version;
    size_t           n_meta;
    fox_meta        *meta;
    size_t           n_tensors;
    fox_tensor_desc *tensors;
    uint32_t         alignment;
    uint64_t         data_offset;
    uint64_t         file_size;
} fox_gguf;

fox_status fox_gguf_open(const char *path, fox_gguf **out);
void       fox_gguf_close(fox_gguf *g);
size_t     fox_gguf_find(const fox_gguf *g, const char *key);
fox_status fox_gguf_get_uint(const fox_gguf *g, size_t idx, uint64_t *out);
fox_status fox_gguf_get_f32(const fox_gguf *g, size_t idx, float *out);
fox_status fox_gguf_get_string(const fox_gguf *g, size_t idx, const char **out);
size_t     fox_gguf_tensor_find(const fox_gguf *g, const char *name);
int        fox_type_layout(uint32_t type, uint32_t *block, uint32_t *bytes);

/* --------------------------------------------------------------- weights */

struct fox_weights {
    fox_gguf         *g;
    fox_weights_mode  mode;
    uint64_t          budget;
    int               fd;
    uint8_t         **host;     /* FOX_WEIGHTS_RESIDENT */
    fox_gpu_tensor  **dev;      /* FOX_WEIGHTS_DEVICE */
    fox_gpu_ctx      *gpu;
    pthread_mutex_t   lock;
    size_t            live;
    uint64_t          held;
    uint64_t          reads;
};

const fox_tensor_desc *fox_weights_desc(const fox_weights *w, size_t idx);

/* ----------------------------------------------------------------- model */

typedef struct {
    size_t attn_norm, attn_q, attn_k, attn_v, attn_out;
    size_t ffn_norm, ffn_gate, ffn_up, ffn_down;
} fox_layer_tensors;

struct fox_model {
    fox_model_info     info;
    fox_weights       *weights;
    fox_layer_tensors *layers;
    size_t             token_embd, output_norm, output;
};

#pragma GCC visibility pop

#endif
