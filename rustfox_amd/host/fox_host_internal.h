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
    char     *key;
    uint32_t  type;
    uint64_t  raw;       /* scalar bits, little endian */
    char     *str;       /* GGUF_STRING */
    uint32_t  atype;     /* GGUF_ARRAY: element type and count */
    uint64_t  acount;
    uint64_t *avals;     /* scalar elements' bits */
    char    **astrs;     /* string elements */
} fox_meta;

typedef struct {
    char    *name;
    uint32_t n_dims;
    uint64_t ne[4];
    uint32_t type;
    uint64_t offset;     /* from the start of the data section */
    uint64_t size_bytes;
} fox_tensor_desc;

/* the parsed file (opaque fox_gguf of include/fox_host.h) */
struct fox_gguf {
    uint32_t         version;
    size_t           n_meta;
    fox_meta        *meta;
    size_t           n_tensors;
    fox_tensor_desc *tensors;
    uint32_t         alignment;
    uint64_t         data_offset;
    uint64_t         file_size;
    char            *path;
};

int        fox_type_layout(uint32_t type, uint32_t *block, uint32_t *bytes);

/* --------------------------------------------------------------- weights */

/* the tensors of one transformer layer, in this order */
enum {
    FOX_ROLE_ATTN_NORM, FOX_ROLE_ATTN_Q, FOX_ROLE_ATTN_K, FOX_ROLE_ATTN_V, FOX_ROLE_ATTN_OUT,
    FOX_ROLE_FFN_NORM, FOX_ROLE_FFN_GATE, FOX_ROLE_FFN_UP, FOX_ROLE_FFN_DOWN, FOX_LAYER_ROLES
};

/* FOX_WEIGHTS_STREAM: one layer's tensors in HBM, reloaded in place */
typedef struct {
    int              layer;          /* layer held, -1 for none */
    fox_gpu_tensor  *t[FOX_LAYER_ROLES];
    fox_gpu_event   *ready;          /* copy stream: the upload of `layer` is done */
    fox_gpu_event   *used;           /* compute stream: its last queued use is done */
    int              used_set;
    int              pins;           /* live leases on its tensors */
    uint64_t         last_used;
} fox_layer_slot;

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
    /* FOX_WEIGHTS_STREAM */
    int              *layer_of;      /* per tensor: its layer, or -1 (kept resident) */
    int              *role_of;       /* per tensor: its FOX_ROLE_* within the layer */
    size_t           *lt;            /* tensor index of (layer, role): lt[l * ROLES + r] */
    uint32_t          n_layer;
    uint64_t          layer_bytes;   /* GGUF bytes of one layer */
    uint64_t          stage_off[FOX_LAYER_ROLES]; /* a layer's tensors in the staging
                                                     buffers (256-byte aligned) */
    uint64_t          stage_bytes;   /* staging bytes of one layer */
    fox_layer_slot   *slots;
    int               n_slots;
    uint8_t          *pinned[2];     /* host staging of one layer, alternating */
    fox_gpu_event    *staged[2];     /* copy stream: done reading pinned[i] */
    int               staged_set[2];
    int               next_pin;
    void             *dev_stage;     /* device staging of one layer's GGUF bytes */
    uint64_t          clock, evictions;
};

const fox_tensor_desc *fox_weights_desc(const fox_weights *w, size_t idx);
/* The device tensor of tensor idx for kernels queued next on the compute
 * stream.  Resident tensors come from the backend's table; in
 * FOX_WEIGHTS_STREAM a layer tensor comes from its layer's slot, the layer
 * being loaded first if no slot holds it, and the compute stream is made to
 * wait for that slot's upload. */
fox_status fox_weights_use(fox_weights *w, size_t idx, const fox_gpu_tensor **out);
/* FOX_WEIGHTS_STREAM: the nine tensors of layer l, as fox_weights_use */
fox_status fox_weights_use_layer(fox_weights *w, uint32_t l, const fox_gpu_tensor **t);
/* FOX_WEIGHTS_STREAM: every kernel reading layer l's slot is queued; its
 * slot may be reloaded once the compute stream has passed this point */
void       fox_weights_done_layer(fox_weights *w, uint32_t l);
/* FOX_WEIGHTS_STREAM: start loading layer l into a free or least recently
 * used slot if none holds it (the upload runs on the copy stream) */
fox_status fox_weights_prefetch_layer(fox_weights *w, uint32_t l);

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
