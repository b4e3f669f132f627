/* weights.c -- the lease API (RustFox include/fox/fox.h:370-403) with three
 * backends:
 *
 *   RESIDENT  host bytes (src/weights.c:461-496 semantics: a tensor is read
 *             on first touch, once);
 *   DEVICE    each tensor in HBM as a fox_gpu_tensor, read once from the file
 *             and uploaded once;
 *   STREAM    the GPU form of RustFox's storage-streamed slots
 *             (src/weights.c:248-459) for models larger than the HBM the
 *             caller grants: embeddings, the output head and other tensors
 *             outside the layers stay resident; the layers go through a ring
 *             of layer slots in HBM.  A layer is read from the file into
 *             pinned host memory (two buffers, alternating) and uploaded on
 *             the copy stream, in place into the least recently used slot
 *             without a lease, while the compute stream works on the layer
 *             before it (the layer-ahead prefetch of src/forward.c:322-337).
 *             Events order the two streams: the compute stream waits for a
 *             slot's upload, the copy stream for the compute stream's last
 *             use of the slot it overwrites.
 *
 * Contract kept from the reference: at most FOX_WEIGHTS_MAX_LIVE_LEASES live
 * leases (src/weights.c:789-797), lease.bytes is the GGUF tensor size,
 * lease.data is borrowed until release and cleared by it (887-890), calls
 * are thread-safe under one lock, fox_weights_reads counts tensor reads from
 * the file (one per tensor for the resident backends, again at every reload
 * when streaming), fox_weights_evictions counts tensors whose slot was
 * reloaded, prefetch_async/_wait report FOX_ERR_UNSUPPORTED where no
 * asynchronous load exists (722, 750).
 *
 * The streaming budget is the HBM the weights may take, in GGUF bytes: the
 * resident tensors plus as many layer slots as fit, at least two (one in
 * use, one loading); a budget below that is refused with FOX_ERR_NOMEM.
 * Budget 0 gives every layer a slot (nothing is reloaded).
 */
#include "fox_host_internal.h"

#include <fcntl.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

static int device_ordinal(void)
{
    const char *e = getenv("FOX_DEVICE");
    return e && *e ? atoi(e) : 0;
}

const fox_tensor_desc *fox_weights_desc(const fox_weights *w, size_t idx)
{
    return (w && idx < w->g->n_tensors) ? &w->g->tensors[idx] : NULL;
}

static const char *const ROLE_NAME[FOX_LAYER_ROLES] = {
    "attn_norm", "attn_q", "attn_k", "attn_v", "attn_output",
    "ffn_norm", "ffn_gate", "ffn_up", "ffn_down",
};

static fox_status read_bytes(fox_weights *w, const fox_tensor_desc *t, uint8_t *dst)
{
    uint64_t done = 0, at = w->g->data_offset + t->offset;
    while (done < t->size_bytes) {
        size_t chunk = t->size_bytes - done > (1u << 30) ? (1u << 30) : (size_t)(t->size_bytes - done);
        ssize_t got = pread(w->fd, dst + done, chunk, (off_t)(at + done));
        if (got <= 0) return fox_fail(FOX_ERR_IO, "weights: short read on '%s'", t->name);
        done += (uint64_t)got;
    }
    return FOX_OK;
}

/* ------------------------------------------------------------ streaming */

/* A layer's bytes are read by up to STREAM_READERS threads: one thread moves
 * about 10-15 GB/s out of the page cache, less than the upload to HBM
 * takes.  The layer's tensors are one list of (file offset, destination,
 * size) segments; thread k reads bytes [k, k + 1) x total / n of their
 * concatenation. */
#define STREAM_READERS 4
#define STREAM_READ_MIN (4u << 20)      /* bytes per reader at least */

typedef struct {
    uint64_t at, size;
    uint8_t *dst;
} read_seg;

typedef struct {
    int fd;
    const read_seg *seg;
    int nseg;
    uint64_t b0, b1;                    /* byte range of the concatenation */
    int failed;
} read_part;

static void *read_part_run(void *arg)
{
    read_part *p = (read_part *)arg;
    uint64_t base = 0;
    int i;
    for (i = 0; i < p->nseg && base < p->b1; base += p->seg[i].size, i++) {
        const uint64_t s0 = base > p->b0 ? base : p->b0;
        const uint64_t e = base + p->seg[i].size, s1 = e < p->b1 ? e : p->b1;
        uint64_t done = 0;
        if (s1 <= s0) continue;
        while (done < s1 - s0) {
            const uint64_t left = s1 - s0 - done;
            const size_t chunk = left > (1u << 30) ? (1u << 30) : (size_t)left;
            const uint64_t o = s0 - base + done;
            ssize_t got = pread(p->fd, p->seg[i].dst + o, chunk, (off_t)(p->seg[i].at + o));
            if (got <= 0) {
                p->failed = 1;
                return NULL;
            }
            done += (uint64_t)got;
        }
    }
    return NULL;
}

static fox_status read_segments(fox_weights *w, const read_seg *seg, int nseg)
{
    uint64_t total = 0;
    read_part part[STREAM_READERS];
    pthread_t th[STREAM_READERS];
    int started[STREAM_READERS] = {0};
    int n, k, failed = 0;
    for (k = 0; k < nseg; k++) total += seg[k].size;
    n = (int)(total / STREAM_READ_MIN);
    n = n < 1 ? 1 : n > STREAM_READERS ? STREAM_READERS : n;
    for (k = 0; k < n; k++) {
        part[k].fd = w->fd;
        part[k].seg = seg;
        part[k].nseg = nseg;
        part[k].b0 = total * (uint64_t)k / (uint64_t)n;
        part[k].b1 = total * (uint64_t)(k + 1) / (uint64_t)n;
        part[k].failed = 0;
    }
    /* parts 1.. on their own threads (a part whose thread cannot start is
     * read here), part 0 on this one */
    for (k = 1; k < n; k++)
        started[k] = pthread_create(&th[k], NULL, read_part_run, &part[k]) == 0;
    read_part_run(&part[0]);
    for (k = 1; k < n; k++) {
        if (started[k]) pthread_join(th[k], NULL);
        else read_part_run(&part[k]);
    }
    for (k = 0; k < n; k++) failed |= part[k].failed;
    return failed ? fox_fail(FOX_ERR_IO, "weights: short read while streaming a layer") : FOX_OK;
}

/* which layer and role each tensor plays ("blk.<l>.<role>.weight") */
static fox_status map_layers(fox_weights *w)
{
    const fox_gguf *g = w->g;
    size_t i, n = g->n_tensors;
    uint32_t l, r;

    w->layer_of = (int *)malloc((n ? n : 1) * sizeof(int));
    w->role_of = (int *)malloc((n ? n : 1) * sizeof(int));
    if (!w->layer_of || !w->role_of) return fox_fail(FOX_ERR_NOMEM, "weights: layer map");
    w->n_layer = 0;
    for (i = 0; i < n; i++) {
        unsigned layer;
        char role[64];
        int used = 0;
        w->layer_of[i] = -1;
        w->role_of[i] = -1;
        if (sscanf(g->tensors[i].name, "blk.%u.%63[^.].weight%n", &layer, role, &used) != 2 ||
            used == 0 || g->tensors[i].name[used] != '\0' || layer > 1000000u)
            continue;
        for (r = 0; r < FOX_LAYER_ROLES; r++) {
            if (strcmp(role, ROLE_NAME[r]) == 0) {
                w->layer_of[i] = (int)layer;
                w->role_of[i] = (int)r;
                if (layer + 1 > w->n_layer) w->n_layer = layer + 1;
                break;
            }
        }
    }
    if (w->n_layer == 0) return fox_fail(FOX_ERR_FORMAT, "weights: no layer tensors to stream");
    w->lt = (size_t *)malloc((size_t)w->n_layer * FOX_LAYER_ROLES * sizeof(size_t));
    if (!w->lt) return fox_fail(FOX_ERR_NOMEM, "weights: layer table");
    for (i = 0; i < (size_t)w->n_layer * FOX_LAYER_ROLES; i++) w->lt[i] = FOX_TENSOR_ABSENT;
    for (i = 0; i < n; i++)
        if (w->layer_of[i] >= 0)
            w->lt[(size_t)w->layer_of[i] * FOX_LAYER_ROLES + w->role_of[i]] = i;
    /* every layer must have the tensors of layer 0, with its types and
     * shapes: a slot holds any layer */
    w->layer_bytes = 0;
    for (l = 0; l < w->n_layer; l++) {
        for (r = 0; r < FOX_LAYER_ROLES; r++) {
            size_t a = w->lt[(size_t)l * FOX_LAYER_ROLES + r], b = w->lt[r];
            const fox_tensor_desc *ta, *tb;
            if (a == FOX_TENSOR_ABSENT || b == FOX_TENSOR_ABSENT)
                return fox_fail(FOX_ERR_NOTFOUND, "weights: the file has no tensor "
                                "'blk.%u.%s.weight'", a == FOX_TENSOR_ABSENT ? l : 0,
                                ROLE_NAME[r]);
            ta = &g->tensors[a];
            tb = &g->tensors[b];
            if (ta->type != tb->type || ta->n_dims != tb->n_dims || ta->ne[0] != tb->ne[0] ||
                ta->ne[1] != tb->ne[1] || ta->size_bytes != tb->size_bytes)
                return fox_fail(FOX_ERR_UNSUPPORTED, "weights: streaming reloads layers in "
                                "place, and '%s' differs from layer 0's in type or shape",
                                ta->name);
            if (l == 0) w->layer_bytes += ta->size_bytes;
        }
    }
    return FOX_OK;
}

static fox_status open_stream(fox_weights *w)
{
    const fox_gguf *g = w->g;
    uint64_t outside = 0;
    size_t i;
    int s, r;
    fox_status st;
    fox_gpu_status gs = FOX_GPU_OK;

    if ((st = map_layers(w)) != FOX_OK) return st;
    for (i = 0; i < g->n_tensors; i++) {
        if (w->layer_of[i] < 0) outside += g->tensors[i].size_bytes;
    }
    /* a layer's tensors at 256-byte aligned places of the staging buffers:
     * each is repacked on the device from its own place */
    w->stage_bytes = 0;
    for (r = 0; r < FOX_LAYER_ROLES; r++) {
        w->stage_off[r] = w->stage_bytes;
        w->stage_bytes += (g->tensors[w->lt[r]].size_bytes + 255) & ~(uint64_t)255;
    }
    if (w->budget == 0) {
        w->n_slots = (int)w->n_layer;
    } else {
        uint64_t fit;
        if (w->budget < outside + 2 * w->layer_bytes)
            return fox_fail(FOX_ERR_NOMEM, "weights: streaming needs the %llu bytes of the "
                            "tensors outside the layers and two %llu-byte layer slots; the "
                            "budget is %llu", (unsigned long long)outside,
                            (unsigned long long)w->layer_bytes, (unsigned long long)w->budget);
        fit = (w->budget - outside) / w->layer_bytes;
        w->n_slots = (int)(fit < w->n_layer ? fit : w->n_layer);
    }
    w->slots = (fox_layer_slot *)calloc((size_t)w->n_slots, sizeof(fox_layer_slot));
    if (!w->slots) return fox_fail(FOX_ERR_NOMEM, "weights: slot table");
    for (s = 0; s < w->n_slots; s++) w->slots[s].layer = -1;
    for (s = 0; s < w->n_slots && gs == FOX_GPU_OK; s++) {
        fox_layer_slot *sl = &w->slots[s];
        for (r = 0; r < FOX_LAYER_ROLES && gs == FOX_GPU_OK; r++) {
            const fox_tensor_desc *t = &g->tensors[w->lt[r]];
            uint64_t rows = 1;
            uint32_t d;
            for (d = 1; d < t->n_dims; d++) rows *= t->ne[d];
            gs = fox_gpu_tensor_alloc(w->gpu, (int)t->type, t->ne[0], rows, &sl->t[r]);
        }
        if (gs == FOX_GPU_OK) gs = fox_gpu_event_create(w->gpu, &sl->ready);
        if (gs == FOX_GPU_OK) gs = fox_gpu_event_create(w->gpu, &sl->used);
    }
    for (i = 0; i < 2 && gs == FOX_GPU_OK; i++) {
        gs = fox_gpu_host_alloc(w->gpu, (size_t)w->stage_bytes, (void **)&w->pinned[i]);
        if (gs == FOX_GPU_OK) gs = fox_gpu_event_create(w->gpu, &w->staged[i]);
    }
    if (gs == FOX_GPU_OK) gs = fox_gpu_malloc(w->gpu, (size_t)w->stage_bytes, &w->dev_stage);
    if (gs != FOX_GPU_OK) return fox_gpu_failed(gs, "weights: streaming buffers");
    return FOX_OK;
}

static void close_stream(fox_weights *w)
{
    int s, r;
    if (w->gpu) fox_gpu_sync(w->gpu);
    for (s = 0; w->slots && s < w->n_slots; s++) {
        for (r = 0; r < FOX_LAYER_ROLES; r++) fox_gpu_tensor_free(w->gpu, w->slots[s].t[r]);
        fox_gpu_event_destroy(w->slots[s].ready);
        fox_gpu_event_destroy(w->slots[s].used);
    }
    for (s = 0; s < 2; s++) {
        if (w->gpu && w->pinned[s]) fox_gpu_host_free(w->gpu, w->pinned[s]);
        fox_gpu_event_destroy(w->staged[s]);
    }
    if (w->gpu && w->dev_stage) fox_gpu_free(w->gpu, w->dev_stage);
    free(w->slots);
    free(w->layer_of);
    free(w->role_of);
    free(w->lt);
}

static fox_layer_slot *slot_of(fox_weights *w, uint32_t l)
{
    int s;
    for (s = 0; s < w->n_slots; s++)
        if (w->slots[s].layer == (int)l) return &w->slots[s];
    return NULL;
}

/* layer l into a slot, started on the copy stream; caller holds the lock */
static fox_status stream_in(fox_weights *w, uint32_t l, fox_layer_slot **out)
{
    fox_layer_slot *sl = slot_of(w, l), *victim = NULL;
    uint8_t *pin;
    fox_gpu_status gs = FOX_GPU_OK;
    fox_status st;
    int s, r, b;

    if (sl) {
        sl->last_used = ++w->clock;
        *out = sl;
        return FOX_OK;
    }
    for (s = 0; s < w->n_slots; s++) {
        fox_layer_slot *c = &w->slots[s];
        if (c->pins) continue;
        if (!victim || c->last_used < victim->last_used) victim = c;
    }
    if (!victim)
        return fox_fail(FOX_ERR_NOMEM, "weights: every one of the %d layer slots holds a live "
                        "lease", w->n_slots);
    /* the pinned buffer of two loads ago is free once its copies are done */
    b = w->next_pin;
    w->next_pin ^= 1;
    if (w->staged_set[b] && (gs = fox_gpu_event_sync(w->staged[b])) != FOX_GPU_OK)
        return fox_gpu_failed(gs, "weights: staging");
    pin = w->pinned[b];
    {
        read_seg seg[FOX_LAYER_ROLES];
        for (r = 0; r < FOX_LAYER_ROLES; r++) {
            const fox_tensor_desc *t = &w->g->tensors[w->lt[(size_t)l * FOX_LAYER_ROLES + r]];
            seg[r].at = w->g->data_offset + t->offset;
            seg[r].size = t->size_bytes;
            seg[r].dst = pin + w->stage_off[r];
        }
        if ((st = read_segments(w, seg, FOX_LAYER_ROLES)) != FOX_OK) return st;
    }
    /* the copy stream overwrites the slot after the compute stream's last
     * queued use of its old layer */
    if (victim->used_set) gs = fox_gpu_event_wait(w->gpu, victim->used, 1);
    /* the layer's bytes in one copy (one long transfer instead of nine),
     * then each tensor repacked from its place in the staging buffer */
    if (gs == FOX_GPU_OK) gs = fox_gpu_stage_async(w->gpu, w->dev_stage, pin, w->stage_bytes);
    for (r = 0; r < FOX_LAYER_ROLES && gs == FOX_GPU_OK; r++) {
        const fox_tensor_desc *t = &w->g->tensors[w->lt[(size_t)l * FOX_LAYER_ROLES + r]];
        gs = fox_gpu_tensor_load_async(w->gpu, victim->t[r], NULL, t->size_bytes,
                                       (uint8_t *)w->dev_stage + w->stage_off[r]);
    }
    if (gs == FOX_GPU_OK) gs = fox_gpu_event_record_copy(w->gpu, w->staged[b]);
    if (gs == FOX_GPU_OK) gs = fox_gpu_event_record_copy(w->gpu, victim->ready);
    if (victim->layer >= 0) {
        w->evictions += FOX_LAYER_ROLES;
        w->held -= w->layer_bytes;
        victim->layer = -1;
    }
    if (gs != FOX_GPU_OK) return fox_gpu_failed(gs, "weights: layer upload");
    w->staged_set[b] = 1;
    victim->layer = (int)l;
    victim->last_used = ++w->clock;
    w->reads += FOX_LAYER_ROLES;
    w->held += w->layer_bytes;
    *out = victim;
    return FOX_OK;
}

fox_status fox_weights_prefetch_layer(fox_weights *w, uint32_t l)
{
    fox_layer_slot *sl;
    fox_status st;
    if (!w || w->mode != FOX_WEIGHTS_STREAM || l >= w->n_layer) return FOX_ERR_ARG;
    pthread_mutex_lock(&w->lock);
    st = stream_in(w, l, &sl);
    pthread_mutex_unlock(&w->lock);
    return st;
}

fox_status fox_weights_use_layer(fox_weights *w, uint32_t l, const fox_gpu_tensor **t)
{
    fox_layer_slot *sl;
    fox_status st;
    int r;
    if (!w || w->mode != FOX_WEIGHTS_STREAM || l >= w->n_layer) return FOX_ERR_ARG;
    pthread_mutex_lock(&w->lock);
    st = stream_in(w, l, &sl);
    if (st == FOX_OK) {
        fox_gpu_status gs = fox_gpu_event_wait(w->gpu, sl->ready, 0);
        if (gs != FOX_GPU_OK) st = fox_gpu_failed(gs, "weights: layer wait");
        for (r = 0; r < FOX_LAYER_ROLES; r++) t[r] = sl->t[r];
    }
    pthread_mutex_unlock(&w->lock);
    return st;
}

void fox_weights_done_layer(fox_weights *w, uint32_t l)
{
    fox_layer_slot *sl;
    if (!w || w->mode != FOX_WEIGHTS_STREAM) return;
    pthread_mutex_lock(&w->lock);
    sl = slot_of(w, l);
    if (sl && fox_gpu_event_record(w->gpu, sl->used) == FOX_GPU_OK) sl->used_set = 1;
    pthread_mutex_unlock(&w->lock);
}

/* ------------------------------------------------------------ open/close */

fox_status fox_weights_open(const char *gguf_path, fox_weights_mode mode,
                            uint64_t budget_bytes, fox_weights **out)
{
    fox_weights *w;
    fox_status st;

    if (!gguf_path || !out) return fox_fail(FOX_ERR_ARG, "weights: null argument");
    *out = NULL;
    if (mode != FOX_WEIGHTS_RESIDENT && mode != FOX_WEIGHTS_DEVICE && mode != FOX_WEIGHTS_STREAM)
        return fox_fail(FOX_ERR_ARG, "weights: unknown mode %d", (int)mode);

    w = (fox_weights *)calloc(1, sizeof(*w));
    if (!w) return fox_fail(FOX_ERR_NOMEM, "weights: handle");
    w->mode = mode;
    w->budget = budget_bytes;
    w->fd = -1;
    st = fox_gguf_open(gguf_path, &w->g);
    if (st != FOX_OK) { free(w); return st; }
    pthread_mutex_init(&w->lock, NULL);
    w->fd = open(gguf_path, O_RDONLY | O_CLOEXEC);
    if (w->fd < 0) {
        fox_weights_close(w);
        return fox_fail(FOX_ERR_IO, "weights: cannot open %s", gguf_path);
    }
    if (mode == FOX_WEIGHTS_RESIDENT)
        w->host = (uint8_t **)calloc(w->g->n_tensors ? w->g->n_tensors : 1, sizeof(uint8_t *));
    else
        w->dev = (fox_gpu_tensor **)calloc(w->g->n_tensors ? w->g->n_tensors : 1,
                                           sizeof(fox_gpu_tensor *));
    if ((mode == FOX_WEIGHTS_RESIDENT && !w->host) || (mode != FOX_WEIGHTS_RESIDENT && !w->dev)) {
        fox_weights_close(w);
        return fox_fail(FOX_ERR_NOMEM, "weights: residency table");
    }
    if (mode != FOX_WEIGHTS_RESIDENT) {
        fox_gpu_status gs = fox_gpu_init(device_ordinal(), &w->gpu);
        const char *mw = getenv("FOX_MAX_WORKGROUPS");
        if (gs != FOX_GPU_OK) {
            st = fox_gpu_failed(gs, "weights: no usable GPU for the device backends");
            fox_weights_close(w);
            return st;
        }
        /* a cap on the fused GEMVs' persistent grid (results unchanged) */
        if (mw && *mw) fox_gpu_set_max_workgroups(w->gpu, atoi(mw));
    }
    if (mode == FOX_WEIGHTS_STREAM && (st = open_stream(w)) != FOX_OK) {
        fox_weights_close(w);
        return st;
    }
    *out = w;
    return FOX_OK;
}

void fox_weights_close(fox_weights *w)
{
    size_t i;
    if (!w) return;
    if (w->live) fox_warn("weights: closing with %zu lease(s) still held", w->live);
    if (w->mode == FOX_WEIGHTS_STREAM) close_stream(w);
    if (w->g) {
        for (i = 0; i < w->g->n_tensors; i++) {
            if (w->host) free(w->host[i]);
            if (w->dev && w->dev[i]) fox_gpu_tensor_free(w->gpu, w->dev[i]);
        }
    }
    free(w->host);
    free(w->dev);
    if (w->gpu) fox_gpu_shutdown(w->gpu);
    if (w->fd >= 0) close(w->fd);
    if (w->g) pthread_mutex_destroy(&w->lock);
    fox_gguf_close(w->g);
    free(w);
}

const fox_gguf *fox_weights_model(const fox_weights *w)
{
    return w ? w->g : NULL;
}

fox_weights_mode fox_weights_get_mode(const fox_weights *w)
{
    return w ? w->mode : FOX_WEIGHTS_RESIDENT;
}

size_t fox_weights_tensor_count(const fox_weights *w) { return w ? w->g->n_tensors : 0; }

size_t fox_weights_tensor_find(const fox_weights *w, const char *name)
{
    return w ? fox_gguf_tensor_find(w->g, name) : FOX_TENSOR_ABSENT;
}

static int streamed(const fox_weights *w, size_t idx)
{
    return w->mode == FOX_WEIGHTS_STREAM && w->layer_of[idx] >= 0;
}

/* load resident tensor idx into its backend; caller holds the lock */
static fox_status load(fox_weights *w, size_t idx)
{
    const fox_tensor_desc *t = &w->g->tensors[idx];
    uint8_t *buf;
    fox_status st;

    if ((w->host && w->host[idx]) || (w->dev && w->dev[idx])) return FOX_OK;
    if (t->size_bytes == 0) return fox_fail(FOX_ERR_FORMAT, "weights: tensor '%s' is empty", t->name);
    if (w->mode != FOX_WEIGHTS_STREAM && w->budget && w->held + t->size_bytes > w->budget)
        return fox_fail(FOX_ERR_NOMEM,
                        "weights: tensor '%s' needs %llu bytes but only %llu of the %llu byte "
                        "budget is left", t->name, (unsigned long long)t->size_bytes,
                        (unsigned long long)(w->budget - w->held), (unsigned long long)w->budget);
    buf = (uint8_t *)aligned_alloc(4096, (t->size_bytes + 4095) / 4096 * 4096);
    if (!buf) return fox_fail(FOX_ERR_NOMEM, "weights: cannot allocate %llu bytes for '%s'",
                              (unsigned long long)t->size_bytes, t->name);
    st = read_bytes(w, t, buf);
    if (st != FOX_OK) { free(buf); return st; }
    w->reads++;
    if (w->mode == FOX_WEIGHTS_RESIDENT) {
        w->host[idx] = buf;
    } else {
        uint64_t ne1 = t->n_dims > 1 ? t->ne[1] : 1;
        uint64_t rest = 1;
        uint32_t d;
        for (d = 2; d < t->n_dims; d++) rest *= t->ne[d];
        fox_gpu_status gs = fox_gpu_tensor_upload(w->gpu, (int)t->type, t->ne[0], ne1 * rest,
                                                  buf, t->size_bytes, &w->dev[idx]);
        free(buf);
        if (gs != FOX_GPU_OK) {
            w->dev[idx] = NULL;
            return fox_gpu_failed(gs, t->name);
        }
    }
    w->held += t->size_bytes;
    return FOX_OK;
}

fox_status fox_weights_use(fox_weights *w, size_t idx, const fox_gpu_tensor **out)
{
    fox_status st;
    if (!w || !out || idx >= w->g->n_tensors || w->mode == FOX_WEIGHTS_RESIDENT)
        return fox_fail(FOX_ERR_ARG, "weights: no device tensor %zu", idx);
    if (streamed(w, idx)) {
        const fox_gpu_tensor *t[FOX_LAYER_ROLES];
        st = fox_weights_use_layer(w, (uint32_t)w->layer_of[idx], t);
        if (st == FOX_OK) *out = t[w->role_of[idx]];
        return st;
    }
    pthread_mutex_lock(&w->lock);
    st = load(w, idx);
    if (st == FOX_OK) *out = w->dev[idx];
    pthread_mutex_unlock(&w->lock);
    return st;
}

fox_status fox_weights_acquire(fox_weights *w, size_t idx, fox_weights_lease *lease)
{
    fox_status st;
    fox_layer_slot *sl = NULL;
    if (!w || !lease) return fox_fail(FOX_ERR_ARG, "weights: null argument");
    if (idx >= w->g->n_tensors)
        return fox_fail(FOX_ERR_NOTFOUND, "weights: no tensor at index %zu", idx);
    pthread_mutex_lock(&w->lock);
    if (w->live >= FOX_WEIGHTS_MAX_LIVE_LEASES) {
        pthread_mutex_unlock(&w->lock);
        return fox_fail(FOX_ERR_INTERNAL, "weights: %d leases already held; release before "
                        "acquiring the next one", FOX_WEIGHTS_MAX_LIVE_LEASES);
    }
    if (streamed(w, idx)) {
        /* the lease holds the slot: its upload is waited for here */
        st = stream_in(w, (uint32_t)w->layer_of[idx], &sl);
        if (st == FOX_OK) {
            fox_gpu_status gs = fox_gpu_event_sync(sl->ready);
            if (gs != FOX_GPU_OK) st = fox_gpu_failed(gs, "weights: layer upload");
        }
        if (st == FOX_OK) {
            sl->pins++;
            lease->data = (const void *)sl->t[w->role_of[idx]];
            lease->slot = sl;
        }
    } else {
        st = load(w, idx);
        if (st == FOX_OK) {
            lease->data = w->mode == FOX_WEIGHTS_RESIDENT ? (const void *)w->host[idx]
                                                          : (const void *)w->dev[idx];
            lease->slot = NULL;
        }
    }
    if (st == FOX_OK) {
        lease->bytes = w->g->tensors[idx].size_bytes;
        lease->tensor_index = idx;
        w->live++;
    }
    pthread_mutex_unlock(&w->lock);
    return st;
}

void fox_weights_release(fox_weights *w, fox_weights_lease *lease)
{
    if (!w || !lease) return;
    pthread_mutex_lock(&w->lock);
    if (w->live == 0) {
        pthread_mutex_unlock(&w->lock);
        fox_warn("weights: release with no lease outstanding");
        return;
    }
    if (lease->slot) {
        fox_layer_slot *sl = (fox_layer_slot *)lease->slot;
        if (sl->pins > 0) sl->pins--;
    }
    w->live--;
    lease->data = NULL;
    lease->bytes = 0;
    lease->slot = NULL;
    pthread_mutex_unlock(&w->lock);
}

fox_status fox_weights_prefetch(fox_weights *w, size_t idx)
{
    fox_status st;
    if (!w) return FOX_ERR_ARG;
    if (idx >= w->g->n_tensors) return FOX_ERR_NOTFOUND;
    pthread_mutex_lock(&w->lock);
    if (streamed(w, idx)) {
        fox_layer_slot *sl;
        st = stream_in(w, (uint32_t)w->layer_of[idx], &sl);
        if (st == FOX_OK && fox_gpu_event_sync(sl->ready) != FOX_GPU_OK)
            st = fox_fail(FOX_ERR_INTERNAL, "weights: layer upload");
    } else {
        st = load(w, idx);
    }
    pthread_mutex_unlock(&w->lock);
    return st;
}

/* FOX_WEIGHTS_STREAM: start the tensor's layer upload without waiting for
 * it; the other backends load synchronously and have nothing to start */
fox_status fox_weights_prefetch_async(fox_weights *w, size_t idx)
{
    if (!w) return FOX_ERR_ARG;
    if (idx >= w->g->n_tensors) return FOX_ERR_NOTFOUND;
    if (!streamed(w, idx)) return FOX_ERR_UNSUPPORTED;
    return fox_weights_prefetch_layer(w, (uint32_t)w->layer_of[idx]);
}

fox_status fox_weights_prefetch_wait(fox_weights *w, size_t idx)
{
    fox_layer_slot *sl;
    fox_status st = FOX_OK;
    if (!w) return FOX_ERR_ARG;
    if (idx >= w->g->n_tensors) return FOX_ERR_NOTFOUND;
    if (!streamed(w, idx)) return FOX_ERR_UNSUPPORTED;
    pthread_mutex_lock(&w->lock);
    sl = slot_of(w, (uint32_t)w->layer_of[idx]);
    if (!sl) st = fox_fail(FOX_ERR_INTERNAL, "weights: no load of '%s' was started",
                           w->g->tensors[idx].name);
    else if (fox_gpu_event_sync(sl->ready) != FOX_GPU_OK)
        st = fox_fail(FOX_ERR_INTERNAL, "weights: layer upload");
    pthread_mutex_unlock(&w->lock);
    return st;
}

size_t fox_weights_live_leases(const fox_weights *w) { return w ? w->live : 0; }
uint64_t fox_weights_resident_bytes(const fox_weights *w) { return w ? w->held : 0; }
uint64_t fox_weights_reads(const fox_weights *w) { return w ? w->reads : 0; }
uint64_t fox_weights_evictions(const fox_weights *w) { return w ? w->evictions : 0; }
