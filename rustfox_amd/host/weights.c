/* weights.c -- the lease API (RustFox include/fox/fox.h:370-403) with two
 * backends: RESIDENT keeps host bytes (src/weights.c:461-496 semantics: a
 * tensor is read on first touch, once); DEVICE keeps each tensor in HBM as a
 * fox_gpu_tensor, read once from the file and uploaded once.  STREAM
 * (storage-streamed slots) is not part of the GPU build.
 *
 * Contract kept from the reference: at most FOX_WEIGHTS_MAX_LIVE_LEASES live
 * leases (src/weights.c:789-797), lease.bytes is the GGUF tensor size,
 * lease.data is borrowed until release and cleared by it (887-890), calls
 * are thread-safe under one lock, fox_weights_reads counts one read per
 * tensor, prefetch_async/_wait report FOX_ERR_UNSUPPORTED without a
 * prefetch thread (722, 750).
 */
#include "fox_host_internal.h"

#include <fcntl.h>
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

fox_status fox_weights_open(const char *gguf_path, fox_weights_mode mode,
                            uint64_t budget_bytes, fox_weights **out)
{
    fox_weights *w;
    fox_status st;

    if (!gguf_path || !out) return fox_fail(FOX_ERR_ARG, "weights: null argument");
    *out = NULL;
    if (mode == FOX_WEIGHTS_STREAM)
        return fox_fail(FOX_ERR_UNSUPPORTED,
                        "weights: streaming from storage is not part of the GPU build; open "
                        "with FOX_WEIGHTS_DEVICE (HBM) or FOX_WEIGHTS_RESIDENT");
    if (mode != FOX_WEIGHTS_RESIDENT && mode != FOX_WEIGHTS_DEVICE)
        return fox_fail(FOX_ERR_ARG, "weights: unknown mode %d", (int)mode);

    w = (fox_weights *)calloc(1, sizeof(*w));
    if (!w) return fox_fail(FOX_ERR_NOMEM, "weights: handle");
    w->mode = mode;
    w->budget = budget_bytes;
    w->fd = -1;
    st = fox_gguf_open(gguf_path, &w->g);
    if (st != FOX_OK) { free(w); return st; }
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
    if ((mode == FOX_WEIGHTS_RESIDENT && !w->host) || (mode == FOX_WEIGHTS_DEVICE && !w->dev)) {
        fox_weights_close(w);
        return fox_fail(FOX_ERR_NOMEM, "weights: residency table");
    }
    if (mode == FOX_WEIGHTS_DEVICE) {
        fox_gpu_status gs = fox_gpu_init(device_ordinal(), &w->gpu);
        const char *mw = getenv("FOX_MAX_WORKGROUPS");
        if (gs != FOX_GPU_OK) {
            st = fox_gpu_failed(gs, "weights: no usable GPU for FOX_WEIGHTS_DEVICE");
            fox_weights_close(w);
            return st;
        }
        /* a cap on the fused GEMVs' persistent grid (results unchanged) */
        if (mw && *mw) fox_gpu_set_max_workgroups(w->gpu, atoi(mw));
    }
    pthread_mutex_init(&w->lock, NULL);
    *out = w;
    return FOX_OK;
}

void fox_weights_close(fox_weights *w)
{
    size_t i;
    if (!w) return;
    if (w->live) fox_warn("weights: closing with %zu lease(s) still held", w->live);
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
    fox_gguf_close(w->g);
    if (w->g) pthread_mutex_destroy(&w->lock);
    free(w);
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

/* load tensor idx into its backend; caller holds the lock */
static fox_status load(fox_weights *w, size_t idx)
{
    const fox_tensor_desc *t = &w->g->tensors[idx];
    uint8_t *buf;
    fox_status st;

    if ((w->host && w->host[idx]) || (w->dev && w->dev[idx])) return FOX_OK;
    if (t->size_bytes == 0) return fox_fail(FOX_ERR_FORMAT, "weights: tensor '%s' is empty", t->name);
    if (w->budget && w->held + t->size_bytes > w->budget)
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

fox_status fox_weights_acquire(fox_weights *w, size_t idx, fox_weights_lease *lease)
{
    fox_status st;
    if (!w || !lease) return fox_fail(FOX_ERR_ARG, "weights: null argument");
    if (idx >= w->g->n_tensors)
        return fox_fail(FOX_ERR_NOTFOUND, "weights: no tensor at index %zu", idx);
    pthread_mutex_lock(&w->lock);
    if (w->live >= FOX_WEIGHTS_MAX_LIVE_LEASES) {
        pthread_mutex_unlock(&w->lock);
        return fox_fail(FOX_ERR_INTERNAL, "weights: %d leases already held; release before "
                        "acquiring the next one", FOX_WEIGHTS_MAX_LIVE_LEASES);
    }
    st = load(w, idx);
    if (st == FOX_OK) {
        lease->data = w->mode == FOX_WEIGHTS_RESIDENT ? (const void *)w->host[idx]
                                                      : (const void *)w->dev[idx];
        lease->bytes = w->g->tensors[idx].size_bytes;
        lease->tensor_index = idx;
        lease->slot = NULL;
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
    st = load(w, idx);
    pthread_mutex_unlock(&w->lock);
    return st;
}

fox_status fox_weights_prefetch_async(fox_weights *w, size_t idx)
{
    if (!w) return FOX_ERR_ARG;
    if (idx >= w->g->n_tensors) return FOX_ERR_NOTFOUND;
    return FOX_ERR_UNSUPPORTED;
}

fox_status fox_weights_prefetch_wait(fox_weights *w, size_t idx)
{
    if (!w) return FOX_ERR_ARG;
    if (idx >= w->g->n_tensors) return FOX_ERR_NOTFOUND;
    return FOX_ERR_UNSUPPORTED;
}

size_t fox_weights_live_leases(const fox_weights *w) { return w ? w->live : 0; }
uint64_t fox_weights_resident_bytes(const fox_weights *w) { return w ? w->held : 0; }
uint64_t fox_weights_reads(const fox_weights *w) { return w ? w->reads : 0; }
uint64_t fox_weights_evictions(const fox_weights *w) { (void)w; return 0; }
