// fox_gpu.hip -- context, errors, memory, weight upload/repack, graphs, events.
#include "fox_internal.h"

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>

// ------------------------------------------------------------------ errors

static thread_local char g_err[512];

fox_gpu_status fox_fail(fox_gpu_status st, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return st;
}

fox_gpu_status fox_hip_fail(hipError_t e, const char *what)
{
    return fox_fail(e == hipErrorOutOfMemory ? FOX_GPU_ERR_NOMEM : FOX_GPU_ERR_INTERNAL,
                    "hip: %s failed: %s", what, hipGetErrorString(e));
}

extern "C" const char *fox_gpu_last_error(void) { return g_err; }

extern "C" const char *fox_gpu_status_str(fox_gpu_status s)
{
    switch (s) {
    case FOX_GPU_OK: return "ok";
    case FOX_GPU_ERR_ARG: return "invalid argument";
    case FOX_GPU_ERR_IO: return "i/o error";
    case FOX_GPU_ERR_NOMEM: return "out of memory";
    case FOX_GPU_ERR_FORMAT: return "bad format";
    case FOX_GPU_ERR_UNSUPPORTED: return "unsupported";
    case FOX_GPU_ERR_NOTFOUND: return "not found";
    case FOX_GPU_ERR_INTERNAL: return "internal error";
    }
    return "unknown status";
}

// ---------------------------------------------------------------- context

static fox_gpu_status set_device(fox_gpu_ctx *ctx)
{
    FOX_HIP(hipSetDevice(ctx->device));
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_init(int device, fox_gpu_ctx **out)
{
    int count = 0;
    hipDeviceProp_t prop;
    fox_gpu_ctx *ctx;

    if (!out) return fox_fail(FOX_GPU_ERR_ARG, "init: null output");
    *out = nullptr;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0)
        return fox_fail(FOX_GPU_ERR_NOTFOUND, "init: no HIP device is visible");
    if (device < 0 || device >= count)
        return fox_fail(FOX_GPU_ERR_ARG, "init: device %d of %d", device, count);
    FOX_HIP(hipSetDevice(device));
    FOX_HIP(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED,
                        "init: device %d is %s; this library is built for gfx950 (MI355X)",
                        device, prop.gcnArchName);
    ctx = new (std::nothrow) fox_gpu_ctx();
    if (!ctx) return fox_fail(FOX_GPU_ERR_NOMEM, "init: context");
    ctx->device = device;
    ctx->n_cu = prop.multiProcessorCount;
    ctx->hbm_bytes = prop.totalGlobalMem;
    snprintf(ctx->name, sizeof(ctx->name), "%s (%s)", prop.name, prop.gcnArchName);
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return fox_fail(FOX_GPU_ERR_INTERNAL, "init: stream creation failed");
    }
    if (hipStreamCreateWithFlags(&ctx->copy, hipStreamNonBlocking) != hipSuccess) {
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return fox_fail(FOX_GPU_ERR_INTERNAL, "init: copy stream creation failed");
    }
    fox_gpu_status st = fox_ws_reserve(ctx, 8u << 20);
    if (st != FOX_GPU_OK) {
        fox_gpu_shutdown(ctx);
        return st;
    }
    if (hipMalloc(&ctx->small, FOX_SMALL_BYTES) != hipSuccess ||
        hipMemset(ctx->small, 0, FOX_SMALL_BYTES) != hipSuccess) {
        fox_gpu_shutdown(ctx);
        return fox_fail(FOX_GPU_ERR_NOMEM, "init: small buffer");
    }
    if ((st = fox_scratch_init(ctx)) != FOX_GPU_OK) {   // (device `device` is current)
        fox_gpu_shutdown(ctx);
        return st;
    }
    *out = ctx;
    return FOX_GPU_OK;
}

extern "C" void fox_gpu_shutdown(fox_gpu_ctx *ctx)
{
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) {
        (void)hipStreamSynchronize(ctx->stream);
        (void)hipStreamDestroy(ctx->stream);
    }
    if (ctx->copy) {
        (void)hipStreamSynchronize(ctx->copy);
        (void)hipStreamDestroy(ctx->copy);
    }
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->small) (void)hipFree(ctx->small);
    for (int i = 0; i < ctx->n_retired; i++) (void)hipFree(ctx->retired[i]);
    delete ctx;
}

extern "C" fox_gpu_status fox_gpu_set_max_workgroups(fox_gpu_ctx *ctx, int n)
{
    if (!ctx || n < 0) return fox_fail(FOX_GPU_ERR_ARG, "set_max_workgroups: bad argument");
    ctx->max_wg = n;
    return FOX_GPU_OK;
}

extern "C" size_t fox_gpu_workspace_bytes(const fox_gpu_ctx *ctx)
{
    return ctx ? ctx->ws_cap : 0;
}

extern "C" fox_gpu_status fox_gpu_device_info(fox_gpu_ctx *ctx, char *name, size_t cap,
                                              int *compute_units, uint64_t *hbm_bytes)
{
    if (!ctx) return fox_fail(FOX_GPU_ERR_ARG, "device_info: null context");
    if (name && cap) snprintf(name, cap, "%s", ctx->name);
    if (compute_units) *compute_units = ctx->n_cu;
    if (hbm_bytes) *hbm_bytes = ctx->hbm_bytes;
    return FOX_GPU_OK;
}

fox_gpu_status fox_ws_reserve(fox_gpu_ctx *ctx, size_t bytes)
{
    if (bytes <= ctx->ws_cap) return FOX_GPU_OK;
    if (ctx->capturing)
        return fox_fail(FOX_GPU_ERR_NOMEM,
                        "workspace: %zu bytes needed but only %zu are reserved, and "
                        "memory cannot be allocated during graph capture; run the same "
                        "calls once before capturing",
                        bytes, ctx->ws_cap);
    size_t cap = ctx->ws_cap ? ctx->ws_cap : (1u << 20);
    while (cap < bytes) cap *= 2;
    uint8_t *fresh = nullptr;
    FOX_HIP(hipMalloc(&fresh, cap));
    if (ctx->ws) {
        if (ctx->n_retired == (int)(sizeof(ctx->retired) / sizeof(ctx->retired[0]))) {
            (void)hipFree(fresh);
            return fox_fail(FOX_GPU_ERR_NOMEM, "workspace: grown too many times");
        }
        ctx->retired[ctx->n_retired++] = ctx->ws;
    }
    ctx->ws = fresh;
    ctx->ws_cap = cap;
    return FOX_GPU_OK;
}

// ----------------------------------------------------------------- memory

extern "C" fox_gpu_status fox_gpu_malloc(fox_gpu_ctx *ctx, size_t bytes, void **out)
{
    if (!ctx || !out || bytes == 0) return fox_fail(FOX_GPU_ERR_ARG, "malloc: bad argument");
    fox_gpu_status st = set_device(ctx);
    if (st) return st;
    hipError_t e = hipMalloc(out, bytes);
    if (e != hipSuccess) {
        *out = nullptr;
        return fox_fail(FOX_GPU_ERR_NOMEM, "malloc: %zu bytes: %s", bytes, hipGetErrorString(e));
    }
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_free(fox_gpu_ctx *ctx, void *ptr)
{
    if (!ctx) return fox_fail(FOX_GPU_ERR_ARG, "free: null context");
    if (!ptr) return FOX_GPU_OK;
    FOX_HIP(hipFree(ptr));
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_memcpy_h2d(fox_gpu_ctx *ctx, void *dst, const void *src, size_t n)
{
    if (!ctx || (!dst && n) || (!src && n)) return fox_fail(FOX_GPU_ERR_ARG, "memcpy_h2d: null pointer");
    if (!n) return FOX_GPU_OK;
    FOX_HIP(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, ctx->stream));
    FOX_HIP(hipStreamSynchronize(ctx->stream));
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_memcpy_d2h(fox_gpu_ctx *ctx, void *dst, const void *src, size_t n)
{
    if (!ctx || (!dst && n) || (!src && n)) return fox_fail(FOX_GPU_ERR_ARG, "memcpy_d2h: null pointer");
    if (!n) return FOX_GPU_OK;
    FOX_HIP(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, ctx->stream));
    FOX_HIP(hipStreamSynchronize(ctx->stream));
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_memcpy_d2d(fox_gpu_ctx *ctx, void *dst, const void *src, size_t n)
{
    if (!ctx || (!dst && n) || (!src && n)) return fox_fail(FOX_GPU_ERR_ARG, "memcpy_d2d: null pointer");
    if (!n) return FOX_GPU_OK;
    FOX_HIP(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, ctx->stream));
    return FOX_GPU_OK;
}

__global__ void fill_bytes(uint8_t *dst, uint8_t v, size_t n)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t step = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += step) dst[i] = v;
}

extern "C" fox_gpu_status fox_gpu_memset(fox_gpu_ctx *ctx, void *dst, int value, size_t n)
{
    if (!ctx || (!dst && n)) return fox_fail(FOX_GPU_ERR_ARG, "memset: null pointer");
    if (!n) return FOX_GPU_OK;
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(fill_bytes, dim3((unsigned)blocks), dim3(256), 0, ctx->stream,
                       (uint8_t *)dst, (uint8_t)value, n);
    FOX_LAUNCHED("memset");
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_sync(fox_gpu_ctx *ctx)
{
    if (!ctx) return fox_fail(FOX_GPU_ERR_ARG, "sync: null context");
    FOX_HIP(hipStreamSynchronize(ctx->stream));
    return FOX_GPU_OK;
}

// ------------------------------------------------------- weight repacking

// Position of byte `o` of a device chunk in the GGUF block of tile row i:
// returns the byte offset k inside that row's block and sets *row.
__device__ __forceinline__ int chunk_source(int type, int o, int *row)
{
    int L, e;
    switch (type) {
    case FOX_GPU_TQ2_0:
        if (o < 1024) { L = o >> 4; e = o & 15; *row = L & 15; return 16 * (L >> 4) + e; }
        *row = (o - 1024) >> 1;
        return 64 + ((o - 1024) & 1);
    case FOX_GPU_Q4_K:
        if (o < 2048) {
            L = o >> 5; e = o & 31; *row = L & 15;
            return 16 + 32 * (e >> 3) + 8 * (L >> 4) + (e & 7);
        }
        *row = (o - 2048) >> 4;
        return (o - 2048) & 15;
    case FOX_GPU_Q6_K:
        if (o < 2048) { *row = o >> 7; return o & 127; }
        if (o < 3072) { *row = (o - 2048) >> 6; return 128 + ((o - 2048) & 63); }
        if (o < 3328) { *row = (o - 3072) >> 4; return 192 + ((o - 3072) & 15); }
        *row = (o - 3328) >> 1;
        return 208 + ((o - 3328) & 1);
    }
    *row = 0;
    return 0;
}

// TQ1_0 <-> the TQ2_0 blocks TQ1_0 tensors are held as.  Element i of a
// TQ1_0 block (src/ternary.c:73-93: bytes 0..31 carry elements l*32 + m at
// level l, bytes 32..47 elements 160 + l*16 + m, the qh bytes 48..51
// elements 240 + l*4 + m) has the trit ((uint8)(b * 3^l) * 3) >> 8
// (src/ternary.c:59-63, before its - 1); element i of a TQ2_0 block
// (src/ternary.c:177-188) is the 2-bit field 2 ((i % 128) / 32) of byte
// (i / 128) * 32 + i % 32 (code - 1 likewise).  The f16 scale moves from
// bytes 52..53 to 64..65.

__device__ __forceinline__ int pow3(int l)
{
    int p = 1;
    for (int k = 0; k < l; k++) p *= 3;
    return p;
}

// the trit of element i of a TQ1_0 block
__device__ __forceinline__ int tq1_trit(const uint8_t *blk, int i)
{
    int byte, level;
    if (i < 160) {
        byte = i & 31;
        level = i >> 5;
    } else if (i < 240) {
        byte = 32 + ((i - 160) & 15);
        level = (i - 160) >> 4;
    } else {
        byte = 48 + ((i - 240) & 3);
        level = (i - 240) >> 2;
    }
    const uint8_t q = (uint8_t)(blk[byte] * pow3(level));
    return (int)(((unsigned)q * 3u) >> 8);
}

// the code of element i of a TQ2_0 block
__device__ __forceinline__ int tq2_code(const uint8_t *blk, int i)
{
    return (blk[(i >> 7) * 32 + (i & 31)] >> (2 * ((i & 127) >> 5))) & 3;
}

// total = blocks * 66: one output byte per step
__global__ void tq1_to_tq2(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                           uint64_t total)
{
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t step = (uint64_t)gridDim.x * blockDim.x;
    for (; i < total; i += step) {
        const uint64_t blk = i / 66;
        const int j = (int)(i - blk * 66);
        const uint8_t *s = src + blk * 54;
        if (j < 64) {
            const int h = j >> 5, m = j & 31;
            int v = 0;
            for (int l = 0; l < 4; l++) v |= tq1_trit(s, h * 128 + l * 32 + m) << (2 * l);
            dst[i] = (uint8_t)v;
        } else {
            dst[i] = s[52 + (j - 64)];
        }
    }
}

// total = blocks * 54: one output byte per step.  A byte carrying the
// digits q = sum_l t_l 3^(4 - l) is written as ceil(q * 256 / 243), the
// encoding the reference's quantiser writes (a qh byte's four digits with a
// fifth digit 0); any byte decoding to the same trits gives the same
// results, this one is the canonical byte.
__global__ void tq2_to_tq1(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                           uint64_t total)
{
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t step = (uint64_t)gridDim.x * blockDim.x;
    for (; i < total; i += step) {
        const uint64_t blk = i / 54;
        const int k = (int)(i - blk * 54);
        const uint8_t *s = src + blk * 66;
        if (k >= 52) {
            dst[i] = s[64 + (k - 52)];
            continue;
        }
        int q = 0;
        if (k < 32) {
            for (int l = 0; l < 5; l++) q = 3 * q + tq2_code(s, l * 32 + k);
        } else if (k < 48) {
            for (int l = 0; l < 5; l++) q = 3 * q + tq2_code(s, 160 + l * 16 + (k - 32));
        } else {
            for (int l = 0; l < 4; l++) q = 3 * q + tq2_code(s, 240 + l * 4 + (k - 48));
            q *= 3;
        }
        dst[i] = (uint8_t)((q * 256 + 242) / 243);
    }
}

// TQ1_0 GGUF bytes straight into the device chunk layout of the TQ2_0
// blocks they are held as (tq1_to_tq2 and repack_blocks in one pass): byte
// o of chunk c is byte k of the TQ2_0 block of tile row r (chunk_source),
// built from the trits of the TQ1_0 block.
__global__ void repack_tq1(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                           uint64_t n_rows, uint64_t nb, uint64_t total)
{
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t c = i / TQ2_CHUNK;
        const int o = (int)(i - c * TQ2_CHUNK);
        const uint64_t tile = c / nb, b = c - tile * nb;
        int r;
        const int k = chunk_source(FOX_GPU_TQ2_0, o, &r);
        const uint64_t row = tile * FOX_TILE + (uint64_t)r;
        if (row >= n_rows) {
            dst[i] = 0;
            continue;
        }
        const uint8_t *s = src + (row * nb + b) * 54;
        if (k < 64) {
            const int h = k >> 5, m = k & 31;
            int v = 0;
            for (int l = 0; l < 4; l++) v |= tq1_trit(s, h * 128 + l * 32 + m) << (2 * l);
            dst[i] = (uint8_t)v;
        } else {
            dst[i] = s[52 + (k - 64)];
        }
    }
}

// dir 0: GGUF bytes (src) -> device layout (dst); dir 1: the inverse.
__global__ void repack_blocks(int type, int dir, const uint8_t *src, uint8_t *dst,
                              uint64_t n_rows, uint64_t nb, uint64_t chunk,
                              uint64_t blk_bytes, uint64_t total)
{
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint64_t step = (uint64_t)gridDim.x * blockDim.x;
    for (; i < total; i += step) {
        uint64_t c = i / chunk;
        int o = (int)(i - c * chunk);
        uint64_t tile = c / nb, b = c - tile * nb;
        int r;
        int k = chunk_source(type, o, &r);
        uint64_t row = tile * FOX_TILE + (uint64_t)r;
        uint64_t g = (row * nb + b) * blk_bytes + (uint64_t)k;
        if (dir == 0) {
            dst[i] = row < n_rows ? src[g] : 0;
        } else if (row < n_rows) {
            dst[g] = src[i];
        }
    }
}

// float tensors, one element per step. dir 0: row-major (src) -> tiles (dst),
// padding zero; dir 1: tiles (src) -> row-major (dst).
template <typename T>
__global__ void repack_float(int dir, const T *src, T *dst, uint64_t n_rows, uint64_t K,
                             uint64_t total)
{
    const uint64_t per = FOX_FCHUNK / sizeof(T), nchunk = (K + per - 1) / per;
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t step = (uint64_t)gridDim.x * blockDim.x;
    for (; i < total; i += step) {
        if (dir == 0) {
            // i: element of the tiled layout
            const uint64_t e = i % per, rest = i / per;
            const uint64_t ri = rest % FOX_FTILE, rest2 = rest / FOX_FTILE;
            const uint64_t c = rest2 % nchunk, tile = rest2 / nchunk;
            const uint64_t r = tile * FOX_FTILE + ri, k = c * per + e;
            dst[i] = (r < n_rows && k < K) ? src[r * K + k] : (T)0;
        } else {
            // i: element of the row-major layout
            const uint64_t r = i / K, k = i % K;
            dst[i] = src[fox_float_offset(r, k, K, sizeof(T)) / sizeof(T)];
        }
    }
}

static unsigned grid_for(uint64_t n, unsigned block)
{
    uint64_t g = (n + block - 1) / block;
    return (unsigned)(g > 65536 ? 65536 : g);
}

extern "C" fox_gpu_status fox_gpu_tensor_upload(fox_gpu_ctx *ctx, int type, uint64_t ne0,
                                                uint64_t ne1, const void *host, uint64_t bytes,
                                                fox_gpu_tensor **out)
{
    size_t be = fox_block_elems(type), bb = fox_block_bytes(type);
    uint64_t rows = ne1 ? ne1 : 1, want;
    fox_gpu_tensor *t;
    fox_gpu_status st;

    if (!ctx || !host || !out || ne0 == 0)
        return fox_fail(FOX_GPU_ERR_ARG, "tensor_upload: bad argument");
    *out = nullptr;
    if (!be)
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED,
                        "tensor_upload: no device layout for ggml type %d; the device "
                        "path handles F32, F16, Q4_K, Q6_K, TQ1_0 and TQ2_0", type);
    if (ne0 % be)
        return fox_fail(FOX_GPU_ERR_ARG,
                        "tensor_upload: %llu columns is not a whole number of %s blocks",
                        (unsigned long long)ne0, fox_type_name(type));
    want = rows * (ne0 / be) * bb;
    if (bytes != want)
        return fox_fail(FOX_GPU_ERR_ARG,
                        "tensor_upload: %s %llux%llu is %llu bytes, %llu were given",
                        fox_type_name(type), (unsigned long long)ne0, (unsigned long long)rows,
                        (unsigned long long)want, (unsigned long long)bytes);
    if ((st = set_device(ctx))) return st;

    t = new (std::nothrow) fox_gpu_tensor();
    if (!t) return fox_fail(FOX_GPU_ERR_NOMEM, "tensor_upload: handle");
    t->type = type;
    t->ne0 = ne0;
    t->ne1 = rows;
    t->gguf_bytes = bytes;

    if (!fox_is_block_type(type)) {
        const uint64_t es = bb, per = FOX_FCHUNK / es, nchunk = (ne0 + per - 1) / per;
        t->n_tiles = (rows + FOX_FTILE - 1) / FOX_FTILE;
        t->dev_bytes = t->n_tiles * nchunk * FOX_FTILE * FOX_FCHUNK;
        uint8_t *stage = nullptr;
        if (hipMalloc(&t->d, t->dev_bytes) != hipSuccess) {
            delete t;
            return fox_fail(FOX_GPU_ERR_NOMEM, "tensor_upload: %llu bytes of HBM",
                            (unsigned long long)t->dev_bytes);
        }
        if (hipMalloc(&stage, bytes) != hipSuccess) {
            fox_gpu_tensor_free(ctx, t);
            return fox_fail(FOX_GPU_ERR_NOMEM, "tensor_upload: %llu bytes of staging",
                            (unsigned long long)bytes);
        }
        st = fox_gpu_memcpy_h2d(ctx, stage, host, bytes);
        if (!st) {
            const uint64_t n = t->dev_bytes / es;
            if (es == 2)
                hipLaunchKernelGGL(repack_float<uint16_t>, dim3(grid_for(n, 256)), dim3(256), 0,
                                   ctx->stream, 0, (const uint16_t *)stage, (uint16_t *)t->d,
                                   rows, ne0, n);
            else
                hipLaunchKernelGGL(repack_float<uint32_t>, dim3(grid_for(n, 256)), dim3(256), 0,
                                   ctx->stream, 0, (const uint32_t *)stage, (uint32_t *)t->d,
                                   rows, ne0, n);
            hipError_t e = hipGetLastError();
            if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
            if (e != hipSuccess) st = fox_hip_fail(e, "tensor_upload: repack");
        }
        (void)hipFree(stage);
        if (st) {
            fox_gpu_tensor_free(ctx, t);
            return st;
        }
        *out = t;
        return FOX_GPU_OK;
    }

    uint64_t nb = ne0 / 256, chunk = fox_chunk_bytes(type);
    t->n_tiles = (rows + FOX_TILE - 1) / FOX_TILE;
    t->dev_bytes = t->n_tiles * nb * chunk;
    uint8_t *stage = nullptr;
    if (hipMalloc(&t->d, t->dev_bytes) != hipSuccess) {
        delete t;
        return fox_fail(FOX_GPU_ERR_NOMEM, "tensor_upload: %llu bytes of HBM",
                        (unsigned long long)t->dev_bytes);
    }
    if (hipMalloc(&stage, bytes) != hipSuccess) {
        fox_gpu_tensor_free(ctx, t);
        return fox_fail(FOX_GPU_ERR_NOMEM, "tensor_upload: %llu bytes of staging",
                        (unsigned long long)bytes);
    }
    st = fox_gpu_memcpy_h2d(ctx, stage, host, bytes);
    const int dt = fox_device_type(type);
    const uint8_t *src = stage;
    uint64_t src_bb = bb;
    uint8_t *stage2 = nullptr;
    if (!st && dt != type) {
        // TQ1_0: the same trits as TQ2_0 blocks first
        src_bb = fox_block_bytes(dt);
        const uint64_t n2 = rows * nb * src_bb;
        if (hipMalloc(&stage2, n2) != hipSuccess) {
            st = fox_fail(FOX_GPU_ERR_NOMEM, "tensor_upload: %llu bytes of staging",
                          (unsigned long long)n2);
        } else {
            hipLaunchKernelGGL(tq1_to_tq2, dim3(grid_for(n2, 256)), dim3(256), 0, ctx->stream,
                               stage, stage2, n2);
            src = stage2;
        }
    }
    if (!st) {
        hipLaunchKernelGGL(repack_blocks, dim3(grid_for(t->dev_bytes, 256)), dim3(256), 0,
                           ctx->stream, dt, 0, src, t->d, rows, nb, chunk, src_bb,
                           t->dev_bytes);
        hipError_t e = hipGetLastError();
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) st = fox_hip_fail(e, "tensor_upload: repack");
    }
    (void)hipFree(stage2);
    (void)hipFree(stage);
    if (st) {
        fox_gpu_tensor_free(ctx, t);
        return st;
    }
    *out = t;
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_tensor_info(const fox_gpu_tensor *t, int *type, uint64_t *ne0,
                                              uint64_t *ne1, uint64_t *gguf_bytes,
                                              uint64_t *device_bytes)
{
    if (!t) return fox_fail(FOX_GPU_ERR_ARG, "tensor_info: null tensor");
    if (type) *type = t->type;
    if (ne0) *ne0 = t->ne0;
    if (ne1) *ne1 = t->ne1;
    if (gguf_bytes) *gguf_bytes = t->gguf_bytes;
    if (device_bytes) *device_bytes = t->dev_bytes;
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_tensor_download(fox_gpu_ctx *ctx, const fox_gpu_tensor *t,
                                                  void *host, uint64_t bytes)
{
    fox_gpu_status st;
    if (!ctx || !t || !host) return fox_fail(FOX_GPU_ERR_ARG, "tensor_download: bad argument");
    if (bytes != t->gguf_bytes)
        return fox_fail(FOX_GPU_ERR_ARG, "tensor_download: tensor holds %llu bytes, %llu asked",
                        (unsigned long long)t->gguf_bytes, (unsigned long long)bytes);
    if ((st = set_device(ctx))) return st;
    uint8_t *stage = nullptr;
    if (hipMalloc(&stage, bytes) != hipSuccess)
        return fox_fail(FOX_GPU_ERR_NOMEM, "tensor_download: staging");
    if (!fox_is_block_type(t->type)) {
        const uint64_t es = fox_block_bytes(t->type), n = bytes / es;
        if (es == 2)
            hipLaunchKernelGGL(repack_float<uint16_t>, dim3(grid_for(n, 256)), dim3(256), 0,
                               ctx->stream, 1, (const uint16_t *)t->d, (uint16_t *)stage, t->ne1,
                               t->ne0, n);
        else
            hipLaunchKernelGGL(repack_float<uint32_t>, dim3(grid_for(n, 256)), dim3(256), 0,
                               ctx->stream, 1, (const uint32_t *)t->d, (uint32_t *)stage, t->ne1,
                               t->ne0, n);
        hipError_t e = hipGetLastError();
        st = e == hipSuccess ? fox_gpu_memcpy_d2h(ctx, host, stage, bytes)
                             : fox_hip_fail(e, "tensor_download: unpack");
        (void)hipFree(stage);
        return st;
    }
    uint64_t nb = t->ne0 / 256;
    const int dt = fox_device_type(t->type);
    const uint64_t dbb = fox_block_bytes(dt), n2 = t->ne1 * nb * dbb;
    uint8_t *stage2 = nullptr;
    if (dt != t->type && hipMalloc(&stage2, n2) != hipSuccess) {
        (void)hipFree(stage);
        return fox_fail(FOX_GPU_ERR_NOMEM, "tensor_download: staging");
    }
    hipLaunchKernelGGL(repack_blocks, dim3(grid_for(t->dev_bytes, 256)), dim3(256), 0,
                       ctx->stream, dt, 1, t->d, stage2 ? stage2 : stage, t->ne1, nb,
                       (uint64_t)fox_chunk_bytes(dt), dbb, t->dev_bytes);
    if (stage2)   // TQ1_0: back from the TQ2_0 blocks it is held as
        hipLaunchKernelGGL(tq2_to_tq1, dim3(grid_for(bytes, 256)), dim3(256), 0, ctx->stream,
                           stage2, stage, (uint64_t)bytes);
    hipError_t e = hipGetLastError();
    st = e == hipSuccess ? fox_gpu_memcpy_d2h(ctx, host, stage, bytes)
                         : fox_hip_fail(e, "tensor_download: unpack");
    (void)hipFree(stage2);
    (void)hipFree(stage);
    return st;
}

extern "C" void fox_gpu_tensor_free(fox_gpu_ctx *ctx, fox_gpu_tensor *t)
{
    if (!t) return;
    if (ctx) (void)hipSetDevice(ctx->device);
    if (t->d) (void)hipFree(t->d);
    delete t;
}

// ------------------------------------------------------ streamed weights

static fox_gpu_status tensor_shape(int type, uint64_t ne0, uint64_t ne1, fox_gpu_tensor *t)
{
    const size_t be = fox_block_elems(type), bb = fox_block_bytes(type);
    if (!be)
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "tensor: no device layout for ggml type %d",
                        type);
    if (ne0 == 0 || ne0 % be)
        return fox_fail(FOX_GPU_ERR_ARG, "tensor: %llu columns is not a whole number of %s "
                        "blocks", (unsigned long long)ne0, fox_type_name(type));
    t->type = type;
    t->ne0 = ne0;
    t->ne1 = ne1 ? ne1 : 1;
    t->gguf_bytes = t->ne1 * (ne0 / be) * bb;
    if (fox_is_block_type(type)) {
        t->n_tiles = (t->ne1 + FOX_TILE - 1) / FOX_TILE;
        t->dev_bytes = t->n_tiles * (ne0 / 256) * fox_chunk_bytes(type);
    } else {
        const uint64_t per = FOX_FCHUNK / bb, nchunk = (ne0 + per - 1) / per;
        t->n_tiles = (t->ne1 + FOX_FTILE - 1) / FOX_FTILE;
        t->dev_bytes = t->n_tiles * nchunk * FOX_FTILE * FOX_FCHUNK;
    }
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_tensor_alloc(fox_gpu_ctx *ctx, int type, uint64_t ne0,
                                               uint64_t ne1, fox_gpu_tensor **out)
{
    if (!ctx || !out) return fox_fail(FOX_GPU_ERR_ARG, "tensor_alloc: bad argument");
    *out = nullptr;
    fox_gpu_tensor *t = new (std::nothrow) fox_gpu_tensor();
    if (!t) return fox_fail(FOX_GPU_ERR_NOMEM, "tensor_alloc: handle");
    fox_gpu_status st = tensor_shape(type, ne0, ne1, t);
    if (st == FOX_GPU_OK) st = set_device(ctx);
    if (st == FOX_GPU_OK && hipMalloc(&t->d, t->dev_bytes) != hipSuccess)
        st = fox_fail(FOX_GPU_ERR_NOMEM, "tensor_alloc: %llu bytes of HBM",
                      (unsigned long long)t->dev_bytes);
    if (st) {
        delete t;
        return st;
    }
    *out = t;
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_tensor_load_async(fox_gpu_ctx *ctx, fox_gpu_tensor *t,
                                                    const void *host, uint64_t bytes,
                                                    void *dev_stage)
{
    if (!ctx || !t || !dev_stage)
        return fox_fail(FOX_GPU_ERR_ARG, "tensor_load_async: bad argument");
    if (bytes != t->gguf_bytes)
        return fox_fail(FOX_GPU_ERR_ARG, "tensor_load_async: %s %llux%llu is %llu bytes, %llu "
                        "were given", fox_type_name(t->type), (unsigned long long)t->ne0,
                        (unsigned long long)t->ne1, (unsigned long long)t->gguf_bytes,
                        (unsigned long long)bytes);
    if (host) FOX_HIP(hipMemcpyAsync(dev_stage, host, bytes, hipMemcpyHostToDevice, ctx->copy));
    const uint8_t *src = (const uint8_t *)dev_stage;
    if (!fox_is_block_type(t->type)) {
        const uint64_t es = fox_block_bytes(t->type), n = t->dev_bytes / es;
        if (es == 2)
            hipLaunchKernelGGL(repack_float<uint16_t>, dim3(grid_for(n, 256)), dim3(256), 0,
                               ctx->copy, 0, (const uint16_t *)src, (uint16_t *)t->d, t->ne1,
                               t->ne0, n);
        else
            hipLaunchKernelGGL(repack_float<uint32_t>, dim3(grid_for(n, 256)), dim3(256), 0,
                               ctx->copy, 0, (const uint32_t *)src, (uint32_t *)t->d, t->ne1,
                               t->ne0, n);
    } else if (t->type == FOX_GPU_TQ1_0) {
        hipLaunchKernelGGL(repack_tq1, dim3(grid_for(t->dev_bytes, 256)), dim3(256), 0,
                           ctx->copy, src, t->d, t->ne1, t->ne0 / 256, t->dev_bytes);
    } else {
        hipLaunchKernelGGL(repack_blocks, dim3(grid_for(t->dev_bytes, 256)), dim3(256), 0,
                           ctx->copy, t->type, 0, src, t->d, t->ne1, t->ne0 / 256,
                           (uint64_t)fox_chunk_bytes(t->type), (uint64_t)fox_block_bytes(t->type),
                           t->dev_bytes);
    }
    FOX_LAUNCHED("tensor_load_async");
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_stage_async(fox_gpu_ctx *ctx, void *dev, const void *host,
                                              uint64_t bytes)
{
    if (!ctx || !dev || !host) return fox_fail(FOX_GPU_ERR_ARG, "stage_async: bad argument");
    if (bytes == 0) return FOX_GPU_OK;
    FOX_HIP(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, ctx->copy));
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_host_alloc(fox_gpu_ctx *ctx, size_t bytes, void **out)
{
    if (!ctx || !out || bytes == 0) return fox_fail(FOX_GPU_ERR_ARG, "host_alloc: bad argument");
    *out = nullptr;
    fox_gpu_status st = set_device(ctx);
    if (st) return st;
    if (hipHostMalloc(out, bytes, hipHostMallocDefault) != hipSuccess) {
        *out = nullptr;
        return fox_fail(FOX_GPU_ERR_NOMEM, "host_alloc: %zu bytes of pinned host memory", bytes);
    }
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_host_free(fox_gpu_ctx *ctx, void *p)
{
    if (!ctx) return fox_fail(FOX_GPU_ERR_ARG, "host_free: null context");
    if (p) FOX_HIP(hipHostFree(p));
    return FOX_GPU_OK;
}

// ----------------------------------------------------------------- graphs

extern "C" fox_gpu_status fox_gpu_graph_begin(fox_gpu_ctx *ctx)
{
    if (!ctx) return fox_fail(FOX_GPU_ERR_ARG, "graph_begin: null context");
    if (ctx->capturing) return fox_fail(FOX_GPU_ERR_ARG, "graph_begin: already capturing");
    FOX_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = 1;
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_graph_end(fox_gpu_ctx *ctx, fox_gpu_graph **out)
{
    hipGraph_t graph = nullptr;
    if (!ctx || !out) return fox_fail(FOX_GPU_ERR_ARG, "graph_end: bad argument");
    if (!ctx->capturing) return fox_fail(FOX_GPU_ERR_ARG, "graph_end: not capturing");
    ctx->capturing = 0;
    FOX_HIP(hipStreamEndCapture(ctx->stream, &graph));
    fox_gpu_graph *g = new (std::nothrow) fox_gpu_graph();
    if (!g) {
        (void)hipGraphDestroy(graph);
        return fox_fail(FOX_GPU_ERR_NOMEM, "graph_end: handle");
    }
    g->graph = graph;
    hipError_t e = hipGraphInstantiate(&g->exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        delete g;
        return fox_hip_fail(e, "graph_end: instantiate");
    }
    *out = g;
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_graph_launch(fox_gpu_ctx *ctx, fox_gpu_graph *g)
{
    if (!ctx || !g) return fox_fail(FOX_GPU_ERR_ARG, "graph_launch: bad argument");
    FOX_HIP(hipGraphLaunch(g->exec, ctx->stream));
    return FOX_GPU_OK;
}

extern "C" void fox_gpu_graph_free(fox_gpu_graph *g)
{
    if (!g) return;
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
}

// ----------------------------------------------------------------- events

extern "C" fox_gpu_status fox_gpu_event_create(fox_gpu_ctx *ctx, fox_gpu_event **out)
{
    if (!ctx || !out) return fox_fail(FOX_GPU_ERR_ARG, "event_create: bad argument");
    fox_gpu_event *e = new (std::nothrow) fox_gpu_event();
    if (!e) return fox_fail(FOX_GPU_ERR_NOMEM, "event_create: handle");
    hipError_t r = hipEventCreate(&e->ev);
    if (r != hipSuccess) {
        delete e;
        return fox_hip_fail(r, "event_create");
    }
    *out = e;
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_event_record(fox_gpu_ctx *ctx, fox_gpu_event *e)
{
    if (!ctx || !e) return fox_fail(FOX_GPU_ERR_ARG, "event_record: bad argument");
    FOX_HIP(hipEventRecord(e->ev, ctx->stream));
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_event_record_copy(fox_gpu_ctx *ctx, fox_gpu_event *e)
{
    if (!ctx || !e) return fox_fail(FOX_GPU_ERR_ARG, "event_record_copy: bad argument");
    FOX_HIP(hipEventRecord(e->ev, ctx->copy));
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_event_wait(fox_gpu_ctx *ctx, fox_gpu_event *e, int on_copy)
{
    if (!ctx || !e) return fox_fail(FOX_GPU_ERR_ARG, "event_wait: bad argument");
    FOX_HIP(hipStreamWaitEvent(on_copy ? ctx->copy : ctx->stream, e->ev, 0));
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_event_sync(fox_gpu_event *e)
{
    if (!e) return fox_fail(FOX_GPU_ERR_ARG, "event_sync: null event");
    FOX_HIP(hipEventSynchronize(e->ev));
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_event_elapsed(fox_gpu_event *start, fox_gpu_event *stop,
                                                float *ms)
{
    if (!start || !stop || !ms) return fox_fail(FOX_GPU_ERR_ARG, "event_elapsed: bad argument");
    FOX_HIP(hipEventSynchronize(stop->ev));
    FOX_HIP(hipEventElapsedTime(ms, start->ev, stop->ev));
    return FOX_GPU_OK;
}

extern "C" void fox_gpu_event_destroy(fox_gpu_event *e)
{
    if (!e) return;
    (void)hipEventDestroy(e->ev);
    delete e;
}
