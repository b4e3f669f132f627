// fox_internal.h -- shared definitions of the gfx950 decode library.
//
// Device weight layouts.  Rows are grouped in tiles of 16 (the M dimension of
// a 16x16xK MFMA); the rows of a tensor are padded with zero rows up to a
// multiple of 16.  For every (tile, 256-element block) one contiguous chunk
// holds the 16 rows' bytes of that block, arranged so that lane
// L = i + 16 g (row i of the tile, k-group g) of a wave reads only its own
// bytes with aligned 4..16-byte loads.  Byte counts per chunk equal 16 GGUF
// blocks (no expansion; TQ1_0 tensors are re-encoded at upload as TQ2_0
// blocks of the same trits, 66 bytes per block instead of 54):
//
//   TQ2_0 1056 B = QS[64 lanes][16]  lane (i,g): qs[16g..16g+15]
//                  D [16 rows][f16]
//   Q4_K  2304 B = QS[64 lanes][32]  lane (i,g): for p<4: qs[32p+8g..32p+8g+7]
//                  HD[16 rows][16]   d, dmin, scales[12]
//   Q6_K  3360 B = QL[16 rows][128]  QH[16 rows][64]  SC[16 rows][16]  D[16 rows][f16]
//
// F16 / F32 tensors are stored in tiles of 256 rows, chunk by chunk: the
// 128-byte pieces (64 halves or 32 floats) of the tile's rows for columns
// c*E .. c*E+E-1 are one contiguous 32 KB block, rows and columns padded
// with zeros.  A GEMV workgroup (one lane per row) then reads each chunk
// as one contiguous run.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/fox_gpu.h"

#define FOX_TILE 16
#define FOX_FTILE 256            // rows per tile of a float tensor
#define FOX_FCHUNK 128           // bytes per row in one chunk of a float tensor

// byte offset of element (r, k) of a float tensor with K columns
__host__ __device__ inline uint64_t fox_float_offset(uint64_t r, uint64_t k, uint64_t K,
                                                     uint64_t esize)
{
    const uint64_t per = FOX_FCHUNK / esize, nchunk = (K + per - 1) / per;
    return (((r / FOX_FTILE) * nchunk + k / per) * FOX_FTILE + r % FOX_FTILE) * FOX_FCHUNK +
           (k % per) * esize;
}
#define TQ2_CHUNK 1056
#define Q4K_CHUNK 2304
#define Q6K_CHUNK 3360

struct fox_gpu_ctx {
    int device;
    hipStream_t stream;
    // second stream for weight uploads of the streaming backend (default
    // priority, like the compute stream)
    hipStream_t copy;
    int n_cu;
    // upper bound on the persistent grid of the fused GEMV (0: two
    // workgroups per compute unit); fox_gpu_set_max_workgroups
    int max_wg;
    uint64_t hbm_bytes;
    char name[128];
    // activation workspace (quantised values, B operands, corrections)
    uint8_t *ws;
    size_t ws_cap;
    int capturing;
    // earlier, smaller workspaces: a captured graph may still address them,
    // so they are freed only at shutdown
    uint8_t *retired[32];
    int n_retired;
    // small fixed buffer (counters, cross-workgroup partials) zeroed at init;
    // its address never changes, so captured graphs may use it
    uint8_t *small;
    // this device's copy of the fixed scratch of fox_gpu_gemv_noalloc
    uint8_t *scratch;
};
#define FOX_SMALL_BYTES (64 * 1024)
// the argmax partials' place in the small buffer
#define FOX_SMALL_AM_OFF 256

struct fox_gpu_tensor {
    int type;
    uint64_t ne0, ne1;        // K, N
    uint64_t gguf_bytes;
    uint64_t dev_bytes;
    uint64_t n_tiles;         // block types: ceil(N / 16)
    uint8_t *d;
};

struct fox_gpu_graph {
    hipGraph_t graph;
    hipGraphExec_t exec;
};

struct fox_gpu_event {
    hipEvent_t ev;
};

// ---- errors (implemented in fox_gpu.hip)
fox_gpu_status fox_fail(fox_gpu_status st, const char *fmt, ...)
    __attribute__((format(printf, 2, 3)));
fox_gpu_status fox_hip_fail(hipError_t e, const char *what);

#define FOX_HIP(call)                                                    \
    do {                                                                 \
        hipError_t fox_e_ = (call);                                      \
        if (fox_e_ != hipSuccess) return fox_hip_fail(fox_e_, #call);    \
    } while (0)

#define FOX_LAUNCHED(what)                                               \
    do {                                                                 \
        hipError_t fox_e_ = hipGetLastError();                           \
        if (fox_e_ != hipSuccess) return fox_hip_fail(fox_e_, what);     \
    } while (0)

// ---- workspace (fox_gpu.hip)
fox_gpu_status fox_ws_reserve(fox_gpu_ctx *ctx, size_t bytes);

// ---- fixed scratch of fox_gpu_gemv_noalloc (fox_gemv.hip): resolves this
// device's copy into ctx->scratch; called by fox_gpu_init with the device
// current
#define FOX_NOALLOC_SCRATCH (2u << 20)
fox_gpu_status fox_scratch_init(fox_gpu_ctx *ctx);

// ---- type helpers
static inline size_t fox_block_bytes(int type)
{
    switch (type) {
    case FOX_GPU_F32: return 4;
    case FOX_GPU_F16: return 2;
    case FOX_GPU_Q4_K: return 144;
    case FOX_GPU_Q6_K: return 210;
    case FOX_GPU_TQ1_0: return 54;
    case FOX_GPU_TQ2_0: return 66;
    default: return 0;
    }
}

static inline size_t fox_block_elems(int type)
{
    switch (type) {
    case FOX_GPU_F32: case FOX_GPU_F16: return 1;
    case FOX_GPU_Q4_K: case FOX_GPU_Q6_K: case FOX_GPU_TQ1_0: case FOX_GPU_TQ2_0:
        return 256;
    default: return 0;
    }
}

static inline bool fox_is_block_type(int type) { return fox_block_elems(type) == 256; }

// The block layout a tensor of `type` has in HBM.  TQ1_0 tensors are held
// as TQ2_0 blocks: the upload re-encodes every trit (base-3 digit of a TQ1_0
// byte) as the 2-bit code of the same element, so the GEMVs decode bit
// fields instead of base-3 digits; integer block sums, and so every result,
// are unchanged.
static inline int fox_device_type(int type)
{
    return type == FOX_GPU_TQ1_0 ? FOX_GPU_TQ2_0 : type;
}

// bytes of one device chunk (16 rows x one block) of a tensor of `type`
static inline size_t fox_chunk_bytes(int type)
{
    switch (fox_device_type(type)) {
    case FOX_GPU_Q4_K: return Q4K_CHUNK;
    case FOX_GPU_Q6_K: return Q6K_CHUNK;
    case FOX_GPU_TQ2_0: return TQ2_CHUNK;
    default: return 0;
    }
}

static inline const char *fox_type_name(int type)
{
    switch (type) {
    case FOX_GPU_F32: return "F32";
    case FOX_GPU_F16: return "F16";
    case FOX_GPU_Q4_0: return "Q4_0";
    case FOX_GPU_Q8_0: return "Q8_0";
    case FOX_GPU_Q4_K: return "Q4_K";
    case FOX_GPU_Q5_K: return "Q5_K";
    case FOX_GPU_Q6_K: return "Q6_K";
    case FOX_GPU_TQ1_0: return "TQ1_0";
    case FOX_GPU_TQ2_0: return "TQ2_0";
    default: return "unknown";
    }
}

// ---- gemv internals shared by fox_gemv.hip and fox_gpu.hip
fox_gpu_status fox_gemv_launch(fox_gpu_ctx *ctx, size_t n, const fox_gpu_tensor *const *ws,
                               const float *x, size_t x_stride, const int8_t *q,
                               const float *scale, size_t M, float *const *outs,
                               const size_t *out_strides, unsigned flags,
                               int32_t *sums);
