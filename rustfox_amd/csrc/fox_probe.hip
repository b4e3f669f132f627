// fox_probe.hip -- diagnostics for bench.py, outside the product ABI
// (rustfox_amd/lib/librustfox_probe.so; nothing in librustfox_amd.so or
// libfox.so calls them, and no include/ header declares them):
//
//   fox_gpu_read_probe(ctx, src, n, loads, grid, sink)
//       a streaming read of n bytes (n and src 16-byte aligned) by `grid`
//       workgroups of 256 threads, each thread keeping `loads` (1, 2, 4, 8
//       or 16) 16-byte loads in flight: the HBM read ceiling the GEMVs are
//       compared with;
//   fox_gpu_empty_probe(ctx, grid, sink)
//       one empty kernel of `grid` workgroups: timed back to back, or
//       captured in a graph, the fixed cost of a launch or of a graph node;
//   fox_gpu_sum_probe(ctx, e, n, acc, out)
//       the attention kernels' whole-wave softmax sum (sum_in_order) of n
//       floats from acc, by one wave, into out[0], and the one-add-at-a-time
//       chain's into out[2] (out[1], out[3]: their shader clocks): its tests
//       compare them with the sum in order on inputs chosen to hit its
//       events.
//
// sink (device memory, 4 bytes) is written only if the folded data hit a
// fixed constant, so the loads cannot be dropped and nothing is written in
// practice.
#include "fox_internal.h"
#include "fox_sum.h"

// ------------------------------------------------------- read probe

// Streaming read of n16 16-byte words: a workgroup reads contiguous
// chunks of U * 4 KB (grid-stride over chunks), every thread keeping U loads
// in flight (the U loads of a chunk are issued before any is used); the
// ragged tail by single loads.  The loaded words are folded into one value
// that is stored only if it equals a constant no input is expected to
// produce, so the loads cannot be dropped and nothing is written in
// practice.
template <int U>
__global__ __launch_bounds__(256) void read_probe_k(const uint4 *__restrict__ src, size_t n16,
                                                    uint32_t *__restrict__ sink)
{
    constexpr size_t CH = (size_t)U * 256;             // words per chunk
    const size_t nch = n16 / CH;
    uint32_t acc = 0;
    for (size_t c = blockIdx.x; c < nch; c += gridDim.x) {
        const uint4 *p = src + c * CH + threadIdx.x;
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = p[u * 256];
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (size_t i = nch * CH + (size_t)blockIdx.x * 256 + threadIdx.x; i < n16;
         i += (size_t)gridDim.x * 256) {
        const uint4 v = src[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;
}

// An empty kernel: what one launch costs on the stream, or one node of a
// graph, before any work (the store never happens: no workgroup has that
// many threads).
__global__ __launch_bounds__(256) void empty_probe_k(uint32_t *sink)
{
    if (threadIdx.x == 1u << 20) sink[0] = 1;
}

extern "C" fox_gpu_status fox_gpu_empty_probe(fox_gpu_ctx *ctx, int grid, uint32_t *sink)
{
    if (!ctx || !sink || grid <= 0 || grid > (1 << 20))
        return fox_fail(FOX_GPU_ERR_ARG, "empty_probe: bad argument");
    hipLaunchKernelGGL(empty_probe_k, dim3((unsigned)grid), dim3(256), 0, ctx->stream, sink);
    FOX_LAUNCHED("empty_probe");
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_read_probe(fox_gpu_ctx *ctx, const void *src, size_t n,
                                             int loads, int grid, uint32_t *sink)
{
    if (!ctx || !src || !sink || n == 0 || n % 16 || (uintptr_t)src % 16 || grid <= 0 ||
        grid > (1 << 20))
        return fox_fail(FOX_GPU_ERR_ARG, "read_probe: bad argument");
    const uint4 *s = (const uint4 *)src;
    const size_t n16 = n / 16;
    switch (loads) {
    case 1: hipLaunchKernelGGL(read_probe_k<1>, dim3((unsigned)grid), dim3(256), 0, ctx->stream, s, n16, sink); break;
    case 2: hipLaunchKernelGGL(read_probe_k<2>, dim3((unsigned)grid), dim3(256), 0, ctx->stream, s, n16, sink); break;
    case 4: hipLaunchKernelGGL(read_probe_k<4>, dim3((unsigned)grid), dim3(256), 0, ctx->stream, s, n16, sink); break;
    case 8: hipLaunchKernelGGL(read_probe_k<8>, dim3((unsigned)grid), dim3(256), 0, ctx->stream, s, n16, sink); break;
    case 16: hipLaunchKernelGGL(read_probe_k<16>, dim3((unsigned)grid), dim3(256), 0, ctx->stream, s, n16, sink); break;
    default: return fox_fail(FOX_GPU_ERR_ARG, "read_probe: 1, 2, 4, 8 or 16 loads in flight");
    }
    FOX_LAUNCHED("read_probe");
    return FOX_GPU_OK;
}

// ------------------------------------------------------- in-order sum

#define SUM_PROBE_MAX 16384

// out[0] the whole-wave sum, out[1] its shader clocks; out[2] the
// one-add-at-a-time chain (chain_quads, then single adds), out[3] its clocks
__global__ __launch_bounds__(64) void sum_probe_k(const float *__restrict__ e, int n, float acc,
                                                  float *__restrict__ out)
{
    extern __shared__ float se[];                      // n + SUM_CHUNK floats
    for (int i = threadIdx.x; i < n + SUM_CHUNK; i += 64) se[i] = i < n ? e[i] : 0.0f;
    __syncthreads();
    const uint64_t t0 = __builtin_amdgcn_s_memtime();
    const float s = sum_in_order(acc, se, n);
    const uint64_t t1 = __builtin_amdgcn_s_memtime();
    float c = chain_quads(acc, (const float4 *)se, n >> 2);
    for (int i = n & ~3; i < n; i++) c = c + se[i];
    const uint64_t t2 = __builtin_amdgcn_s_memtime();
    if (threadIdx.x == 0) {
        out[0] = s;
        out[1] = (float)(t1 - t0);
        out[2] = c;
        out[3] = (float)(t2 - t1);
    }
}

extern "C" fox_gpu_status fox_gpu_sum_probe(fox_gpu_ctx *ctx, const float *e, int n, float acc,
                                            float *out)
{
    if (!ctx || !out || n < 0 || n > SUM_PROBE_MAX || (n > 0 && !e))
        return fox_fail(FOX_GPU_ERR_ARG, "sum_probe: bad argument (n at most %d)", SUM_PROBE_MAX);
    const size_t lds = ((size_t)n + SUM_CHUNK) * sizeof(float);
    hipError_t err = hipFuncSetAttribute((const void *)sum_probe_k,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (err != hipSuccess) return fox_hip_fail(err, "sum_probe: LDS size");
    hipLaunchKernelGGL(sum_probe_k, dim3(1), dim3(64), lds, ctx->stream, e, n, acc, out);
    FOX_LAUNCHED("sum_probe");
    return FOX_GPU_OK;
}
