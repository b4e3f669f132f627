// fox_ops.hip -- bandwidth-bound decode ops: row gather, RMSNorm, RoPE + KV
// store, split-position GQA attention, SwiGLU, residual add, argmax.
// Built with -ffp-contract=off like the rest of the library: every float op
// rounds once, in the reference's order where the reference fixes an order.
#include "fox_gemv_dev.h"
#include "fox_internal.h"
#include "fox_math.h"

#include <cmath>
#include <utility>

// ------------------------------------------------------------------ rows

// the wave index as a wave-uniform (scalar) value: loops and tests on it
// are then scalar branches, not masked vector code
__device__ __forceinline__ int wave_index()
{
    return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

template <typename WT>
__global__ void get_rows_k(const WT *__restrict__ src, uint64_t K, uint64_t N,
                           const uint32_t *__restrict__ rows, int n, float *__restrict__ out,
                           size_t out_stride, uint32_t *bad)
{
    const int i = blockIdx.y;
    const uint32_t r = rows[i];
    if (r >= N) {
        if (bad && blockIdx.x == 0 && threadIdx.x == 0) *bad = 1u;
        return;
    }
    for (uint64_t k = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; k < K;
         k += (uint64_t)gridDim.x * blockDim.x)
        out[(size_t)i * out_stride + k] =
            (float)src[fox_float_offset(r, k, K, sizeof(WT)) / sizeof(WT)];
}

extern "C" fox_gpu_status fox_gpu_get_rows(fox_gpu_ctx *ctx, const fox_gpu_tensor *t,
                                           const uint32_t *rows, size_t n, float *out,
                                           size_t out_stride, uint32_t *bad)
{
    if (!ctx || !t || !rows || !out || n == 0)
        return fox_fail(FOX_GPU_ERR_ARG, "get_rows: bad argument");
    if (n > 65535) return fox_fail(FOX_GPU_ERR_ARG, "get_rows: %zu rows per call", n);
    if (n > 1 && out_stride < t->ne0) return fox_fail(FOX_GPU_ERR_ARG, "get_rows: stride < K");
    dim3 grid((unsigned)((t->ne0 + 255) / 256 < 64 ? (t->ne0 + 255) / 256 : 64), (unsigned)n);
    size_t os = n > 1 ? out_stride : t->ne0;
    if (t->type == FOX_GPU_F16)
        hipLaunchKernelGGL(get_rows_k<_Float16>, grid, dim3(256), 0, ctx->stream,
                           (const _Float16 *)t->d, t->ne0, t->ne1, rows, (int)n, out, os, bad);
    else if (t->type == FOX_GPU_F32)
        hipLaunchKernelGGL(get_rows_k<float>, grid, dim3(256), 0, ctx->stream,
                           (const float *)t->d, t->ne0, t->ne1, rows, (int)n, out, os, bad);
    else
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED,
                        "get_rows: %s rows are read by the gemv kernels only; embeddings and "
                        "norms on the device path are F16 or F32", fox_type_name(t->type));
    FOX_LAUNCHED("get_rows");
    return FOX_GPU_OK;
}

// ------------------------------------------------------------- dequant

// f16 bits -> f32 bits by field arithmetic (src/kernels.c:14-39 semantics):
// NaN payloads are shifted as they are, without the quieting a hardware
// conversion may apply to a signalling NaN.
__device__ __forceinline__ float f16_exact(uint32_t h)
{
    const uint32_t sign = (h >> 15) << 31, e = (h >> 10) & 31u, f = h & 0x3FFu;
    uint32_t u;
    if (e == 31) {
        u = sign | 0x7F800000u | (f << 13);
    } else if (e == 0) {
        if (f == 0) {
            u = sign;
        } else {
            // f = 1.m * 2^(p) with p the top set bit (0..9): value f * 2^-24
            const int p = 31 - __builtin_clz(f);
            u = sign | ((uint32_t)(p - 24 + 127) << 23) | ((f << (23 - p)) & 0x7FFFFFu);
        }
    } else {
        u = sign | ((e + 112u) << 23) | (f << 13);
    }
    return __uint_as_float(u);
}

// One element per thread of a row in its GGUF bytes: F32 copy, F16
// conversion, Q8_0 y = q*d and Q4_0 y = (nibble-8)*d (src/kernels.c:896-920:
// 32-element blocks, a block's low nibbles its first 16 elements), Q4_K
// y = (d*sc)*q - dmin*m (src/kernels.c:257-283), Q5_K the same with a fifth
// bit from qh (src/kernels.c:286-306: groups 0-3 take the low nibbles of
// qs, groups 4-7 the high ones, group g's fifth bit is bit g of qh[l]),
// Q6_K y = (d*sc)*(q-32) (src/kernels.c:217-244), each product rounded as
// there.
__device__ __forceinline__ void k4_scale_min(const uint8_t *s, int j, uint32_t &sc, uint32_t &m)
{
    if (j < 4) {
        sc = s[j] & 63u;
        m = s[j + 4] & 63u;
    } else {
        sc = (s[j + 4] & 15u) | ((uint32_t)(s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((uint32_t)(s[j] >> 6) << 4);
    }
}

__global__ void dequant_gguf_k(int type, const uint8_t *__restrict__ w, uint64_t n,
                               float *__restrict__ out)
{
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        float y;
        if (type == FOX_GPU_F32) {
            y = ((const float *)w)[i];
        } else if (type == FOX_GPU_F16) {
            y = f16_exact(((const uint16_t *)w)[i]);
        } else if (type == FOX_GPU_Q8_0) {
            const uint8_t *blk = w + (i >> 5) * 34;
            const float d = f16_exact(blk[0] | (uint32_t)blk[1] << 8);
            y = (float)(int8_t)blk[2 + (i & 31)] * d;
        } else if (type == FOX_GPU_Q4_0) {
            const uint8_t *blk = w + (i >> 5) * 18;
            const int e = (int)(i & 31);
            const uint8_t qb = blk[2 + (e & 15)];
            const int q = (int)(e < 16 ? (qb & 15u) : (qb >> 4)) - 8;
            const float d = f16_exact(blk[0] | (uint32_t)blk[1] << 8);
            y = (float)q * d;
        } else if (type == FOX_GPU_Q5_K) {
            const uint8_t *blk = w + (i >> 8) * 176;
            const int e = (int)(i & 255), grp = e >> 5, l = e & 31;
            uint32_t sc, m;
            k4_scale_min(blk + 4, grp, sc, m);
            const uint8_t qb = blk[48 + 32 * (grp & 3) + l];
            const uint32_t q = (grp < 4 ? (qb & 15u) : (qb >> 4)) | (((blk[16 + l] >> grp) & 1u) << 4);
            const float d = f16_exact(blk[0] | (uint32_t)blk[1] << 8);
            const float dmin = f16_exact(blk[2] | (uint32_t)blk[3] << 8);
            y = d * (float)sc * (float)q - dmin * (float)m;
        } else if (type == FOX_GPU_Q4_K) {
            const uint8_t *blk = w + (i >> 8) * 144;
            const int e = (int)(i & 255), p = e >> 6, l = e & 63, j = 2 * p + (l >> 5);
            uint32_t sc, m;
            k4_scale_min(blk + 4, j, sc, m);
            const uint8_t qb = blk[16 + 32 * p + (l & 31)];
            const uint32_t q = l < 32 ? (qb & 15u) : (qb >> 4);
            const float d = f16_exact(blk[0] | (uint32_t)blk[1] << 8);
            const float dmin = f16_exact(blk[2] | (uint32_t)blk[3] << 8);
            const float d1 = d * (float)sc, m1 = dmin * (float)m;
            y = d1 * (float)q - m1;
        } else {   // Q6_K
            const uint8_t *blk = w + (i >> 8) * 210;
            const int e = (int)(i & 255), h = e >> 7, g = (e >> 5) & 3, l = e & 31;
            const uint8_t *ql = blk + 64 * h, *qh = blk + 128 + 32 * h;
            const int8_t *sc = (const int8_t *)(blk + 192 + 8 * h);
            const uint32_t lo = (g & 1) ? ql[l + 32] : ql[l];
            const uint32_t q = ((g & 2) ? lo >> 4 : lo & 15u) | (((qh[l] >> (2 * g)) & 3u) << 4);
            const float d = f16_exact(blk[208] | (uint32_t)blk[209] << 8);
            y = d * (float)sc[l / 16 + 2 * g] * (float)((int)q - 32);
        }
        out[i] = y;
    }
}

extern "C" fox_gpu_status fox_gpu_dequant(fox_gpu_ctx *ctx, int type, const void *row, size_t n,
                                          float *out)
{
    if (!ctx || !row || !out || n == 0) return fox_fail(FOX_GPU_ERR_ARG, "dequant: bad argument");
    size_t be;
    switch (type) {
    case FOX_GPU_F32: case FOX_GPU_F16: be = 1; break;
    case FOX_GPU_Q8_0: case FOX_GPU_Q4_0: be = 32; break;
    case FOX_GPU_Q4_K: case FOX_GPU_Q5_K: case FOX_GPU_Q6_K: be = 256; break;
    default:
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "dequant: %s rows are not dequantised",
                        fox_type_name(type));
    }
    if (n % be)
        return fox_fail(FOX_GPU_ERR_ARG, "dequant: %zu elements is not a whole number of %s "
                        "blocks", n, fox_type_name(type));
    const uint64_t g = (n + 255) / 256;
    hipLaunchKernelGGL(dequant_gguf_k, dim3((unsigned)(g < 4096 ? g : 4096)), dim3(256), 0,
                       ctx->stream, type, (const uint8_t *)row, (uint64_t)n, out);
    FOX_LAUNCHED("dequant");
    return FOX_GPU_OK;
}

// --------------------------------------------------------------- rmsnorm

__device__ __forceinline__ double wave_sum_d(double v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// src/ops.c:7-22: scale = (float)(1 / sqrt(sum x^2 / n + eps)) with the
// squares (exact in double) summed in double in index order, then
// out = x * scale * w, two float roundings.  The in-order double sum is
// replaced by a tree sum S_t; the in-order sum lies within
// (n + 64) * 2^-52 * S_t of it, so if both ends of that interval give the
// same float scale (double operations widened by a few ulps), that float is
// the reference's.  Otherwise (about one call in 10^5) one lane redoes the
// sum in index order.
__device__ __forceinline__ double rms_scale_d(double ss, int n, float eps)
{
    return 1.0 / __builtin_sqrt(ss / (double)n + (double)eps);
}

// the float scale from the tree sum tot of the squares of x[0 .. n) (one
// thread calls it; the rare undecided case rereads x in index order)
__device__ float rms_scale_f(double tot, const float *xt, int n, float eps)
{
    const double rel = (double)(n + 64) * 0x1p-52;
    const double y_hi = rms_scale_d(tot * (1.0 - rel), n, eps) * (1.0 + 0x1p-50);
    const double y_lo = rms_scale_d(tot * (1.0 + rel), n, eps) * (1.0 - 0x1p-50);
    const float f_hi = (float)y_hi, f_lo = (float)y_lo;
    if (f_hi == f_lo) return f_hi;
    double seq = 0.0;
    for (int i = 0; i < n; i++) seq += (double)xt[i] * (double)xt[i];
    return (float)rms_scale_d(seq, n, eps);
}

// R > 0: n <= 256 R, and each thread holds its R values of x (and w) in
// registers, every load issued before the first use (one memory round trip
// instead of one per loop step).  R = 0: any n, strided loops.
template <int R>
__global__ __launch_bounds__(256) void rmsnorm_k(float *__restrict__ out, size_t out_stride,
                                                 const float *__restrict__ x, size_t x_stride,
                                                 const float *__restrict__ w, int n, float eps)
{
    __shared__ double red[4];
    __shared__ float sc;
    const int t = blockIdx.x, tid = threadIdx.x;
    const float *xt = x + (size_t)t * x_stride;
    float *ot = out + (size_t)t * out_stride;
    constexpr int RR = R > 0 ? R : 1;
    float xv[RR], wv[RR];
    double s = 0.0;
    if (R > 0) {
#pragma unroll
        for (int r = 0; r < RR; r++) {
            const int i = tid + 256 * r, ic = i < n ? i : n - 1;
            xv[r] = xt[ic];
            wv[r] = w ? w[ic] : 1.0f;
        }
#pragma unroll
        for (int r = 0; r < RR; r++)
            if (tid + 256 * r < n) s += (double)xv[r] * (double)xv[r];
    } else {
        for (int i = tid; i < n; i += 256) s += (double)xt[i] * (double)xt[i];
    }
    s = wave_sum_d(s);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    if (tid == 0) sc = rms_scale_f((red[0] + red[1]) + (red[2] + red[3]), xt, n, eps);
    __syncthreads();
    const float scale = sc;
    if (R > 0) {
#pragma unroll
        for (int r = 0; r < RR; r++) {
            const int i = tid + 256 * r;
            if (i < n) {
                const float v = xv[r] * scale;
                ot[i] = w ? v * wv[r] : v;
            }
        }
    } else {
        for (int i = tid; i < n; i += 256) {
            const float v = xt[i] * scale;
            ot[i] = w ? v * w[i] : v;
        }
    }
}

extern "C" fox_gpu_status fox_gpu_rmsnorm(fox_gpu_ctx *ctx, float *out, size_t out_stride,
                                          const float *x, size_t x_stride, const float *w,
                                          size_t n, size_t M, float eps)
{
    if (!ctx || !out || !x || n == 0 || M == 0)
        return fox_fail(FOX_GPU_ERR_ARG, "rmsnorm: bad argument");
    if (M > 1 && (out_stride < n || x_stride < n))
        return fox_fail(FOX_GPU_ERR_ARG, "rmsnorm: stride < n");
    const size_t r = (n + 255) / 256;
    const void *k = r <= 2 ? (const void *)rmsnorm_k<2> : r <= 4 ? (const void *)rmsnorm_k<4>
                  : r <= 6 ? (const void *)rmsnorm_k<6> : r <= 8 ? (const void *)rmsnorm_k<8>
                  : r <= 10 ? (const void *)rmsnorm_k<10> : r <= 12 ? (const void *)rmsnorm_k<12>
                  : r <= 16 ? (const void *)rmsnorm_k<16> : (const void *)rmsnorm_k<0>;
    size_t os = M > 1 ? out_stride : n, xs = M > 1 ? x_stride : n;
    int in = (int)n;
    void *args[] = {(void *)&out, (void *)&os, (void *)&x, (void *)&xs, (void *)&w, (void *)&in,
                    (void *)&eps};
    hipError_t e = hipLaunchKernel(k, dim3((unsigned)M), dim3(256), args, 0, ctx->stream);
    if (e != hipSuccess) return fox_hip_fail(e, "rmsnorm");
    FOX_LAUNCHED("rmsnorm");
    return FOX_GPU_OK;
}

// ------------------------------------------------------------ rope+store

// Cache layout.  K rows are f32 [n_ctx][kv_dim] as in the reference.  V is
// position-quad interleaved: element (p, c) at ((p / 4) * kv_dim + c) * 4 +
// p % 4, so four consecutive positions of one column are one 16-byte load
// (the value sums walk positions in order, one column per lane).
__device__ __forceinline__ size_t vq_index(size_t p, size_t c, size_t kvd)
{
    return ((p >> 2) * kvd + c) * 4 + (p & 3);
}

// src/ops.c:56-73 on q and k of token t at position pos[0]+t, then the
// src/forward.c:357-361 copies of k and v into cache row pos[0]+t.
__global__ void rope_store_k(float *__restrict__ q, size_t q_stride, float *__restrict__ k,
                             size_t k_stride, const float *__restrict__ v, size_t v_stride,
                             int n_head, int n_head_kv, int hd, const float *__restrict__ cos_t,
                             const float *__restrict__ sin_t, const uint32_t *__restrict__ pos,
                             size_t n_ctx, float *__restrict__ kc, float *__restrict__ vc)
{
    const int t = blockIdx.x;
    const size_t p = (size_t)pos[0] + (size_t)t;
    if (p >= n_ctx) return;
    const int half = hd / 2;
    const float *cr = cos_t + p * half, *sr = sin_t + p * half;
    float *qt = q + (size_t)t * q_stride, *kt = k + (size_t)t * k_stride;
    const float *vt = v + (size_t)t * v_stride;
    const int nq = n_head * half, nk = n_head_kv * half;
    for (int i = threadIdx.x; i < nq + nk; i += blockDim.x) {
        float *vec = i < nq ? qt : kt;
        const int ii = i < nq ? i : i - nq;
        const int h = ii / half, j = ii % half;
        float *pr = vec + (size_t)h * hd + 2 * j;
        const float a = pr[0], b = pr[1], c = cr[j], s = sr[j];
        pr[0] = a * c - b * s;
        pr[1] = a * s + b * c;
    }
    __syncthreads();
    const int kvd = n_head_kv * hd;
    for (int i = threadIdx.x; i < kvd; i += blockDim.x) {
        kc[p * kvd + i] = kt[i];
        vc[vq_index(p, (size_t)i, (size_t)kvd)] = vt[i];
    }
}

extern "C" fox_gpu_status fox_gpu_rope_store(fox_gpu_ctx *ctx, float *q, size_t q_stride,
                                             float *k, size_t k_stride, const float *v,
                                             size_t v_stride, size_t n_head, size_t n_head_kv,
                                             size_t head_dim, size_t M, const float *cos_t,
                                             const float *sin_t, const uint32_t *pos,
                                             size_t n_ctx, float *k_cache, float *v_cache)
{
    if (!ctx || !q || !k || !v || !cos_t || !sin_t || !pos || !k_cache || !v_cache ||
        n_head == 0 || n_head_kv == 0 || head_dim == 0 || M == 0 || n_ctx == 0)
        return fox_fail(FOX_GPU_ERR_ARG, "rope_store: bad argument");
    if (head_dim % 2) return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "rope_store: odd head dimension");
    if (M > FOX_GPU_MAX_TOKENS) return fox_fail(FOX_GPU_ERR_ARG, "rope_store: too many tokens");
    hipLaunchKernelGGL(rope_store_k, dim3((unsigned)M), dim3(256), 0, ctx->stream, q, q_stride, k,
                       k_stride, v, v_stride, (int)n_head, (int)n_head_kv, (int)head_dim, cos_t,
                       sin_t, pos, n_ctx, k_cache, v_cache);
    FOX_LAUNCHED("rope_store");
    return FOX_GPU_OK;
}

// rows p0 .. p0+n-1 of both caches from row-major [n][kv_dim] k and v
__global__ void kv_write_k(float *__restrict__ kc, float *__restrict__ vc, int kvd, size_t p0,
                           const float *__restrict__ k, const float *__restrict__ v)
{
    const size_t i = blockIdx.x, p = p0 + i;
    for (int c = threadIdx.x; c < kvd; c += blockDim.x) {
        kc[p * kvd + c] = k[i * kvd + c];
        vc[vq_index(p, (size_t)c, (size_t)kvd)] = v[i * kvd + c];
    }
}

extern "C" fox_gpu_status fox_gpu_kv_write(fox_gpu_ctx *ctx, float *k_cache, float *v_cache,
                                           size_t kv_dim, size_t n_ctx, size_t p0, size_t n,
                                           const float *k, const float *v)
{
    if (!ctx || !k_cache || !v_cache || !k || !v || kv_dim == 0 || n == 0)
        return fox_fail(FOX_GPU_ERR_ARG, "kv_write: bad argument");
    if (p0 + n > n_ctx || n > 0x7fffffff)
        return fox_fail(FOX_GPU_ERR_ARG, "kv_write: rows %zu..%zu outside the %zu-row cache", p0,
                        p0 + n, n_ctx);
    hipLaunchKernelGGL(kv_write_k, dim3((unsigned)n), dim3(256), 0, ctx->stream, k_cache, v_cache,
                       (int)kv_dim, p0, k, v);
    FOX_LAUNCHED("kv_write");
    return FOX_GPU_OK;
}

// -------------------------------------------------------------- attention
//
#define ATT_SPLIT 32   // cache rows per workgroup
#define ATT_MAXG 8     // query heads per kv head handled by one workgroup
#define ATT_MAXHD 256

__device__ __forceinline__ float wave_sum_f(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// One workgroup per (split of ATT_SPLIT rows, kv head, token): scores of the
// kv head's query heads against the split's keys, a local softmax (max m, sum
// l of exp(s - m)) and the exp-weighted value sum o.  Splits past the token's
// causal end write m = -inf, l = 0.
__global__ __launch_bounds__(256) void attn_partial(const float *__restrict__ q, size_t q_stride,
                                                    const float *__restrict__ kc,
                                                    const float *__restrict__ vc, int n_head,
                                                    int n_head_kv, int hd,
                                                    const uint32_t *__restrict__ pos,
                                                    int n_ctx, int n_splits,
                                                    float *__restrict__ part)
{
    __shared__ float qs[ATT_MAXG * ATT_MAXHD];
    __shared__ float sc[ATT_MAXG * ATT_SPLIT];
    const int s = blockIdx.x, kvh = blockIdx.y, t = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_index();
    const int gqa = n_head / n_head_kv, kvd = n_head_kv * hd;
    // rows 0 .. upto-1 are visible; never past the cache
    const int upto = (int)min((size_t)pos[0] + (size_t)t + 1, (size_t)n_ctx);
    const int p0 = s * ATT_SPLIT;
    const int pn = upto - p0 < ATT_SPLIT ? upto - p0 : ATT_SPLIT;
    const size_t rec = 2 + (size_t)hd;
    float *base = part + (((size_t)t * n_head + (size_t)kvh * gqa) * n_splits + s) * rec;

    if (pn <= 0) {
        for (int i = tid; i < gqa; i += 256) {
            float *r = base + (size_t)i * n_splits * rec;
            r[0] = -INFINITY;
            r[1] = 0.0f;
        }
        return;
    }
    const float scale = fox_div(1.0f, fox_sqrtf((float)hd));
    for (int i = tid; i < gqa * hd; i += 256)
        qs[i] = q[(size_t)t * q_stride + (size_t)kvh * gqa * hd + i];
    __syncthreads();
    // scores: wave w takes rows w, w+4, ...; lanes split the head dimension
    for (int pp = wave; pp < pn; pp += 4) {
        const float *kr = kc + (size_t)(p0 + pp) * kvd + (size_t)kvh * hd;
        float kv[ATT_MAXHD / 64];
#pragma unroll
        for (int e = 0; e < ATT_MAXHD / 64; e++) {
            int d = lane + 64 * e;
            kv[e] = d < hd ? kr[d] : 0.0f;
        }
        for (int g = 0; g < gqa; g++) {
            float a = 0.0f;
#pragma unroll
            for (int e = 0; e < ATT_MAXHD / 64; e++) {
                int d = lane + 64 * e;
                if (d < hd) a += qs[g * hd + d] * kv[e];
            }
            a = wave_sum_f(a);
            if (lane == 0) sc[g * ATT_SPLIT + pp] = a * scale;
        }
    }
    __syncthreads();
    // local softmax statistics per query head: wave w takes heads w, w+4
    __shared__ float st_m[ATT_MAXG], st_l[ATT_MAXG];
    for (int g = wave; g < gqa; g += 4) {
        float v = lane < pn ? sc[g * ATT_SPLIT + lane] : -INFINITY;
        float m = v;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        float e = lane < pn ? fox_expf(v - m) : 0.0f;
        if (lane < pn) sc[g * ATT_SPLIT + lane] = e;
        float l = wave_sum_f(e);
        if (lane == 0) {
            st_m[g] = m;
            st_l[g] = l;
        }
    }
    __syncthreads();
    // o = sum_p e_p v_p, one (head, dim) per thread
    for (int i = tid; i < gqa * hd; i += 256) {
        const int g = i / hd, d = i % hd;
        const size_t c = (size_t)kvh * hd + d;
        float o = 0.0f;
        for (int pp = 0; pp < pn; pp++)
            o += sc[g * ATT_SPLIT + pp] * vc[vq_index((size_t)(p0 + pp), c, (size_t)kvd)];
        float *r = base + (size_t)g * n_splits * rec;
        if (d == 0) {
            r[0] = st_m[g];
            r[1] = st_l[g];
        }
        r[2 + d] = o;
    }
}

// Merge the splits of one (head, token): out = sum_s o_s e^{m_s - M} /
// sum_s l_s e^{m_s - M}.
__global__ void attn_merge(const float *__restrict__ part, int n_head, int hd, int n_splits,
                           float *__restrict__ out, size_t out_stride)
{
    const int h = blockIdx.x, t = blockIdx.y;
    const size_t rec = 2 + (size_t)hd;
    const float *base = part + (((size_t)t * n_head + h) * n_splits) * rec;
    float mx = -INFINITY;
    for (int s = 0; s < n_splits; s++) mx = fmaxf(mx, base[s * rec]);
    float L = 0.0f;
    for (int s = 0; s < n_splits; s++) {
        float m = base[s * rec];
        if (m > -INFINITY) L += base[s * rec + 1] * fox_expf(m - mx);
    }
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float o = 0.0f;
        for (int s = 0; s < n_splits; s++) {
            float m = base[s * rec];
            if (m > -INFINITY) o += base[s * rec + 2 + d] * fox_expf(m - mx);
        }
        out[(size_t)t * out_stride + (size_t)h * hd + d] = o / L;
    }
}

// ---- attention in the reference's order (src/forward.c:222-257,
// src/ops.c:24-39), bit for bit:
//   score_j = (sum_d q_d k_jd, summed in d order) * (1 / sqrtf(hd));
//   softmax: max, e_j = expf(score_j - max), sum in j order, e_j * (1/sum);
//   out_d = sum in j order of a_j v_jd.
// Each in-order sum is one lane's chain.  Three kernels: scores (a lane per
// position, K tile in LDS) with per-tile maxima; softmax (one lane runs the
// position-order sum from LDS); values (a lane per output column, walking
// the interleaved V and the weights four positions per load).

#define SC_TILE 64
#define SC_CQ 8                     // quads (4 dimensions) per chunk of a K row

// vmcnt(n) alone (s_waitcnt fields of gfx9: vmcnt [3:0] and [15:14],
// expcnt [6:4], lgkmcnt [11:8]; the others at their maximum)
#define VMCNT_ONLY(n) ((((n) & 15) | (((n) >> 4) << 14)) | (7 << 4) | (15 << 8))

// s_waitcnt vmcnt(n) for n known once loops are unrolled (the instruction
// takes an immediate)
__device__ __forceinline__ void wait_vmcnt(int n)
{
    switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(VMCNT_ONLY(0)); break;
    case 1: __builtin_amdgcn_s_waitcnt(VMCNT_ONLY(1)); break;
    case 2: __builtin_amdgcn_s_waitcnt(VMCNT_ONLY(2)); break;
    case 3: __builtin_amdgcn_s_waitcnt(VMCNT_ONLY(3)); break;
    case 4: __builtin_amdgcn_s_waitcnt(VMCNT_ONLY(4)); break;
    case 5: __builtin_amdgcn_s_waitcnt(VMCNT_ONLY(5)); break;
    case 6: __builtin_amdgcn_s_waitcnt(VMCNT_ONLY(6)); break;
    case 7: __builtin_amdgcn_s_waitcnt(VMCNT_ONLY(7)); break;
    case 8: __builtin_amdgcn_s_waitcnt(VMCNT_ONLY(8)); break;
    case 10: __builtin_amdgcn_s_waitcnt(VMCNT_ONLY(10)); break;
    case 12: __builtin_amdgcn_s_waitcnt(VMCNT_ONLY(12)); break;
    case 14: __builtin_amdgcn_s_waitcnt(VMCNT_ONLY(14)); break;
    default: __builtin_amdgcn_s_waitcnt(VMCNT_ONLY(0)); break;
    }
}

// global -> LDS copy of 16 bytes per lane: lane l's bytes land at dst + 16 l
// (dst wave-uniform), counted by vmcnt like a load
__device__ __forceinline__ void copy_to_lds16(const void *src, void *dst)
{
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)dst, 16, 0, 0);
}

// the products of one chunk (SC_CQ quads) added to acc in dimension order:
// every read of the chunk is issued before the first add (with FULL the
// chunk is known to be whole, and no per-quad branch splits the reads from
// the adds)
template <bool FULL>
__device__ __forceinline__ float sc_chunk(float acc, const float4 *qr, const float4 *kr, int sw,
                                          int c, int nv)
{
    float4 qv[SC_CQ], kv[SC_CQ];
#pragma unroll
    for (int j = 0; j < SC_CQ; j++) {
        if (FULL || SC_CQ * c + j < nv) {
            qv[j] = qr[j];
            kv[j] = kr[j ^ sw];
        }
    }
#pragma unroll
    for (int j = 0; j < SC_CQ; j++) {
        if (FULL || SC_CQ * c + j < nv) {
            acc = acc + qv[j].x * kv[j].x;
            acc = acc + qv[j].y * kv[j].y;
            acc = acc + qv[j].z * kv[j].z;
            acc = acc + qv[j].w * kv[j].w;
        }
    }
    return acc;
}

// tokens per scores workgroup (27B-class heads, 8192 positions, 8 tokens:
// 241.6 us for the whole attention with one, 220.1 with two, 213.4 with
// four, 216.3 with eight; 4B-class heads at 2048: 57.5 to 58.3 us up to four,
// 63.9 with eight)
#define SC_TPW 4
// One workgroup per (64-position tile, kv head, TPW tokens); wave w
// takes query heads w, w + 4, ... of the kv head, one lane per position.  The
// tile's K rows arrive in NCH chunks of 32 dimensions, copied straight into
// LDS: every copy is issued at the start, and the first token's dot products
// of chunk c run once that chunk is in, while the later ones are still
// arriving (each sum stays in head-dimension order, chunk after chunk).  The
// later tokens reuse the tile (only their query heads are copied), so K is
// read once for every TPW tokens.  A chunk holds 64 rows of 8
// quads (128 B a row); quad j of row r sits in slot j ^ ((r >> 1) & 7), so
// that sixteen consecutive lanes' reads of one quad fall in different banks
// (rows r and r + 1 differ in the 32-bank half, r and r + 2 .. r + 14 in the
// slot).
template <int NCH>
__global__ __launch_bounds__(256) void attn_scores_x(const float *__restrict__ q,
                                                     size_t q_stride,
                                                     const float *__restrict__ kc, int n_head,
                                                     int n_head_kv, int hd,
                                                     const uint32_t *__restrict__ pos,
                                                     int n_ctx, size_t att_stride,
                                                     float *__restrict__ att,
                                                     float *__restrict__ tmax, int n_tiles,
                                                     int M, int tpw)
{
    // one array per chunk: separate objects, so that waiting for a chunk's
    // copies does not wait for the later chunks' copies
    __shared__ float4 kq0[SC_TILE * SC_CQ], kq1[NCH > 1 ? SC_TILE * SC_CQ : 1],
        kq2[NCH > 2 ? SC_TILE * SC_CQ : 1], kq3[NCH > 3 ? SC_TILE * SC_CQ : 1],
        kq4[NCH > 4 ? SC_TILE * SC_CQ : 1], kq5[NCH > 5 ? SC_TILE * SC_CQ : 1],
        kq6[NCH > 6 ? SC_TILE * SC_CQ : 1], kq7[NCH > 7 ? SC_TILE * SC_CQ : 1];
    __shared__ float4 qq[ATT_MAXG * ATT_MAXHD / 4];             // [gqa][hd / 4]
    auto kq = [&](int c) -> float4 * {                          // chunk c: [64 rows][8 slots]
        return c == 0 ? kq0 : c == 1 ? kq1 : c == 2 ? kq2 : c == 3 ? kq3
             : c == 4 ? kq4 : c == 5 ? kq5 : c == 6 ? kq6 : kq7;
    };
    const int tile = blockIdx.x, p0 = tile * SC_TILE, kvh = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = wave_index();
    const int gqa = n_head / n_head_kv, kvd = n_head_kv * hd, nv = hd >> 2;
    // token t sees positions below upto(t), which grows with t: the first
    // token that reaches this tile, and the rows the last one uses
    auto upto_of = [&](int t) {
        return (int)min((size_t)pos[0] + (size_t)t + 1, (size_t)n_ctx);
    };
    // this workgroup's tokens: tz .. t_end - 1
    const int tz = (int)blockIdx.z * tpw, t_end = min(tz + tpw, M);
    const int upto_last = upto_of(t_end - 1);
    if (p0 >= upto_last) return;
    int t0 = tz;
    while (upto_of(t0) <= p0) t0++;                         // (uniform)
    const int pn_last = upto_last - p0 < SC_TILE ? upto_last - p0 : SC_TILE;
    // the query heads: blocks of 64 quads, wave w takes blocks w, w + 4
    const int nqq = gqa * nv, nqb = (nqq + 63) >> 6;
    constexpr int QB = ATT_MAXG * ATT_MAXHD / 4 / 64 / 4;   // blocks per wave at most
    auto copy_q = [&](int t) {
        const float *qbase = q + (size_t)t * q_stride + (size_t)kvh * gqa * hd;
#pragma unroll
        for (int k = 0; k < QB; k++) {
            const int b = wave + 4 * k;
            if (b < nqb) copy_to_lds16(qbase + 4 * min(64 * b + lane, nqq - 1), qq + 64 * b);
        }
    };
    copy_q(t0);
    // K: chunk c is 8 blocks of 8 rows; wave w copies blocks 2w and 2w + 1
    // (the rows of the last token; an earlier token ignores those past its own)
    const float *kbase = kc + (size_t)p0 * kvd + (size_t)kvh * hd;
#pragma unroll
    for (int c = 0; c < NCH; c++) {
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int b = 2 * wave + r, row = 8 * b + (lane >> 3);
            const int j = (lane & 7) ^ ((row >> 1) & 7);
            const int cq = min(SC_CQ * c + j, nv - 1);
            copy_to_lds16(kbase + (size_t)min(row, pn_last - 1) * kvd + 4 * cq,
                          kq(c) + 8 * b * SC_CQ);
        }
    }
    const bool full = nv == NCH * SC_CQ;            // (uniform) every chunk whole
    constexpr int HW = ATT_MAXG / 4;                // heads per wave at most
    const float scale = fox_div(1.0f, fox_sqrtf((float)hd));
    for (int t = t0; t < t_end; t++) {
        const int upto = upto_of(t);
        const int pn = upto - p0 < SC_TILE ? upto - p0 : SC_TILE;
        const bool ok = lane < pn;
        const int row = ok ? lane : 0, sw = (row >> 1) & 7;
        if (t > t0) {
            // every wave is done with the previous token's query heads
            __syncthreads();
            copy_q(t);
        }
        float a[HW];
#pragma unroll
        for (int h = 0; h < HW; h++) a[h] = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            // this wave's copies of chunk c (and the query heads) are in once
            // at most 2 (NCH - 1 - c) copies are pending (later tokens: only
            // their query heads are pending); the barrier covers the other
            // waves' copies
            if (t == t0) {
                wait_vmcnt(2 * (NCH - 1 - c));
            } else if (c == 0) {
                wait_vmcnt(0);
            }
            if (t == t0 || c == 0) {
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
            }
            const float4 *kr = kq(c) + row * SC_CQ;
#pragma unroll
            for (int h = 0; h < HW; h++) {
                const int g = wave + 4 * h;
                if (g < gqa) {
                    const float4 *qr = qq + g * nv + SC_CQ * c;
                    a[h] = full ? sc_chunk<true>(a[h], qr, kr, sw, c, nv)
                                : sc_chunk<false>(a[h], qr, kr, sw, c, nv);
                }
            }
        }
#pragma unroll
        for (int h = 0; h < HW; h++) {
            const int g = wave + 4 * h;
            if (g < gqa) {
                const float sc = a[h] * scale;
                const int hh = kvh * gqa + g;
                if (ok) att[((size_t)t * n_head + hh) * att_stride + p0 + lane] = sc;
                // tile maximum, NaN never taken
                const float m = wave_reduce((ok && sc == sc) ? sc : -INFINITY, -INFINITY,
                                            [](float x, float y) { return y > x ? y : x; });
                if (lane == 0) tmax[((size_t)t * n_head + hh) * n_tiles + tile] = m;
            }
        }
    }
}

__global__ __launch_bounds__(256) void attn_softmax_x(float *__restrict__ att,
                                                      size_t att_stride,
                                                      const float *__restrict__ tmax,
                                                      int n_tiles, int n_head,
                                                      const uint32_t *__restrict__ pos,
                                                      int n_ctx)
{
    extern __shared__ float4 e4[];
    float *e = (float *)e4;
    __shared__ float red[4];
    __shared__ float inv_s;
    __shared__ int norm;
    const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    const int upto = (int)min((size_t)pos[0] + (size_t)t + 1, (size_t)n_ctx);
    const int used = (upto + SC_TILE - 1) / SC_TILE;
    float *row = att + ((size_t)t * n_head + h) * att_stride;
    const float *tm = tmax + ((size_t)t * n_head + h) * n_tiles;
    float m = -INFINITY;
    for (int i = tid; i < used; i += 256) {
        const float v = tm[i];
        m = v > m ? v : m;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float w = __shfl_xor(m, o);
        m = w > m ? w : m;
    }
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    // src/ops.c:26-30: max starts at x[0] and moves on a strict '>', so a
    // NaN first score stays the maximum; otherwise NaNs are skipped
    float mx = red[0];
    for (int w = 1; w < 4; w++) mx = red[w] > mx ? red[w] : mx;
    const float s0 = row[0];
    if (s0 != s0) mx = s0;
    for (int j = tid; j < upto; j += 256) e[j] = fox_expf(row[j] - mx);
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        int j = 0;
        for (; j + 16 <= upto; j += 16) {
            const float4 a = *(const float4 *)(e + j), b = *(const float4 *)(e + j + 4);
            const float4 c = *(const float4 *)(e + j + 8), d = *(const float4 *)(e + j + 12);
            sum = sum + a.x; sum = sum + a.y; sum = sum + a.z; sum = sum + a.w;
            sum = sum + b.x; sum = sum + b.y; sum = sum + b.z; sum = sum + b.w;
            sum = sum + c.x; sum = sum + c.y; sum = sum + c.z; sum = sum + c.w;
            sum = sum + d.x; sum = sum + d.y; sum = sum + d.z; sum = sum + d.w;
        }
        for (; j < upto; j++) sum = sum + e[j];
        norm = sum > 0.0f;
        inv_s = norm ? fox_div(1.0f, sum) : 1.0f;
    }
    __syncthreads();
    const float inv = inv_s;
    const int nrm = norm;
    for (int j = tid; j < upto; j += 256) row[j] = nrm ? e[j] * inv : e[j];
}

// One wave per (kv head, column slice, token).  Lane = (query head g of the
// kv head's group, column d); the wave covers gqa heads x (64 / gqa) columns.
#define VX_U 8

__device__ __forceinline__ float vx_quad(float acc, float4 a, float4 v)
{
    acc = acc + a.x * v.x;
    acc = acc + a.y * v.y;
    acc = acc + a.z * v.z;
    acc = acc + a.w * v.w;
    return acc;
}

__global__ __launch_bounds__(64) void attn_values_x(const float *__restrict__ att,
                                                    size_t att_stride,
                                                    const float *__restrict__ vc, int n_head,
                                                    int n_head_kv, int hd, int ds,
                                                    const uint32_t *__restrict__ pos,
                                                    int n_ctx, float *__restrict__ out,
                                                    size_t out_stride)
{
    const int lane = threadIdx.x, t = blockIdx.y;
    const int gqa = n_head / n_head_kv, kvd = n_head_kv * hd;
    const int n_sl = (hd + ds - 1) / ds;
    const int kvh = blockIdx.x / n_sl, sl = blockIdx.x - kvh * n_sl;
    const int g = lane / ds, d = sl * ds + (lane - g * ds);
    if (g >= gqa || d >= hd) return;
    const int h = kvh * gqa + g;
    const int upto = (int)min((size_t)pos[0] + (size_t)t + 1, (size_t)n_ctx);
    const int nq = upto >> 2;
    const float4 *ap = (const float4 *)(att + ((size_t)t * n_head + h) * att_stride);
    const float4 *vp = (const float4 *)vc + (size_t)kvh * hd + d;   // quad jq at vp[jq * kvd]
    float acc = 0.0f;
    int jq = 0;
    if (nq >= 2 * VX_U) {
        float4 va[VX_U], aa[VX_U], vb[VX_U], ab[VX_U];
#pragma unroll
        for (int u = 0; u < VX_U; u++) {
            va[u] = vp[(size_t)u * kvd];
            aa[u] = ap[u];
        }
        for (; jq + 2 * VX_U <= nq; jq += 2 * VX_U) {
#pragma unroll
            for (int u = 0; u < VX_U; u++) {
                vb[u] = vp[(size_t)(jq + VX_U + u) * kvd];
                ab[u] = ap[jq + VX_U + u];
            }
#pragma unroll
            for (int u = 0; u < VX_U; u++) acc = vx_quad(acc, aa[u], va[u]);
#pragma unroll
            for (int u = 0; u < VX_U; u++) {
                // the next pair's first half, clamped inside the visible rows
                const int k = jq + 2 * VX_U + u < nq ? jq + 2 * VX_U + u : nq - 1;
                va[u] = vp[(size_t)k * kvd];
                aa[u] = ap[k];
            }
#pragma unroll
            for (int u = 0; u < VX_U; u++) acc = vx_quad(acc, ab[u], vb[u]);
        }
    }
    for (; jq < nq; jq++) acc = vx_quad(acc, ap[jq], vp[(size_t)jq * kvd]);
    const float *as = (const float *)(ap + nq);
    const float *vs = (const float *)(vp + (size_t)nq * kvd);
    for (int r = 0; r < (upto & 3); r++) acc = acc + as[r] * vs[r];
    out[(size_t)t * out_stride + (size_t)h * hd + d] = acc;
}

// ---- fused softmax + values (exact order), one workgroup per (kv head,
// column slice, token), 16 waves; the kv head's G query heads x 64/G columns
// make the 64 lanes of wave 0:
//   waves 0-3: head maxima from the per-tile maxima (the scores themselves
//     are already on their way to the loader waves);
//   loader waves: e_j = expf(s_j - max) into LDS for the G heads, in rounds of
//     SV_EXR positions, each round counted when a wave completes it;
//   wave 0: one lane per head runs the position-order sum, round by round as
//     the rounds complete, then 1/sum;
//   loader waves: stream the slice's V columns (each 16-byte quad loaded once,
//     two 64-position tiles in flight per wave from the start of the kernel),
//     multiply by the G heads' a_j and hand the products to wave 0 through a
//     ring of LDS stages;
//   wave 0: one lane per (head, column) adds the products in position order.
// Stages are handed over with workgroup-scope release/acquire flags in LDS;
// every wait is bounded (a wave that times out writes NaN, sets its bit in the
// device error word and leaves).
#define SV_WAVES 16
#define SV_QT 16                    // quads (4 positions) per stage
#define SV_NP_MAX 8                 // product stages: as many as fit beside the weights
#define SV_NP_MIN 3
#define SV_LOADERS 12               // waves 1-3, 5-7, 9-11, 13-15
#define SV_LDS_MAX (159 * 1024)     // dynamic LDS of the kernel (160 KB less its static part)
#define SV_STAGE (SV_QT * 64 * 16)  // bytes per product stage
#define SV_EXR (SV_LOADERS * 64)    // positions per exp round
#define SV_EXP_PF 3                 // exp rounds whose scores are loaded up front
#define SV_VPF 8                    // product units of V in flight per loader
#define SV_SPIN (1 << 22)
#define SV_IDLE_SLEEP 2             // s_sleep units (64 clocks each) between idle polls

// v of lane (quad base + sel) for each lane, sel from a quad_perm control
// word known at compile time (DPP, no LDS traffic)
__device__ __forceinline__ float dpp_bcast(float v, int ctl)
{
    switch (ctl) {
    case 0x00: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x00, 0xF, 0xF, false));
    case 0x55: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x55, 0xF, 0xF, false));
    case 0xAA: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xAA, 0xF, 0xF, false));
    case 0xFF: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xFF, 0xF, 0xF, false));
    case 0xA0: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xA0, 0xF, 0xF, false));
    default:   return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xF5, 0xF, 0xF, false));
    }
}

// Hand-over flags live in LDS and guard LDS data only, so the fences order
// LDS accesses only: global loads a wave has in flight stay in flight.
__device__ __forceinline__ int sv_load(int *flag)
{
    return __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// (read as a wave-uniform value: tests on it are then scalar branches and
// the loops around them stay uniform)
__device__ __forceinline__ int sv_peek(int *flag)
{
    return __builtin_amdgcn_readfirstlane(sv_load(flag));
}

// (a tight loop: waves that poll with s_sleep 1 between reads slow the
// dependent adds of a wave on another SIMD by about a tenth; polling
// without a sleep does not)
__device__ __forceinline__ bool sv_wait_ge(int *flag, int v)
{
    for (int n = 0; n < SV_SPIN; n++) {
        if (sv_peek(flag) >= v) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
            return true;
        }
    }
    return false;
}

// The same for waves that are not on the chains' critical path: a read every
// few hundred cycles, so that their polling does not queue ahead of the
// chain wave's LDS reads
__device__ __forceinline__ bool sv_wait_ge_idle(int *flag, int v)
{
    for (int n = 0; n < SV_SPIN; n++) {
        if (sv_peek(flag) >= v) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
            return true;
        }
        __builtin_amdgcn_s_sleep(SV_IDLE_SLEEP);
    }
    return false;
}

// a timed-out wait reports itself in the device error word (read by the
// host after the pass: fox_gpu_take_error)
__device__ __forceinline__ void sv_error(unsigned *err, unsigned bit)
{
    __hip_atomic_fetch_or(err, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void sv_signal(int *flag, int v)
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __hip_atomic_store(flag, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// acc + x_0 + x_1 + ... over 4 * nq floats of LDS, in index order.  A
// dependent add chain is bound by the wave's instruction issue, so the
// operand reads must cost as few instructions as possible: banks of eight
// quads alternate, the eight reads of one bank (ds_read_b128 at constant
// offsets from one address, one wait) in flight while the other bank's 32
// adds run.  One block of 64 quads is one asm statement (reads, waits and
// adds, v64-v127 its banks): compiled from C, the reads of such a block are
// hoisted and reordered across the adds, and a bank carried from one loop
// iteration to the next is copied every iteration.  LDS reads complete in
// order, so lgkmcnt(8) after a bank's reads means the previous bank is in.
// Read-write operands are early-clobber ("+&"): the asm writes them before
// it has read every input, so no input may share their registers (an input
// equal to acc's initial bits would otherwise be given acc's register).
// (Measured on gfx950, one wave: 2.5 ns per add this way, 4 ns with a wait
// and a read between every four adds, 1.8 ns from registers.)
// the LDS address of a pointer into LDS
__device__ __forceinline__ uint32_t lds_addr(const void *p)
{
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)p;
}

__device__ __forceinline__ float chain64_lds(float acc, const float4 *q)
{
    const uint32_t p = lds_addr(q);
    asm volatile(
        "ds_read_b128 v[64:67], %[p] offset:0\n" "ds_read_b128 v[68:71], %[p] offset:16\n" "ds_read_b128 v[72:75], %[p] offset:32\n" "ds_read_b128 v[76:79], %[p] offset:48\n"
        "ds_read_b128 v[80:83], %[p] offset:64\n" "ds_read_b128 v[84:87], %[p] offset:80\n" "ds_read_b128 v[88:91], %[p] offset:96\n" "ds_read_b128 v[92:95], %[p] offset:112\n"
        "ds_read_b128 v[96:99], %[p] offset:128\n" "ds_read_b128 v[100:103], %[p] offset:144\n" "ds_read_b128 v[104:107], %[p] offset:160\n" "ds_read_b128 v[108:111], %[p] offset:176\n"
        "ds_read_b128 v[112:115], %[p] offset:192\n" "ds_read_b128 v[116:119], %[p] offset:208\n" "ds_read_b128 v[120:123], %[p] offset:224\n" "ds_read_b128 v[124:127], %[p] offset:240\n"
        "s_waitcnt lgkmcnt(8)\n" "v_add_f32 %[acc], %[acc], v64\n" "v_add_f32 %[acc], %[acc], v65\n" "v_add_f32 %[acc], %[acc], v66\n"
        "v_add_f32 %[acc], %[acc], v67\n" "v_add_f32 %[acc], %[acc], v68\n" "v_add_f32 %[acc], %[acc], v69\n" "v_add_f32 %[acc], %[acc], v70\n"
        "v_add_f32 %[acc], %[acc], v71\n" "v_add_f32 %[acc], %[acc], v72\n" "v_add_f32 %[acc], %[acc], v73\n" "v_add_f32 %[acc], %[acc], v74\n"
        "v_add_f32 %[acc], %[acc], v75\n" "v_add_f32 %[acc], %[acc], v76\n" "v_add_f32 %[acc], %[acc], v77\n" "v_add_f32 %[acc], %[acc], v78\n"
        "v_add_f32 %[acc], %[acc], v79\n" "v_add_f32 %[acc], %[acc], v80\n" "v_add_f32 %[acc], %[acc], v81\n" "v_add_f32 %[acc], %[acc], v82\n"
        "v_add_f32 %[acc], %[acc], v83\n" "v_add_f32 %[acc], %[acc], v84\n" "v_add_f32 %[acc], %[acc], v85\n" "v_add_f32 %[acc], %[acc], v86\n"
        "v_add_f32 %[acc], %[acc], v87\n" "v_add_f32 %[acc], %[acc], v88\n" "v_add_f32 %[acc], %[acc], v89\n" "v_add_f32 %[acc], %[acc], v90\n"
        "v_add_f32 %[acc], %[acc], v91\n" "v_add_f32 %[acc], %[acc], v92\n" "v_add_f32 %[acc], %[acc], v93\n" "v_add_f32 %[acc], %[acc], v94\n"
        "v_add_f32 %[acc], %[acc], v95\n" "ds_read_b128 v[64:67], %[p] offset:256\n" "ds_read_b128 v[68:71], %[p] offset:272\n" "ds_read_b128 v[72:75], %[p] offset:288\n"
        "ds_read_b128 v[76:79], %[p] offset:304\n" "ds_read_b128 v[80:83], %[p] offset:320\n" "ds_read_b128 v[84:87], %[p] offset:336\n" "ds_read_b128 v[88:91], %[p] offset:352\n"
        "ds_read_b128 v[92:95], %[p] offset:368\n" "s_waitcnt lgkmcnt(8)\n" "v_add_f32 %[acc], %[acc], v96\n" "v_add_f32 %[acc], %[acc], v97\n"
        "v_add_f32 %[acc], %[acc], v98\n" "v_add_f32 %[acc], %[acc], v99\n" "v_add_f32 %[acc], %[acc], v100\n" "v_add_f32 %[acc], %[acc], v101\n"
        "v_add_f32 %[acc], %[acc], v102\n" "v_add_f32 %[acc], %[acc], v103\n" "v_add_f32 %[acc], %[acc], v104\n" "v_add_f32 %[acc], %[acc], v105\n"
        "v_add_f32 %[acc], %[acc], v106\n" "v_add_f32 %[acc], %[acc], v107\n" "v_add_f32 %[acc], %[acc], v108\n" "v_add_f32 %[acc], %[acc], v109\n"
        "v_add_f32 %[acc], %[acc], v110\n" "v_add_f32 %[acc], %[acc], v111\n" "v_add_f32 %[acc], %[acc], v112\n" "v_add_f32 %[acc], %[acc], v113\n"
        "v_add_f32 %[acc], %[acc], v114\n" "v_add_f32 %[acc], %[acc], v115\n" "v_add_f32 %[acc], %[acc], v116\n" "v_add_f32 %[acc], %[acc], v117\n"
        "v_add_f32 %[acc], %[acc], v118\n" "v_add_f32 %[acc], %[acc], v119\n" "v_add_f32 %[acc], %[acc], v120\n" "v_add_f32 %[acc], %[acc], v121\n"
        "v_add_f32 %[acc], %[acc], v122\n" "v_add_f32 %[acc], %[acc], v123\n" "v_add_f32 %[acc], %[acc], v124\n" "v_add_f32 %[acc], %[acc], v125\n"
        "v_add_f32 %[acc], %[acc], v126\n" "v_add_f32 %[acc], %[acc], v127\n" "ds_read_b128 v[96:99], %[p] offset:384\n" "ds_read_b128 v[100:103], %[p] offset:400\n"
        "ds_read_b128 v[104:107], %[p] offset:416\n" "ds_read_b128 v[108:111], %[p] offset:432\n" "ds_read_b128 v[112:115], %[p] offset:448\n" "ds_read_b128 v[116:119], %[p] offset:464\n"
        "ds_read_b128 v[120:123], %[p] offset:480\n" "ds_read_b128 v[124:127], %[p] offset:496\n" "s_waitcnt lgkmcnt(8)\n" "v_add_f32 %[acc], %[acc], v64\n"
        "v_add_f32 %[acc], %[acc], v65\n" "v_add_f32 %[acc], %[acc], v66\n" "v_add_f32 %[acc], %[acc], v67\n" "v_add_f32 %[acc], %[acc], v68\n"
        "v_add_f32 %[acc], %[acc], v69\n" "v_add_f32 %[acc], %[acc], v70\n" "v_add_f32 %[acc], %[acc], v71\n" "v_add_f32 %[acc], %[acc], v72\n"
        "v_add_f32 %[acc], %[acc], v73\n" "v_add_f32 %[acc], %[acc], v74\n" "v_add_f32 %[acc], %[acc], v75\n" "v_add_f32 %[acc], %[acc], v76\n"
        "v_add_f32 %[acc], %[acc], v77\n" "v_add_f32 %[acc], %[acc], v78\n" "v_add_f32 %[acc], %[acc], v79\n" "v_add_f32 %[acc], %[acc], v80\n"
        "v_add_f32 %[acc], %[acc], v81\n" "v_add_f32 %[acc], %[acc], v82\n" "v_add_f32 %[acc], %[acc], v83\n" "v_add_f32 %[acc], %[acc], v84\n"
        "v_add_f32 %[acc], %[acc], v85\n" "v_add_f32 %[acc], %[acc], v86\n" "v_add_f32 %[acc], %[acc], v87\n" "v_add_f32 %[acc], %[acc], v88\n"
        "v_add_f32 %[acc], %[acc], v89\n" "v_add_f32 %[acc], %[acc], v90\n" "v_add_f32 %[acc], %[acc], v91\n" "v_add_f32 %[acc], %[acc], v92\n"
        "v_add_f32 %[acc], %[acc], v93\n" "v_add_f32 %[acc], %[acc], v94\n" "v_add_f32 %[acc], %[acc], v95\n" "ds_read_b128 v[64:67], %[p] offset:512\n"
        "ds_read_b128 v[68:71], %[p] offset:528\n" "ds_read_b128 v[72:75], %[p] offset:544\n" "ds_read_b128 v[76:79], %[p] offset:560\n" "ds_read_b128 v[80:83], %[p] offset:576\n"
        "ds_read_b128 v[84:87], %[p] offset:592\n" "ds_read_b128 v[88:91], %[p] offset:608\n" "ds_read_b128 v[92:95], %[p] offset:624\n" "s_waitcnt lgkmcnt(8)\n"
        "v_add_f32 %[acc], %[acc], v96\n" "v_add_f32 %[acc], %[acc], v97\n" "v_add_f32 %[acc], %[acc], v98\n" "v_add_f32 %[acc], %[acc], v99\n"
        "v_add_f32 %[acc], %[acc], v100\n" "v_add_f32 %[acc], %[acc], v101\n" "v_add_f32 %[acc], %[acc], v102\n" "v_add_f32 %[acc], %[acc], v103\n"
        "v_add_f32 %[acc], %[acc], v104\n" "v_add_f32 %[acc], %[acc], v105\n" "v_add_f32 %[acc], %[acc], v106\n" "v_add_f32 %[acc], %[acc], v107\n"
        "v_add_f32 %[acc], %[acc], v108\n" "v_add_f32 %[acc], %[acc], v109\n" "v_add_f32 %[acc], %[acc], v110\n" "v_add_f32 %[acc], %[acc], v111\n"
        "v_add_f32 %[acc], %[acc], v112\n" "v_add_f32 %[acc], %[acc], v113\n" "v_add_f32 %[acc], %[acc], v114\n" "v_add_f32 %[acc], %[acc], v115\n"
        "v_add_f32 %[acc], %[acc], v116\n" "v_add_f32 %[acc], %[acc], v117\n" "v_add_f32 %[acc], %[acc], v118\n" "v_add_f32 %[acc], %[acc], v119\n"
        "v_add_f32 %[acc], %[acc], v120\n" "v_add_f32 %[acc], %[acc], v121\n" "v_add_f32 %[acc], %[acc], v122\n" "v_add_f32 %[acc], %[acc], v123\n"
        "v_add_f32 %[acc], %[acc], v124\n" "v_add_f32 %[acc], %[acc], v125\n" "v_add_f32 %[acc], %[acc], v126\n" "v_add_f32 %[acc], %[acc], v127\n"
        "ds_read_b128 v[96:99], %[p] offset:640\n" "ds_read_b128 v[100:103], %[p] offset:656\n" "ds_read_b128 v[104:107], %[p] offset:672\n" "ds_read_b128 v[108:111], %[p] offset:688\n"
        "ds_read_b128 v[112:115], %[p] offset:704\n" "ds_read_b128 v[116:119], %[p] offset:720\n" "ds_read_b128 v[120:123], %[p] offset:736\n" "ds_read_b128 v[124:127], %[p] offset:752\n"
        "s_waitcnt lgkmcnt(8)\n" "v_add_f32 %[acc], %[acc], v64\n" "v_add_f32 %[acc], %[acc], v65\n" "v_add_f32 %[acc], %[acc], v66\n"
        "v_add_f32 %[acc], %[acc], v67\n" "v_add_f32 %[acc], %[acc], v68\n" "v_add_f32 %[acc], %[acc], v69\n" "v_add_f32 %[acc], %[acc], v70\n"
        "v_add_f32 %[acc], %[acc], v71\n" "v_add_f32 %[acc], %[acc], v72\n" "v_add_f32 %[acc], %[acc], v73\n" "v_add_f32 %[acc], %[acc], v74\n"
        "v_add_f32 %[acc], %[acc], v75\n" "v_add_f32 %[acc], %[acc], v76\n" "v_add_f32 %[acc], %[acc], v77\n" "v_add_f32 %[acc], %[acc], v78\n"
        "v_add_f32 %[acc], %[acc], v79\n" "v_add_f32 %[acc], %[acc], v80\n" "v_add_f32 %[acc], %[acc], v81\n" "v_add_f32 %[acc], %[acc], v82\n"
        "v_add_f32 %[acc], %[acc], v83\n" "v_add_f32 %[acc], %[acc], v84\n" "v_add_f32 %[acc], %[acc], v85\n" "v_add_f32 %[acc], %[acc], v86\n"
        "v_add_f32 %[acc], %[acc], v87\n" "v_add_f32 %[acc], %[acc], v88\n" "v_add_f32 %[acc], %[acc], v89\n" "v_add_f32 %[acc], %[acc], v90\n"
        "v_add_f32 %[acc], %[acc], v91\n" "v_add_f32 %[acc], %[acc], v92\n" "v_add_f32 %[acc], %[acc], v93\n" "v_add_f32 %[acc], %[acc], v94\n"
        "v_add_f32 %[acc], %[acc], v95\n" "ds_read_b128 v[64:67], %[p] offset:768\n" "ds_read_b128 v[68:71], %[p] offset:784\n" "ds_read_b128 v[72:75], %[p] offset:800\n"
        "ds_read_b128 v[76:79], %[p] offset:816\n" "ds_read_b128 v[80:83], %[p] offset:832\n" "ds_read_b128 v[84:87], %[p] offset:848\n" "ds_read_b128 v[88:91], %[p] offset:864\n"
        "ds_read_b128 v[92:95], %[p] offset:880\n" "s_waitcnt lgkmcnt(8)\n" "v_add_f32 %[acc], %[acc], v96\n" "v_add_f32 %[acc], %[acc], v97\n"
        "v_add_f32 %[acc], %[acc], v98\n" "v_add_f32 %[acc], %[acc], v99\n" "v_add_f32 %[acc], %[acc], v100\n" "v_add_f32 %[acc], %[acc], v101\n"
        "v_add_f32 %[acc], %[acc], v102\n" "v_add_f32 %[acc], %[acc], v103\n" "v_add_f32 %[acc], %[acc], v104\n" "v_add_f32 %[acc], %[acc], v105\n"
        "v_add_f32 %[acc], %[acc], v106\n" "v_add_f32 %[acc], %[acc], v107\n" "v_add_f32 %[acc], %[acc], v108\n" "v_add_f32 %[acc], %[acc], v109\n"
        "v_add_f32 %[acc], %[acc], v110\n" "v_add_f32 %[acc], %[acc], v111\n" "v_add_f32 %[acc], %[acc], v112\n" "v_add_f32 %[acc], %[acc], v113\n"
        "v_add_f32 %[acc], %[acc], v114\n" "v_add_f32 %[acc], %[acc], v115\n" "v_add_f32 %[acc], %[acc], v116\n" "v_add_f32 %[acc], %[acc], v117\n"
        "v_add_f32 %[acc], %[acc], v118\n" "v_add_f32 %[acc], %[acc], v119\n" "v_add_f32 %[acc], %[acc], v120\n" "v_add_f32 %[acc], %[acc], v121\n"
        "v_add_f32 %[acc], %[acc], v122\n" "v_add_f32 %[acc], %[acc], v123\n" "v_add_f32 %[acc], %[acc], v124\n" "v_add_f32 %[acc], %[acc], v125\n"
        "v_add_f32 %[acc], %[acc], v126\n" "v_add_f32 %[acc], %[acc], v127\n" "ds_read_b128 v[96:99], %[p] offset:896\n" "ds_read_b128 v[100:103], %[p] offset:912\n"
        "ds_read_b128 v[104:107], %[p] offset:928\n" "ds_read_b128 v[108:111], %[p] offset:944\n" "ds_read_b128 v[112:115], %[p] offset:960\n" "ds_read_b128 v[116:119], %[p] offset:976\n"
        "ds_read_b128 v[120:123], %[p] offset:992\n" "ds_read_b128 v[124:127], %[p] offset:1008\n" "s_waitcnt lgkmcnt(8)\n" "v_add_f32 %[acc], %[acc], v64\n"
        "v_add_f32 %[acc], %[acc], v65\n" "v_add_f32 %[acc], %[acc], v66\n" "v_add_f32 %[acc], %[acc], v67\n" "v_add_f32 %[acc], %[acc], v68\n"
        "v_add_f32 %[acc], %[acc], v69\n" "v_add_f32 %[acc], %[acc], v70\n" "v_add_f32 %[acc], %[acc], v71\n" "v_add_f32 %[acc], %[acc], v72\n"
        "v_add_f32 %[acc], %[acc], v73\n" "v_add_f32 %[acc], %[acc], v74\n" "v_add_f32 %[acc], %[acc], v75\n" "v_add_f32 %[acc], %[acc], v76\n"
        "v_add_f32 %[acc], %[acc], v77\n" "v_add_f32 %[acc], %[acc], v78\n" "v_add_f32 %[acc], %[acc], v79\n" "v_add_f32 %[acc], %[acc], v80\n"
        "v_add_f32 %[acc], %[acc], v81\n" "v_add_f32 %[acc], %[acc], v82\n" "v_add_f32 %[acc], %[acc], v83\n" "v_add_f32 %[acc], %[acc], v84\n"
        "v_add_f32 %[acc], %[acc], v85\n" "v_add_f32 %[acc], %[acc], v86\n" "v_add_f32 %[acc], %[acc], v87\n" "v_add_f32 %[acc], %[acc], v88\n"
        "v_add_f32 %[acc], %[acc], v89\n" "v_add_f32 %[acc], %[acc], v90\n" "v_add_f32 %[acc], %[acc], v91\n" "v_add_f32 %[acc], %[acc], v92\n"
        "v_add_f32 %[acc], %[acc], v93\n" "v_add_f32 %[acc], %[acc], v94\n" "v_add_f32 %[acc], %[acc], v95\n" "s_waitcnt lgkmcnt(0)\n"
        "v_add_f32 %[acc], %[acc], v96\n" "v_add_f32 %[acc], %[acc], v97\n" "v_add_f32 %[acc], %[acc], v98\n" "v_add_f32 %[acc], %[acc], v99\n"
        "v_add_f32 %[acc], %[acc], v100\n" "v_add_f32 %[acc], %[acc], v101\n" "v_add_f32 %[acc], %[acc], v102\n" "v_add_f32 %[acc], %[acc], v103\n"
        "v_add_f32 %[acc], %[acc], v104\n" "v_add_f32 %[acc], %[acc], v105\n" "v_add_f32 %[acc], %[acc], v106\n" "v_add_f32 %[acc], %[acc], v107\n"
        "v_add_f32 %[acc], %[acc], v108\n" "v_add_f32 %[acc], %[acc], v109\n" "v_add_f32 %[acc], %[acc], v110\n" "v_add_f32 %[acc], %[acc], v111\n"
        "v_add_f32 %[acc], %[acc], v112\n" "v_add_f32 %[acc], %[acc], v113\n" "v_add_f32 %[acc], %[acc], v114\n" "v_add_f32 %[acc], %[acc], v115\n"
        "v_add_f32 %[acc], %[acc], v116\n" "v_add_f32 %[acc], %[acc], v117\n" "v_add_f32 %[acc], %[acc], v118\n" "v_add_f32 %[acc], %[acc], v119\n"
        "v_add_f32 %[acc], %[acc], v120\n" "v_add_f32 %[acc], %[acc], v121\n" "v_add_f32 %[acc], %[acc], v122\n" "v_add_f32 %[acc], %[acc], v123\n"
        "v_add_f32 %[acc], %[acc], v124\n" "v_add_f32 %[acc], %[acc], v125\n" "v_add_f32 %[acc], %[acc], v126\n" "v_add_f32 %[acc], %[acc], v127\n"
        : [acc] "+&v"(acc)
        : [p] "v"(p)
        : "v64", "v65", "v66", "v67", "v68", "v69", "v70", "v71",
          "v72", "v73", "v74", "v75", "v76", "v77", "v78", "v79",
          "v80", "v81", "v82", "v83", "v84", "v85", "v86", "v87",
          "v88", "v89", "v90", "v91", "v92", "v93", "v94", "v95",
          "v96", "v97", "v98", "v99", "v100", "v101", "v102", "v103",
          "v104", "v105", "v106", "v107", "v108", "v109", "v110", "v111",
          "v112", "v113", "v114", "v115", "v116", "v117", "v118", "v119",
          "v120", "v121", "v122", "v123", "v124", "v125", "v126", "v127",
          "memory");
    return acc;
}

__device__ __forceinline__ float chain_add_lds(float acc, const float4 *p, int nq)
{
    int q = 0;
    for (; q + 64 <= nq; q += 64) acc = chain64_lds(acc, p + q);
    for (; q < nq; q++) {
        const float4 v = p[q];
        acc = acc + v.x; acc = acc + v.y; acc = acc + v.z; acc = acc + v.w;
    }
    return acc;
}

template <int G>
__global__ __launch_bounds__(SV_WAVES * 64) void attn_sv_x(
    const float *__restrict__ att, size_t att_stride, const float *__restrict__ tmax, int n_tiles,
    const float *__restrict__ vc, int n_head, int n_head_kv, int hd,
    const uint32_t *__restrict__ pos, int n_ctx, float *__restrict__ out, size_t out_stride,
    int np, unsigned *err)
{
    constexpr int DS = 64 / G;               // columns per slice
    constexpr int NLD = SV_QT / G;           // product units per tile (G quads each)
    extern __shared__ float4 sv_lds[];
    float4 *ring = sv_lds;                                  // [np][SV_QT][64]
    float *e = (float *)(sv_lds + np * SV_QT * 64);         // [G][att_stride + 4]
    __shared__ float mx_s[G], inv_s[G];
    __shared__ int nrm_s[G];
    __shared__ uint64_t tab[32];
    __shared__ int ready[SV_NP_MAX], cnt[SV_NP_MAX], consumed, a_ready, e_done;

    const int tid = threadIdx.x, lane = tid & 63, wave = wave_index();
    const int kvd = n_head_kv * hd;
    const int n_sl = (hd + DS - 1) / DS;
    const int kvh = blockIdx.x / n_sl, sl = blockIdx.x - kvh * n_sl, t = blockIdx.y;
    const int upto = (int)min((size_t)pos[0] + (size_t)t + 1, (size_t)n_ctx);
    const int nq = upto >> 2, rem = upto & 3, nq_all = (upto + 3) >> 2;
    const int ntile = (nq_all + SV_QT - 1) / SV_QT;
    const int estr = (int)att_stride + 4;        // padded: heads in different banks
    const float *srow = att + ((size_t)t * n_head + (size_t)kvh * G) * att_stride;

    // loaders: lane -> (quad lq of each group of G quads, column ld)
    const int lq = lane / DS, ld = sl * DS + (lane - lq * DS);
    const float4 *v4 = (const float4 *)vc + kvh * hd + (ld < hd ? ld : sl * DS);
    const bool loader = (wave & 3) != 0;     // waves on SIMD 0 do not load
    const int li = wave - 1 - (wave >> 2);
    const int nunit = ntile * NLD;
    // V of the loader's units li + SV_LOADERS m, SV_VPF of them in flight
    // (unit u: quads (u % NLD) G .. + G - 1 of tile u / NLD; the lane's
    // quad is the lq-th of them)
    auto v_of = [&](int u) -> float4 {
        const int i = u / NLD, k = u - i * NLD;
        const int jq = min(i * SV_QT + k * G + lq, nq_all - 1);
        return v4[(size_t)jq * kvd];
    };
    float4 vq[SV_VPF];

    // scores of the first SV_EXP_PF exp rounds, loaded first: a wave's loads
    // complete in order, and these are needed as soon as the maxima are
    // known, the V tiles only after the softmax sum
    const int ex0 = li * 64 + lane;                 // loader's position in a round
    float sc[SV_EXP_PF][G];
    if (loader) {
#pragma unroll
        for (int k = 0; k < SV_EXP_PF; k++) {
            const int p = k * SV_EXR + ex0;
#pragma unroll
            for (int gg = 0; gg < G; gg++)
                sc[k][gg] = srow[(size_t)gg * att_stride + (p < upto ? p : 0)];
        }
    }
    if (loader) {
#pragma unroll
        for (int m = 0; m < SV_VPF; m++) vq[m] = v_of(min(li + m * SV_LOADERS, nunit - 1));
    }

    // ---- head maxima (src/ops.c:26-30: a NaN first score stays the max),
    // by the waves that load no V (wave 4 n takes heads n, n + 4): their
    // tile-maximum loads are not queued behind V loads
    if (!loader) {
        for (int hg = wave >> 2; hg < G; hg += 4) {
            const float *tm = tmax + ((size_t)t * n_head + (size_t)kvh * G + hg) * n_tiles;
            const int used = (upto + SC_TILE - 1) / SC_TILE;
            float m = -INFINITY;
            for (int i = lane; i < used; i += 64) {
                const float v = tm[i];
                m = v > m ? v : m;
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float w = __shfl_xor(m, o);
                m = w > m ? w : m;
            }
            const float s0 = srow[(size_t)hg * att_stride];
            if (lane == 0) mx_s[hg] = s0 != s0 ? s0 : m;
        }
    }
    if (tid < SV_NP_MAX) {
        ready[tid] = -1;
        cnt[tid] = 0;
    }
    if (tid < 32) tab[tid] = fox_exp2_tab[tid];
    if (tid == 0) {
        consumed = 0;
        a_ready = 0;
        e_done = 0;
    }
    __syncthreads();
    if (!loader && wave != 0) return;                // (SIMD 0 stays with wave 0)

    if (loader) {
        // ---- e_j = expf(s_j - max) (src/ops.c:31-34) in rounds of SV_EXR
        // positions; a wave counts each round it completes
        float mx[G];
#pragma unroll
        for (int gg = 0; gg < G; gg++) mx[gg] = mx_s[gg];
        auto exp_round = [&](int k, const float *scr) {
            const int p = k * SV_EXR + ex0;
            if (p < upto) {
#pragma unroll
                for (int gg = 0; gg < G; gg++) e[gg * estr + p] = fox_expf_t(scr[gg] - mx[gg], tab);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            if (lane == 0) __hip_atomic_fetch_add(&e_done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        };
#pragma unroll
        for (int k = 0; k < SV_EXP_PF; k++)
            if (k * SV_EXR < upto) exp_round(k, sc[k]);
        for (int k = SV_EXP_PF; k * SV_EXR < upto; k++) {
            const int p = k * SV_EXR + ex0;
            float s2[G];
#pragma unroll
            for (int gg = 0; gg < G; gg++) s2[gg] = srow[(size_t)gg * att_stride + (p < upto ? p : 0)];
            exp_round(k, s2);
        }
    }

    if (wave == 0) {
        // ---- softmax sums, one lane per head, position order; round k is
        // added once every loader wave has counted it
        float sum = 0.0f;
        bool eok = true;
        for (int k = 0; k * SV_EXR < upto; k++) {
            if (!sv_wait_ge(&e_done, SV_LOADERS * (k + 1))) {
                eok = false;
                break;
            }
            const int p0 = k * SV_EXR, p1 = min(upto, p0 + SV_EXR);
            if (lane < G) {
                const float *er = e + lane * estr;
                const int nqk = (p1 - p0) >> 2;
                sum = chain_add_lds(sum, (const float4 *)(er + p0), nqk);
                for (int j = p0 + 4 * nqk; j < p1; j++) sum = sum + er[j];
            }
        }
        if (!eok) {
            sum = __builtin_nanf("");
            if (lane == 0) sv_error(err, FOX_DEV_ERR_ATTN_SUM);
        }
        // a_j = e_j * (1/sum) is formed by the loaders (src/ops.c:35-38)
        if (lane < G) {
            nrm_s[lane] = sum > 0.0f;
            inv_s[lane] = sum > 0.0f ? fox_div(1.0f, sum) : 1.0f;
        }
        sv_signal(&a_ready, 1);

        // ---- value sums: lane (head g, column d) adds its products in order.
        // Whole tiles run in one asm loop (the reasons of chain64_lds): a
        // tile's second half (eight quads, v96-v127) is read while its first
        // half (v64-v95) is added, then, once tile i + 1 is marked ready, the
        // next tile's first half while the second half is added.  Tile i + 1's
        // flag is read a tile ahead (with tile i's first half) and tested
        // after tile i's first half's adds; a tile not marked by then is
        // waited for out of line (bounded: a timed-out wait clears ok, after
        // which the loop runs on without waiting and the sum is replaced by
        // NaN below).  Tile i's stage is released once all its reads are in,
        // before the next reads go out; the stage's four base addresses
        // (v56-v59) are computed once per tile.
        // Ring slots are XOR-swizzled by (quad & 3) (the loaders' four quads
        // per store fall in different banks): quad u of a stage sits at
        // lane ^ 4 (u & 3), so four base addresses cover the sixteen quads
        // with constant offsets.
        static_assert(SV_QT == 16 && SV_QT * 64 * 16 == 1 << 14 && SV_SPIN == 0x400000,
                      "the asm loop's tile size, stage size and spin limit");
        const int g = lane / DS, d = sl * DS + (lane - g * DS);
        float acc = 0.0f;
        bool ok = eok && sv_wait_ge(&ready[0], 0);
        const int nwhole = __builtin_amdgcn_readfirstlane(nq / SV_QT);
        int i = 0, st = 0;
        if (ok && nwhole > 0) {
            const uint32_t ra = lds_addr(ring);
            const uint32_t l0 = ra + ((uint32_t)lane << 4), l1 = ra + ((uint32_t)(lane ^ 4) << 4);
            const uint32_t l2 = ra + ((uint32_t)(lane ^ 8) << 4), l3 = ra + ((uint32_t)(lane ^ 12) << 4);
            const uint32_t rb = lds_addr(ready), vc = lds_addr(&consumed);
            const int npu = __builtin_amdgcn_readfirstlane(np);
            int oks = 1, so, sn, sf, si1, sp;
            uint32_t va, vv, vf;
            asm volatile(
        "v_mov_b32 v56, %[l0]\n"
        "v_mov_b32 v57, %[l1]\n"
        "v_mov_b32 v58, %[l2]\n"
        "v_mov_b32 v59, %[l3]\n"
        "ds_read_b128 v[64:67], v56 offset:0\n"
        "ds_read_b128 v[68:71], v57 offset:1024\n"
        "ds_read_b128 v[72:75], v58 offset:2048\n"
        "ds_read_b128 v[76:79], v59 offset:3072\n"
        "ds_read_b128 v[80:83], v56 offset:4096\n"
        "ds_read_b128 v[84:87], v57 offset:5120\n"
        "ds_read_b128 v[88:91], v58 offset:6144\n"
        "ds_read_b128 v[92:95], v59 offset:7168\n"
        "s_add_u32 %[si1], %[i], 1\n"
        "s_cmp_ge_u32 %[si1], %[nw]\n"
        "s_cbranch_scc1 5f\n"
        "s_add_u32 %[sn], %[st], 1\n"
        "s_cmp_eq_u32 %[sn], %[np]\n"
        "s_cselect_b32 %[sn], 0, %[sn]\n"
        "s_lshl_b32 %[sf], %[sn], 2\n"
        "v_add_u32 %[va], %[sf], %[rb]\n"
        "ds_read_b32 %[vf], %[va]\n"
        "5:\n"
        "6:\n"
        "ds_read_b128 v[96:99], v56 offset:8192\n"
        "ds_read_b128 v[100:103], v57 offset:9216\n"
        "ds_read_b128 v[104:107], v58 offset:10240\n"
        "ds_read_b128 v[108:111], v59 offset:11264\n"
        "ds_read_b128 v[112:115], v56 offset:12288\n"
        "ds_read_b128 v[116:119], v57 offset:13312\n"
        "ds_read_b128 v[120:123], v58 offset:14336\n"
        "ds_read_b128 v[124:127], v59 offset:15360\n"
        "s_add_u32 %[si1], %[i], 1\n"
        "s_add_u32 %[sn], %[st], 1\n"
        "s_cmp_eq_u32 %[sn], %[np]\n"
        "s_cselect_b32 %[sn], 0, %[sn]\n"
        "s_waitcnt lgkmcnt(8)\n"
        "v_add_f32 %[acc], %[acc], v64\n" "v_add_f32 %[acc], %[acc], v65\n" "v_add_f32 %[acc], %[acc], v66\n" "v_add_f32 %[acc], %[acc], v67\n"
        "v_add_f32 %[acc], %[acc], v68\n" "v_add_f32 %[acc], %[acc], v69\n" "v_add_f32 %[acc], %[acc], v70\n" "v_add_f32 %[acc], %[acc], v71\n"
        "v_add_f32 %[acc], %[acc], v72\n" "v_add_f32 %[acc], %[acc], v73\n" "v_add_f32 %[acc], %[acc], v74\n" "v_add_f32 %[acc], %[acc], v75\n"
        "v_add_f32 %[acc], %[acc], v76\n" "v_add_f32 %[acc], %[acc], v77\n" "v_add_f32 %[acc], %[acc], v78\n" "v_add_f32 %[acc], %[acc], v79\n"
        "v_add_f32 %[acc], %[acc], v80\n" "v_add_f32 %[acc], %[acc], v81\n" "v_add_f32 %[acc], %[acc], v82\n" "v_add_f32 %[acc], %[acc], v83\n"
        "v_add_f32 %[acc], %[acc], v84\n" "v_add_f32 %[acc], %[acc], v85\n" "v_add_f32 %[acc], %[acc], v86\n" "v_add_f32 %[acc], %[acc], v87\n"
        "v_add_f32 %[acc], %[acc], v88\n" "v_add_f32 %[acc], %[acc], v89\n" "v_add_f32 %[acc], %[acc], v90\n" "v_add_f32 %[acc], %[acc], v91\n"
        "v_add_f32 %[acc], %[acc], v92\n" "v_add_f32 %[acc], %[acc], v93\n" "v_add_f32 %[acc], %[acc], v94\n" "v_add_f32 %[acc], %[acc], v95\n"
        "s_waitcnt lgkmcnt(0)\n"
        "v_mov_b32 %[vv], %[si1]\n"
        "ds_write_b32 %[vc], %[vv]\n"
        "s_cmp_ge_u32 %[si1], %[nw]\n"
        "s_cbranch_scc1 3f\n"
        "s_cmp_eq_u32 %[ok], 0\n"
        "s_cbranch_scc1 4f\n"
        "v_readfirstlane_b32 %[sf], %[vf]\n"
        "s_cmp_lt_i32 %[sf], %[si1]\n"
        "s_cbranch_scc1 8f\n"
        "4:\n"
        "s_lshl_b32 %[so], %[sn], 14\n"
        "v_add_u32 v56, %[so], %[l0]\n"
        "v_add_u32 v57, %[so], %[l1]\n"
        "v_add_u32 v58, %[so], %[l2]\n"
        "v_add_u32 v59, %[so], %[l3]\n"
        "ds_read_b128 v[64:67], v56 offset:0\n"
        "ds_read_b128 v[68:71], v57 offset:1024\n"
        "ds_read_b128 v[72:75], v58 offset:2048\n"
        "ds_read_b128 v[76:79], v59 offset:3072\n"
        "ds_read_b128 v[80:83], v56 offset:4096\n"
        "ds_read_b128 v[84:87], v57 offset:5120\n"
        "ds_read_b128 v[88:91], v58 offset:6144\n"
        "ds_read_b128 v[92:95], v59 offset:7168\n"
        "s_add_u32 %[so], %[si1], 1\n"
        "s_cmp_ge_u32 %[so], %[nw]\n"
        "s_cbranch_scc1 3f\n"
        "s_add_u32 %[sf], %[sn], 1\n"
        "s_cmp_eq_u32 %[sf], %[np]\n"
        "s_cselect_b32 %[sf], 0, %[sf]\n"
        "s_lshl_b32 %[sf], %[sf], 2\n"
        "v_add_u32 %[va], %[sf], %[rb]\n"
        "ds_read_b32 %[vf], %[va]\n"
        "3:\n"
        "v_add_f32 %[acc], %[acc], v96\n" "v_add_f32 %[acc], %[acc], v97\n" "v_add_f32 %[acc], %[acc], v98\n" "v_add_f32 %[acc], %[acc], v99\n"
        "v_add_f32 %[acc], %[acc], v100\n" "v_add_f32 %[acc], %[acc], v101\n" "v_add_f32 %[acc], %[acc], v102\n" "v_add_f32 %[acc], %[acc], v103\n"
        "v_add_f32 %[acc], %[acc], v104\n" "v_add_f32 %[acc], %[acc], v105\n" "v_add_f32 %[acc], %[acc], v106\n" "v_add_f32 %[acc], %[acc], v107\n"
        "v_add_f32 %[acc], %[acc], v108\n" "v_add_f32 %[acc], %[acc], v109\n" "v_add_f32 %[acc], %[acc], v110\n" "v_add_f32 %[acc], %[acc], v111\n"
        "v_add_f32 %[acc], %[acc], v112\n" "v_add_f32 %[acc], %[acc], v113\n" "v_add_f32 %[acc], %[acc], v114\n" "v_add_f32 %[acc], %[acc], v115\n"
        "v_add_f32 %[acc], %[acc], v116\n" "v_add_f32 %[acc], %[acc], v117\n" "v_add_f32 %[acc], %[acc], v118\n" "v_add_f32 %[acc], %[acc], v119\n"
        "v_add_f32 %[acc], %[acc], v120\n" "v_add_f32 %[acc], %[acc], v121\n" "v_add_f32 %[acc], %[acc], v122\n" "v_add_f32 %[acc], %[acc], v123\n"
        "v_add_f32 %[acc], %[acc], v124\n" "v_add_f32 %[acc], %[acc], v125\n" "v_add_f32 %[acc], %[acc], v126\n" "v_add_f32 %[acc], %[acc], v127\n"
        "s_mov_b32 %[st], %[sn]\n"
        "s_mov_b32 %[i], %[si1]\n"
        "s_cmp_lt_u32 %[i], %[nw]\n"
        "s_cbranch_scc1 6b\n"
        "s_branch 9f\n"
        "8:\n"
        "s_lshl_b32 %[sf], %[sn], 2\n"
        "v_add_u32 %[va], %[sf], %[rb]\n"
        "s_mov_b32 %[sp], 0x400000\n"
        "1:\n"
        "ds_read_b32 %[vf], %[va]\n"
        "s_waitcnt lgkmcnt(0)\n"
        "v_readfirstlane_b32 %[sf], %[vf]\n"
        "s_cmp_ge_i32 %[sf], %[si1]\n"
        "s_cbranch_scc1 4b\n"
        "s_sub_u32 %[sp], %[sp], 1\n"
        "s_cmp_eq_u32 %[sp], 0\n"
        "s_cbranch_scc0 1b\n"
        "s_mov_b32 %[ok], 0\n"
        "s_branch 4b\n"
        "9:\n"
        "s_waitcnt lgkmcnt(0)\n"
                : [acc] "+&v"(acc), [ok] "+&s"(oks), [i] "+&s"(i), [st] "+&s"(st), [so] "=&s"(so),
                  [sn] "=&s"(sn), [sf] "=&s"(sf), [si1] "=&s"(si1), [sp] "=&s"(sp), [va] "=&v"(va),
                  [vv] "=&v"(vv), [vf] "=&v"(vf)
                : [nw] "s"(nwhole), [np] "s"(npu), [l0] "v"(l0), [l1] "v"(l1), [l2] "v"(l2),
                  [l3] "v"(l3), [rb] "v"(rb), [vc] "v"(vc)
                : "v56", "v57", "v58", "v59", "v60", "v61", "v62", "v63",
                  "v64", "v65", "v66", "v67", "v68", "v69", "v70", "v71",
                  "v72", "v73", "v74", "v75", "v76", "v77", "v78", "v79",
                  "v80", "v81", "v82", "v83", "v84", "v85", "v86", "v87",
                  "v88", "v89", "v90", "v91", "v92", "v93", "v94", "v95",
                  "v96", "v97", "v98", "v99", "v100", "v101", "v102", "v103",
                  "v104", "v105", "v106", "v107", "v108", "v109", "v110", "v111",
                  "v112", "v113", "v114", "v115", "v116", "v117", "v118", "v119",
                  "v120", "v121", "v122", "v123", "v124", "v125", "v126", "v127",
                  "scc", "memory");
            ok = oks != 0;
        }
        // the last tile, partly filled: nfull whole quads, then rem positions
        if (ok && i < ntile) {
            ok = sv_wait_ge(&ready[st], i);
            if (ok) {
                const float4 *P = ring + st * SV_QT * 64;
                float4 X[SV_QT];
#pragma unroll
                for (int u = 0; u < SV_QT; u++) X[u] = P[u * 64 + (lane ^ ((u & 3) << 2))];
                const int nfull = nq - i * SV_QT;
#pragma unroll
                for (int u = 0; u < SV_QT; u++) {
                    const float4 v = X[u];
                    if (u < nfull) {
                        acc = acc + v.x; acc = acc + v.y; acc = acc + v.z; acc = acc + v.w;
                    } else if (u == nfull && rem) {
                        acc = acc + v.x;
                        if (rem > 1) acc = acc + v.y;
                        if (rem > 2) acc = acc + v.z;
                    }
                }
            }
            sv_signal(&consumed, i + 1);
        }
        if (!ok) {
            sv_signal(&consumed, 1 << 30);
            acc = __builtin_nanf("");
            if (lane == 0 && eok) sv_error(err, FOX_DEV_ERR_ATTN_VALUES);
        }
        if (g < G && d < hd) out[(size_t)t * out_stride + (size_t)(kvh * G + g) * hd + d] = acc;
        return;
    }
    if (!loader) return;

    // ---- loaders: product units u = li, li + SV_LOADERS, ...  A unit is G
    // quads of one tile for every lane (its G heads x DS columns); the
    // NLD units of a tile come from NLD different loaders, the last of them
    // marks the tile ready, so that the first tile is ready after one unit
    // of work per loader.
    if (!sv_wait_ge_idle(&a_ready, 1)) {
        if (lane == 0) sv_error(err, FOX_DEV_ERR_ATTN_LOADER);
        return;
    }
    // a_j = e_j * (1/sum), or e_j where the sum is not positive
    // (src/ops.c:35-38; e * 1 is e exactly): the scale per head, and that of
    // the lane's own head for the DPP exchange below
    float ivg[G];
#pragma unroll
    for (int gg = 0; gg < G; gg++) ivg[gg] = nrm_s[gg] ? inv_s[gg] : 1.0f;
    constexpr bool DPPX = G == 2 || G == 4;  // the G heads exchanged within lane quads
    const int mine = (lane - lq * DS) % G;
    float ivm = ivg[0];
#pragma unroll
    for (int gg = 1; gg < G; gg++) ivm = mine == gg ? ivg[gg] : ivm;
    // weight quads read per unit (one per head, or the lane's own head's
    // for the DPP exchange)
    constexpr int RK = DPPX ? 1 : G;
    int cons_seen = 0;                       // consumed is known to be at least this
    // the stage of the unit's tile, i mod np, kept as a running index (a
    // division per unit is scalar work every wave of the compute unit
    // shares one scalar unit for, the chain wave's included)
    int st_i = li / NLD, st = st_i % np;
    for (int u0 = li; u0 < nunit; u0 += SV_VPF * SV_LOADERS) {
#pragma unroll
        for (int m = 0; m < SV_VPF; m++) {
            const int u = u0 + m * SV_LOADERS;
            if (u >= nunit) break;
            const float4 v = vq[m];
            const int un = u + SV_VPF * SV_LOADERS;
            if (un < nunit) vq[m] = v_of(un);
            const int i = u / NLD, k = u - i * NLD;
            const int qi = k * G + lq;                       // the lane's quad in the tile
            const int jq = min(i * SV_QT + qi, nq_all - 1);
            float4 wq[RK];
#pragma unroll
            for (int r = 0; r < RK; r++) wq[r] = ((const float4 *)(e + (DPPX ? mine : r) * estr))[jq];
            // the tile's stage is free once tile i - np is consumed
            if (i >= np && cons_seen < i - np + 1) {
                if (!sv_wait_ge_idle(&consumed, i - np + 1)) {
                    if (lane == 0) sv_error(err, FOX_DEV_ERR_ATTN_LOADER);
                    return;
                }
                cons_seen = i - np + 1;
            }
            for (st += i - st_i, st_i = i; st >= np;) st -= np;
            float4 *P = ring + st * SV_QT * 64;
            float4 am = wq[0];
            if (DPPX) {
                am.x = am.x * ivm; am.y = am.y * ivm; am.z = am.z * ivm; am.w = am.w * ivm;
            }
#pragma unroll
            for (int gg = 0; gg < G; gg++) {
                float4 a;
                if (DPPX) {
                    // quad_perm: every lane of a quad takes lane (quad base + gg)
                    const int ctl = G == 4 ? gg * 0x55 : (gg ? 0xF5 : 0xA0);
                    a.x = dpp_bcast(am.x, ctl);
                    a.y = dpp_bcast(am.y, ctl);
                    a.z = dpp_bcast(am.z, ctl);
                    a.w = dpp_bcast(am.w, ctl);
                } else {
                    a = wq[DPPX ? 0 : gg];
                    a.x = a.x * ivg[gg]; a.y = a.y * ivg[gg];
                    a.z = a.z * ivg[gg]; a.w = a.w * ivg[gg];
                }
                float4 p;
                p.x = a.x * v.x; p.y = a.y * v.y; p.z = a.z * v.z; p.w = a.w * v.w;
                P[qi * 64 + ((gg * DS + (lane - lq * DS)) ^ ((qi & 3) << 2))] = p;
            }
            // count the unit; the tile's last unit marks it ready (its
            // writes, and through their own counts every other unit's, are
            // complete by then)
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            int old = 0;
            if (lane == 0) old = __hip_atomic_fetch_add(&cnt[st], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            old = __builtin_amdgcn_readfirstlane(old);
            if (old == NLD - 1) {
                if (lane == 0) cnt[st] = 0;          // (no unit of the stage's next tile runs before
                sv_signal(&ready[st], i);            //  this tile is consumed)
            }
        }
    }
}

extern "C" fox_gpu_status fox_gpu_attention(fox_gpu_ctx *ctx, float *out, size_t out_stride,
                                            const float *q, size_t q_stride, const float *k_cache,
                                            const float *v_cache, size_t n_head, size_t n_head_kv,
                                            size_t head_dim, size_t M, const uint32_t *pos,
                                            size_t n_ctx, int mode)
{
    if (!ctx || !out || !q || !k_cache || !v_cache || !pos || n_head == 0 || n_head_kv == 0 ||
        head_dim == 0 || M == 0 || n_ctx == 0)
        return fox_fail(FOX_GPU_ERR_ARG, "attention: bad argument");
    if (n_head % n_head_kv)
        return fox_fail(FOX_GPU_ERR_ARG, "attention: %zu heads over %zu kv heads", n_head,
                        n_head_kv);
    if (n_head / n_head_kv > ATT_MAXG || head_dim > ATT_MAXHD || head_dim % 4)
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED,
                        "attention: at most %d query heads per kv head, head_dim a multiple of "
                        "4 up to %d", ATT_MAXG, ATT_MAXHD);
    if (M > FOX_GPU_MAX_TOKENS) return fox_fail(FOX_GPU_ERR_ARG, "attention: too many tokens");
    if (n_ctx > (1u << 30)) return fox_fail(FOX_GPU_ERR_ARG, "attention: n_ctx too large");
    const size_t qs = M > 1 ? q_stride : n_head * head_dim;
    const size_t os = M > 1 ? out_stride : n_head * head_dim;
    if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 || qs % 4)
        return fox_fail(FOX_GPU_ERR_ARG, "attention: q and the caches must be 16-byte aligned "
                        "and the q stride a multiple of 4");
    if (mode == FOX_GPU_ATTN_EXACT) {
        if (n_ctx * sizeof(float) > 60 * 1024)
            return fox_fail(FOX_GPU_ERR_UNSUPPORTED,
                            "attention: exact mode keeps a head's %zu weights in LDS; at most "
                            "15360 positions", n_ctx);
        const size_t att_stride = (n_ctx + 3) & ~(size_t)3;
        const int n_tiles = (int)((n_ctx + SC_TILE - 1) / SC_TILE);
        const size_t att_bytes = M * n_head * att_stride * sizeof(float);
        const size_t bytes = att_bytes + M * n_head * (size_t)n_tiles * sizeof(float);
        fox_gpu_status st = fox_ws_reserve(ctx, bytes);
        if (st) return st;
        float *att = (float *)ctx->ws;
        float *tmax = (float *)(ctx->ws + att_bytes);
        const size_t gqa = n_head / n_head_kv;
        const int nch = (int)((head_dim / 4 + SC_CQ - 1) / SC_CQ);
        const size_t lds = 0;                                   // (static arrays)
        const void *sk = nch == 1 ? (const void *)attn_scores_x<1>
                       : nch == 2 ? (const void *)attn_scores_x<2>
                       : nch == 3 ? (const void *)attn_scores_x<3>
                       : nch == 4 ? (const void *)attn_scores_x<4>
                       : nch == 5 ? (const void *)attn_scores_x<5>
                       : nch == 6 ? (const void *)attn_scores_x<6>
                       : nch == 7 ? (const void *)attn_scores_x<7>
                                  : (const void *)attn_scores_x<8>;
        if (lds > 64 * 1024) {
            hipError_t e = hipFuncSetAttribute(sk, hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)lds);
            if (e != hipSuccess) return fox_hip_fail(e, "attention: LDS size");
        }
        {
            const int ih = (int)n_head, ikv = (int)n_head_kv, ihd = (int)head_dim;
            const int ictx = (int)n_ctx, iM = (int)M;
            const int tpw = SC_TPW;
            void *args[] = {(void *)&q, (void *)&qs, (void *)&k_cache, (void *)&ih, (void *)&ikv,
                            (void *)&ihd, (void *)&pos, (void *)&ictx, (void *)&att_stride,
                            (void *)&att, (void *)&tmax, (void *)&n_tiles, (void *)&iM,
                            (void *)&tpw};
            hipError_t e = hipLaunchKernel(sk, dim3((unsigned)n_tiles, (unsigned)n_head_kv,
                                                    (unsigned)((M + tpw - 1) / tpw)),
                                           dim3(256), args, lds, ctx->stream);
            if (e != hipSuccess) return fox_hip_fail(e, "attention scores");
        }
        FOX_LAUNCHED("attention scores");
        const int ds = (int)(64 / gqa);
        const int n_sl = (int)((head_dim + ds - 1) / ds);
        const size_t e_bytes = gqa * (att_stride + 4) * sizeof(float);
        const int ih = (int)n_head, ikv = (int)n_head_kv, ihd = (int)head_dim, ictx = (int)n_ctx;
        const void *sv = gqa == 1 ? (const void *)attn_sv_x<1>
                       : gqa == 2 ? (const void *)attn_sv_x<2>
                       : gqa == 4 ? (const void *)attn_sv_x<4>
                       : gqa == 8 ? (const void *)attn_sv_x<8> : nullptr;
        // product stages: as many as fit beside the weights (at least SV_NP_MIN)
        const size_t np_fit = e_bytes < SV_LDS_MAX ? (SV_LDS_MAX - e_bytes) / SV_STAGE : 0;
        const int np = (int)(np_fit < SV_NP_MAX ? np_fit : SV_NP_MAX);
        if (sv && np >= SV_NP_MIN) {
            const size_t sv_lds = (size_t)np * SV_STAGE + e_bytes;
            hipError_t e = hipFuncSetAttribute(sv, hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)sv_lds);
            if (e != hipSuccess) return fox_hip_fail(e, "attention: LDS size");
            const int sv_ds = (int)(64 / gqa);
            const unsigned nsl = (unsigned)((head_dim + sv_ds - 1) / sv_ds);
            const int n_attn = (int)(n_head_kv * nsl);
            unsigned *err = (unsigned *)(ctx->small + FOX_SMALL_ERR_OFF);
            void *args[] = {(void *)&att, (void *)&att_stride, (void *)&tmax, (void *)&n_tiles,
                            (void *)&v_cache, (void *)&ih, (void *)&ikv, (void *)&ihd,
                            (void *)&pos, (void *)&ictx, (void *)&out, (void *)&os,
                            (void *)&np, (void *)&err};
            e = hipLaunchKernel(sv, dim3((unsigned)n_attn, (unsigned)M),
                                dim3(SV_WAVES * 64), args, sv_lds, ctx->stream);
            if (e != hipSuccess) return fox_hip_fail(e, "attention softmax+values");
            FOX_LAUNCHED("attention softmax+values");
            return FOX_GPU_OK;
        }
        hipLaunchKernelGGL(attn_softmax_x, dim3((unsigned)n_head, (unsigned)M), dim3(256),
                           att_stride * sizeof(float), ctx->stream, att, att_stride, tmax,
                           n_tiles, (int)n_head, pos, (int)n_ctx);
        FOX_LAUNCHED("attention softmax");
        hipLaunchKernelGGL(attn_values_x, dim3((unsigned)(n_head_kv * n_sl), (unsigned)M),
                           dim3(64), 0, ctx->stream, att, att_stride, v_cache, (int)n_head,
                           (int)n_head_kv, (int)head_dim, ds, pos, (int)n_ctx, out, os);
        FOX_LAUNCHED("attention values");
        return FOX_GPU_OK;
    }
    if (mode != FOX_GPU_ATTN_SPLIT) return fox_fail(FOX_GPU_ERR_ARG, "attention: unknown mode %d", mode);
    const int n_splits = (int)((n_ctx + ATT_SPLIT - 1) / ATT_SPLIT);
    const size_t bytes = M * n_head * (size_t)n_splits * (2 + head_dim) * sizeof(float);
    fox_gpu_status st = fox_ws_reserve(ctx, bytes);
    if (st) return st;
    float *part = (float *)ctx->ws;
    hipLaunchKernelGGL(attn_partial, dim3((unsigned)n_splits, (unsigned)n_head_kv, (unsigned)M),
                       dim3(256), 0, ctx->stream, q, qs, k_cache, v_cache, (int)n_head,
                       (int)n_head_kv, (int)head_dim, pos, (int)n_ctx, n_splits, part);
    FOX_LAUNCHED("attention partial");
    hipLaunchKernelGGL(attn_merge, dim3((unsigned)n_head, (unsigned)M), dim3(128), 0, ctx->stream,
                       part, (int)n_head, (int)head_dim, n_splits, out, os);
    FOX_LAUNCHED("attention merge");
    return FOX_GPU_OK;
}

// ------------------------------------------------------- swiglu, add

__global__ void silu_mul_k(float *__restrict__ g, const float *__restrict__ u, int n,
                           size_t stride)
{
    const int t = blockIdx.y;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        float x = g[(size_t)t * stride + i];
        g[(size_t)t * stride + i] = fox_div(x, 1.0f + fox_expf(-x)) * u[(size_t)t * stride + i];
    }
}

__global__ void add_k(float *__restrict__ d, const float *__restrict__ s, int n, size_t stride)
{
    const int t = blockIdx.y;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        d[(size_t)t * stride + i] = d[(size_t)t * stride + i] + s[(size_t)t * stride + i];
}

static unsigned ew_grid(size_t n)
{
    size_t g = (n + 255) / 256;
    return (unsigned)(g > 1024 ? 1024 : g);
}

extern "C" fox_gpu_status fox_gpu_silu_mul(fox_gpu_ctx *ctx, float *gate, const float *up,
                                           size_t n, size_t M, size_t stride)
{
    if (!ctx || !gate || !up || n == 0 || M == 0 || M > 65535)
        return fox_fail(FOX_GPU_ERR_ARG, "silu_mul: bad argument");
    hipLaunchKernelGGL(silu_mul_k, dim3(ew_grid(n), (unsigned)M), dim3(256), 0, ctx->stream,
                       gate, up, (int)n, M > 1 ? stride : n);
    FOX_LAUNCHED("silu_mul");
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_add(fox_gpu_ctx *ctx, float *dst, const float *src, size_t n,
                                      size_t M, size_t stride)
{
    if (!ctx || !dst || !src || n == 0 || M == 0 || M > 65535)
        return fox_fail(FOX_GPU_ERR_ARG, "add: bad argument");
    hipLaunchKernelGGL(add_k, dim3(ew_grid(n), (unsigned)M), dim3(256), 0, ctx->stream, dst, src,
                       (int)n, M > 1 ? stride : n);
    FOX_LAUNCHED("add");
    return FOX_GPU_OK;
}

// ----------------------------------------------------------------- argmax

// First index of the maximum, NaN never winning (src/sample.c:147-153:
// best starts at 0 and moves only on a strict '>'; a NaN at index 0 stays).
// Two launches: argmax_part_k reduces contiguous ranges to (max, first
// index) partials, one per workgroup; argmax_merge_k, one workgroup, merges
// them in index order, applies the index-0 rule and writes the result and,
// for a decode loop, the history entry and the advanced position.  The
// partials cross a kernel boundary, as every other producer/consumer pair of
// the decode does: a single launch whose last workgroup merged the others'
// partials (a device-scope arrival counter, agent-scope relaxed stores and
// loads) read a partial of the previous launch now and then, on a graph
// replay, and picked the runner-up workgroup's maximum.
#define AM_THREADS 256
#define AM_MAX_WG 256
#define AM_UNROLL 8

__device__ __forceinline__ void am_merge(float &best, int &bidx, float ov, int oi)
{
    if (ov > best || (ov == best && oi < bidx)) {
        best = ov;
        bidx = oi;
    }
}

// (best, bidx) of the workgroup into thread 0's registers (NaN never taken)
__device__ __forceinline__ void am_reduce_wg(float &best, int &bidx, float *bv, int *bi)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_index();
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) am_merge(best, bidx, __shfl_xor(best, o), __shfl_xor(bidx, o));
    if (lane == 0) {
        bv[wave] = best;
        bi[wave] = bidx;
    }
    __syncthreads();
    if (tid == 0)
        for (int w = 1; w < AM_THREADS / 64; w++) am_merge(best, bidx, bv[w], bi[w]);
}

__global__ __launch_bounds__(AM_THREADS) void argmax_part_k(const float *__restrict__ x, int n,
                                                            int per, float *__restrict__ pv,
                                                            int *__restrict__ pi)
{
    __shared__ float bv[AM_THREADS / 64];
    __shared__ int bi[AM_THREADS / 64];
    const int tid = threadIdx.x;
    const int i0 = blockIdx.x * per, i1 = min(n, i0 + per);
    float best = -INFINITY;
    int bidx = 0x7fffffff;
    // a thread's values in index order, AM_UNROLL loads issued before the
    // first comparison
    for (int b0 = i0; b0 < i1; b0 += AM_THREADS * AM_UNROLL) {
        float v[AM_UNROLL];
#pragma unroll
        for (int k = 0; k < AM_UNROLL; k++) {
            const int i = b0 + tid + k * AM_THREADS;
            v[k] = x[i < i1 ? i : i1 - 1];
        }
#pragma unroll
        for (int k = 0; k < AM_UNROLL; k++) {
            const int i = b0 + tid + k * AM_THREADS;
            if (i < i1 && v[k] > best) {
                best = v[k];
                bidx = i;
            }
        }
    }
    am_reduce_wg(best, bidx, bv, bi);
    if (tid == 0) {
        pv[blockIdx.x] = best;
        pi[blockIdx.x] = bidx;
    }
}

__global__ __launch_bounds__(AM_THREADS) void argmax_merge_k(const float *__restrict__ x,
                                                             const float *__restrict__ pv,
                                                             const int *__restrict__ pi, int nwg,
                                                             uint32_t *__restrict__ idx,
                                                             uint32_t *__restrict__ pos,
                                                             uint32_t advance,
                                                             uint32_t *__restrict__ history)
{
    __shared__ float bv[AM_THREADS / 64];
    __shared__ int bi[AM_THREADS / 64];
    const int tid = threadIdx.x;
    float best = -INFINITY;
    int bidx = 0x7fffffff;
    for (int b = tid; b < nwg; b += AM_THREADS) am_merge(best, bidx, pv[b], pi[b]);
    am_reduce_wg(best, bidx, bv, bi);
    if (tid == 0) {
        // index 0 wins unless something is strictly greater than x[0]
        const float x0 = x[0];
        const uint32_t r = (x0 != x0 || !(best > x0)) ? 0u : (uint32_t)bidx;
        *idx = r;
        if (pos) {
            const uint32_t p = *pos;
            if (history) history[p] = r;
            *pos = p + advance;
        }
    }
}

extern "C" fox_gpu_status fox_gpu_argmax(fox_gpu_ctx *ctx, const float *logits, size_t n,
                                         uint32_t *idx, uint32_t *pos, uint32_t advance,
                                         uint32_t *history)
{
    if (!ctx || !logits || !idx || n == 0 || n > 0x7fffffff)
        return fox_fail(FOX_GPU_ERR_ARG, "argmax: bad argument");
    // the partials live in the context's fixed small buffer
    float *pv = (float *)(ctx->small + FOX_SMALL_AM_OFF);
    int *pi = (int *)(ctx->small + FOX_SMALL_AM_OFF + 4 * AM_MAX_WG);
    size_t nwg = (n + 2047) / 2048;
    if (nwg > AM_MAX_WG) nwg = AM_MAX_WG;
    const size_t per = (n + nwg - 1) / nwg;
    nwg = (n + per - 1) / per;
    hipLaunchKernelGGL(argmax_part_k, dim3((unsigned)nwg), dim3(AM_THREADS), 0, ctx->stream,
                       logits, (int)n, (int)per, pv, pi);
    FOX_LAUNCHED("argmax partials");
    hipLaunchKernelGGL(argmax_merge_k, dim3(1), dim3(AM_THREADS), 0, ctx->stream, logits,
                       (const float *)pv, (const int *)pi, (int)nwg, idx, pos, advance, history);
    FOX_LAUNCHED("argmax merge");
    return FOX_GPU_OK;
}
