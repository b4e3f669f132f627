// fox_ops.hip -- bandwidth-bound decode ops: row gather, RMSNorm, RoPE + KV
// store, split-position GQA attention, SwiGLU, residual add, argmax.
// Built with -ffp-contract=off like the rest of the library: every float op
// rounds once, in the reference's order where the reference fixes an order.
#include "fox_gemv_dev.h"
#include "fox_internal.h"
#include "fox_math.h"
#include "fox_sum.h"

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
#define ATT_MAXG 8     // query heads per kv head handled by one workgroup
#define ATT_MAXHD 256

__device__ __forceinline__ float wave_sum_f(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// ---- split mode (flash decoding): positions in splits of FD_SPLIT, each
// split's softmax and value sum local to a workgroup, then a merge.  Sums run
// in any order (float reassociation): results differ from the reference's in
// their last bits.
//   attn_fd128 (head_dim 128) and attn_fd (other head dims; described here)
//   attn_fd   a workgroup per (split, kv head, token): the split's K rows, V
//             quads and the G query heads in LDS (every thread's loads issued
//             in one round before the first use; a wave's load is eight
//             128-byte row pieces), scores as dot products with four partial
//             sums, a wave per head for the split's maximum m, e = exp(s - m)
//             and their sum l, then o = sum of e v per (head, column); writes
//             the record (m, l, -, -, o) per (token, head, split);
//   attn_fdm  a workgroup per (head, token), over the splits that hold the
//             token's positions: eight split groups, each thread loading its
//             group's (m, l, column quad of o) for eight splits in one round
//             and keeping a running maximum and rescaled sums; then the
//             groups' sums weighted by exp(m_g - M), divided by their l sum.
#define FD_SPLIT 32
#define FD_MAXS 1024        // splits the merge holds (32768 positions, 65536 at head_dim 128)
#define FD_LOADS 9          // 16-byte loads per thread: one round for G <= 8, head_dim <= 128

template <int G>
__global__ __launch_bounds__(256) void attn_fd(const float *__restrict__ q, size_t q_stride,
                                               const float *__restrict__ kc,
                                               const float *__restrict__ vc, int n_head_kv,
                                               int hd, const uint32_t *__restrict__ pos,
                                               int n_ctx, int n_splits, float *__restrict__ part)
{
    extern __shared__ float4 fd_lds[];
    const int hd4 = hd >> 2, ks = hd4 + 1;
    float4 *Ks = fd_lds;                           // [FD_SPLIT][ks]
    float4 *Qs = Ks + FD_SPLIT * ks;               // [G][hd4]
    float4 *Vs = Qs + G * hd4;                     // [FD_SPLIT / 4 quad rows][hd]
    float *Ps = (float *)(Vs + (FD_SPLIT / 4) * hd);   // [G][FD_SPLIT]
    __shared__ float st_m[G], st_l[G];
    const int s = blockIdx.x, kvh = blockIdx.y, t = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_index();
    const int n_head = n_head_kv * G, kvd = n_head_kv * hd;
    const int upto = (int)min((size_t)pos[0] + (size_t)t + 1, (size_t)n_ctx);
    const int p0 = s * FD_SPLIT, pn = min(FD_SPLIT, upto - p0);
    if (pn <= 0) return;                           // (uniform) past the token's end: the merge
                                                   // reads only the splits below it
    const size_t rec = 4 + (size_t)hd;
    float *base = part + (((size_t)t * n_head + (size_t)kvh * G) * n_splits + s) * rec;
    // queries, K rows and V quads, all requested before the first is stored;
    // a K "chunk" is eight quads of every row, a V chunk eight columns of
    // every quad row (rows past pn re-read row pn - 1; quads past hd4 re-read
    // the last one and are not stored)
    const float4 *qb = (const float4 *)(q + (size_t)t * q_stride + (size_t)kvh * G * hd);
    const float4 *kb = (const float4 *)(kc + (size_t)p0 * kvd + (size_t)kvh * hd);
    const float4 *vb = (const float4 *)vc + (size_t)(p0 >> 2) * kvd + (size_t)kvh * hd;
    const int nkq = FD_SPLIT * ((hd4 + 7) & ~7), nvq = (FD_SPLIT / 4) * ((hd + 7) & ~7);
    const int rows_q = (pn + 3) >> 2;
    // (native 4-vectors: an array of float4 structs stays in scratch memory)
    typedef float f4v __attribute__((ext_vector_type(4)));
    for (int f0 = 0; f0 < nkq + nvq + G * hd4; f0 += FD_LOADS * 256) {
        f4v r[FD_LOADS];
#pragma unroll
        for (int k = 0; k < FD_LOADS; k++) {
            const int f = f0 + k * 256 + tid;
            if (f < nkq) {
                const int row = (f >> 3) & (FD_SPLIT - 1), qd = 8 * (f / (8 * FD_SPLIT)) + (f & 7);
                r[k] = ((const f4v *)kb)[(size_t)min(row, pn - 1) * (kvd / 4) + min(qd, hd4 - 1)];
            } else if (f < nkq + nvq) {
                const int g = f - nkq, row = (g >> 3) & (FD_SPLIT / 4 - 1);
                const int col = 8 * (g / (2 * FD_SPLIT)) + (g & 7);
                r[k] = ((const f4v *)vb)[(size_t)min(row, rows_q - 1) * kvd + min(col, hd - 1)];
            } else {
                r[k] = ((const f4v *)qb)[min(f - nkq - nvq, G * hd4 - 1)];
            }
        }
#pragma unroll
        for (int k = 0; k < FD_LOADS; k++) {
            const int f = f0 + k * 256 + tid;
            if (f < nkq) {
                const int row = (f >> 3) & (FD_SPLIT - 1), qd = 8 * (f / (8 * FD_SPLIT)) + (f & 7);
                if (qd < hd4) ((f4v *)Ks)[row * ks + qd] = r[k];
            } else if (f < nkq + nvq) {
                const int g = f - nkq, row = (g >> 3) & (FD_SPLIT / 4 - 1);
                const int col = 8 * (g / (2 * FD_SPLIT)) + (g & 7);
                if (col < hd) ((f4v *)Vs)[row * hd + col] = r[k];
            } else if (f < nkq + nvq + G * hd4) {
                ((f4v *)Qs)[f - nkq - nvq] = r[k];
            }
        }
    }
    __syncthreads();
    // scores: item (head i / FD_SPLIT, position i % FD_SPLIT)
    const float scale = fox_div(1.0f, fox_sqrtf((float)hd));
    for (int i = tid; i < G * FD_SPLIT; i += 256) {
        const int g = i / FD_SPLIT, pl = i % FD_SPLIT;
        const float4 *kr = Ks + pl * ks, *qr = Qs + g * hd4;
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
        for (int d = 0; d < hd4; d++) {
            const float4 kv = kr[d], qv = qr[d];
            a0 += qv.x * kv.x;
            a1 += qv.y * kv.y;
            a2 += qv.z * kv.z;
            a3 += qv.w * kv.w;
        }
        Ps[i] = pl < pn ? ((a0 + a1) + (a2 + a3)) * scale : -INFINITY;
    }
    __syncthreads();
    // the split's softmax per head: wave w takes heads w, w + 4
    for (int g = wave; g < G; g += 4) {
        const float v = lane < FD_SPLIT ? Ps[g * FD_SPLIT + lane] : -INFINITY;
        const float m = wave_reduce(v, -INFINITY, [](float x, float y) { return y > x ? y : x; });
        const float e = lane < pn ? __expf(v - m) : 0.0f;
        if (lane < FD_SPLIT) Ps[g * FD_SPLIT + lane] = e;
        const float l = wave_reduce(e, 0.0f, [](float x, float y) { return x + y; });
        if (lane == 0) {
            st_m[g] = m;
            st_l[g] = l;
        }
    }
    __syncthreads();
    // o = sum of e v, item (head i / hd, column i % hd)
    for (int i = tid; i < G * hd; i += 256) {
        const int g = i / hd, c = i % hd;
        const float4 *pe = (const float4 *)(Ps + g * FD_SPLIT);
        float o = 0.0f;
        for (int rq = 0; rq < (pn >> 2); rq++) {
            const float4 v = Vs[rq * hd + c], e = pe[rq];
            o += ((e.x * v.x + e.y * v.y) + (e.z * v.z + e.w * v.w));
        }
        // the ragged last quad: only positions below pn (the cache rows past
        // the token's end may hold anything, and 0 * inf is NaN)
        if (pn & 3) {
            const float4 v = Vs[(pn >> 2) * hd + c], e = pe[pn >> 2];
            o += e.x * v.x;
            if ((pn & 3) > 1) o += e.y * v.y;
            if ((pn & 3) > 2) o += e.z * v.z;
        }
        float *r = base + (size_t)g * n_splits * rec;
        if (c == 0) {
            r[0] = st_m[g];
            r[1] = st_l[g];
        }
        r[4 + c] = o;
    }
}

// attn_fd for head_dim 128 in splits of FD_SPLIT_W positions, 512 threads,
// K and V straight into registers: thread (position tid / 8, part tid % 8)
// holds quads 4 part .. 4 part + 3 of its K row and forms the partial dots of
// all G heads (fused multiply-adds), summed over the 8 parts by DPP; thread
// (column tid / 4, quarter tid % 4) holds its column's 16 positions of V
// (four quads), whose products with every head's weights are summed over
// the quarters by DPP.  Only the queries, the scores and the weights pass
// through LDS; a wave per head takes the split's softmax.
#define FD_SPLIT_W 64
template <int G>
__global__ __launch_bounds__(512) void attn_fd128(const float *__restrict__ q, size_t q_stride,
                                                  const float *__restrict__ kc,
                                                  const float *__restrict__ vc, int n_head_kv,
                                                  const uint32_t *__restrict__ pos, int n_ctx,
                                                  int n_splits, float *__restrict__ part)
{
    constexpr int HD = 128, HD4 = 32, SP = FD_SPLIT_W;
    static_assert(SP == 64 && G <= 8, "a position per 8 threads, a wave per head");
    typedef float f4v __attribute__((ext_vector_type(4)));
    __shared__ f4v Qs[G * HD4];
    __shared__ __attribute__((aligned(16))) float Ps[G][SP];   // (read as 4-vectors)
    __shared__ float st_m[G], st_l[G];
    const int s = blockIdx.x, kvh = blockIdx.y, t = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_index();
    const int n_head = n_head_kv * G, kvd = n_head_kv * HD;
    const int upto = (int)min((size_t)pos[0] + (size_t)t + 1, (size_t)n_ctx);
    const int p0 = s * SP, pn = min(SP, upto - p0);
    if (pn <= 0) return;                           // (uniform) past the token's end
    // loads: K row piece, V column quads, then (G * 32 threads) a query quad
    // (rows past pn re-read row pn - 1, quad rows past the last re-read it)
    const int pk = tid >> 3, dp = tid & 7;
    const f4v *kr = (const f4v *)(kc + (size_t)(p0 + min(pk, pn - 1)) * kvd + (size_t)kvh * HD) +
                    4 * dp;
    const int c = tid >> 2, hq = tid & 3, rows_q = (pn + 3) >> 2;
    const f4v *vr = (const f4v *)vc + (size_t)(p0 >> 2) * kvd + (size_t)kvh * HD + c;
    f4v kq[4], vq[4];
#pragma unroll
    for (int k = 0; k < 4; k++) kq[k] = kr[k];
#pragma unroll
    for (int k = 0; k < 4; k++) vq[k] = vr[(size_t)min(4 * hq + k, rows_q - 1) * kvd];
    if (tid < G * HD4)
        Qs[tid] = ((const f4v *)(q + (size_t)t * q_stride + (size_t)kvh * G * HD))[tid];
    __syncthreads();
    // scores: the G partial dots of this part, then the sums over the parts
    float sc[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const f4v qq = Qs[g * HD4 + 4 * dp + k];
            a0 = __builtin_fmaf(qq.x, kq[k].x, a0);
            a1 = __builtin_fmaf(qq.y, kq[k].y, a1);
            a2 = __builtin_fmaf(qq.z, kq[k].z, a2);
            a3 = __builtin_fmaf(qq.w, kq[k].w, a3);
        }
        sc[g] = (a0 + a1) + (a2 + a3);
    }
#pragma unroll
    for (int g = 0; g < G; g++) sc[g] += dpp_t<0xB1, 0xF>(0.0f, sc[g]);
#pragma unroll
    for (int g = 0; g < G; g++) sc[g] += dpp_t<0x4E, 0xF>(0.0f, sc[g]);
#pragma unroll
    for (int g = 0; g < G; g++) sc[g] += dpp_t<0x141, 0xF>(0.0f, sc[g]);
    const float scale = fox_div(1.0f, fox_sqrtf((float)HD));
#pragma unroll
    for (int g = 0; g < G; g++)
        if (dp == g) Ps[g][pk] = pk < pn ? sc[g] * scale : -INFINITY;
    __syncthreads();
    // the split's softmax: wave g takes head g
    if (wave < G) {
        const float v = Ps[wave][lane];
        const float m = wave_reduce(v, -INFINITY, [](float x, float y) { return y > x ? y : x; });
        const float e = lane < pn ? __expf(v - m) : 0.0f;
        Ps[wave][lane] = e;
        const float l = wave_reduce(e, 0.0f, [](float x, float y) { return x + y; });
        if (lane == 0) {
            st_m[wave] = m;
            st_l[wave] = l;
        }
    }
    __syncthreads();
    // values: the V components past pn are zeroed (cache rows past the
    // token's end may hold anything, and 0 * inf is NaN)
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int pb = 16 * hq + 4 * k;
        vq[k].x = pb < pn ? vq[k].x : 0.0f;
        vq[k].y = pb + 1 < pn ? vq[k].y : 0.0f;
        vq[k].z = pb + 2 < pn ? vq[k].z : 0.0f;
        vq[k].w = pb + 3 < pn ? vq[k].w : 0.0f;
    }
    float o[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const f4v *pe = (const f4v *)&Ps[g][16 * hq];
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const f4v e = pe[k];
            a0 = __builtin_fmaf(e.x, vq[k].x, a0);
            a1 = __builtin_fmaf(e.y, vq[k].y, a1);
            a0 = __builtin_fmaf(e.z, vq[k].z, a0);
            a1 = __builtin_fmaf(e.w, vq[k].w, a1);
        }
        o[g] = a0 + a1;
    }
#pragma unroll
    for (int g = 0; g < G; g++) o[g] += dpp_t<0xB1, 0xF>(0.0f, o[g]);
#pragma unroll
    for (int g = 0; g < G; g++) o[g] += dpp_t<0x4E, 0xF>(0.0f, o[g]);
    const size_t rec = 4 + (size_t)HD;
    float *base = part + (((size_t)t * n_head + (size_t)kvh * G) * n_splits + s) * rec;
#pragma unroll
    for (int g = 0; g < G; g++) {
        float *r = base + (size_t)g * n_splits * rec;
        if (hq == 0) r[4 + c] = o[g];
        if (tid == 0) {
            r[0] = st_m[g];
            r[1] = st_l[g];
        }
    }
}

__global__ __launch_bounds__(256) void attn_fdm(const float *__restrict__ part,
                                                const uint32_t *__restrict__ pos, int n_ctx,
                                                int n_head, int hd, int split, int n_splits,
                                                float *__restrict__ out, size_t out_stride)
{
    typedef float f4v __attribute__((ext_vector_type(4)));
    constexpr int R = 8;                       // splits a thread loads in one round
    __shared__ float gm[8], gl[8];
    __shared__ f4v go[8][32];
    const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    const int upto = (int)min((size_t)pos[0] + (size_t)t + 1, (size_t)n_ctx);
    const int nu = (upto + split - 1) / split;     // the splits attn_fd wrote
    const size_t rec = 4 + (size_t)hd;
    const float *base = part + (((size_t)t * n_head + h) * n_splits) * rec;
    // split group sg takes splits sg, sg + 8, ... (a running maximum, the
    // sums rescaled when it grows), column quad c0 + cq
    const int sg = tid >> 5, cq = tid & 31, hd4 = hd >> 2;
    for (int c0 = 0; c0 < hd4; c0 += 32) {
        const int c4 = min(c0 + cq, hd4 - 1);          // (past the end: re-read, not stored)
        float m = -INFINITY, l = 0.0f;
        f4v o = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int s0 = sg; s0 < nu; s0 += 8 * R) {
            float ms[R], ls[R];
            f4v os[R];
#pragma unroll
            for (int k = 0; k < R; k++) {
                const float *r = base + (size_t)min(s0 + 8 * k, nu - 1) * rec;
                ms[k] = r[0];
                ls[k] = r[1];
                os[k] = *(const f4v *)(r + 4 + 4 * c4);
            }
            float mn = m;
#pragma unroll
            for (int k = 0; k < R; k++)
                if (s0 + 8 * k < nu) mn = fmaxf(mn, ms[k]);
            const float sc = m > -INFINITY ? __expf(m - mn) : 0.0f;
            l *= sc;
            o *= sc;
#pragma unroll
            for (int k = 0; k < R; k++) {
                const float w = s0 + 8 * k < nu && ms[k] > -INFINITY ? __expf(ms[k] - mn) : 0.0f;
                l += w * ls[k];
                o += w * os[k];
            }
            m = mn;
        }
        if (cq == 0) {
            gm[sg] = m;
            gl[sg] = l;
        }
        go[sg][cq] = o;
        __syncthreads();
        if (tid < 32 && c0 + cq < hd4) {
            float M = gm[0];
#pragma unroll
            for (int g = 1; g < 8; g++) M = fmaxf(M, gm[g]);
            float L = 0.0f;
            f4v O = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int g = 0; g < 8; g++) {
                const float w = gm[g] > -INFINITY ? __expf(gm[g] - M) : 0.0f;
                L += w * gl[g];
                O += w * go[g][cq];
            }
            float *dst = out + (size_t)t * out_stride + (size_t)h * hd + 4 * (c0 + cq);
            dst[0] = O.x / L;
            dst[1] = O.y / L;
            dst[2] = O.z / L;
            dst[3] = O.w / L;
        }
        __syncthreads();
    }
}

// ---- attention in the reference's order (src/forward.c:222-257,
// src/ops.c:24-39), bit for bit:
//   score_j = (sum_d q_d k_jd, summed in d order) * (1 / sqrtf(hd));
//   softmax: max (a NaN first score stays the maximum, other NaNs are
//     skipped), e_j = expf(score_j - max), sum in j order, a_j = e_j * (1/sum)
//     when the sum is positive;
//   out_d = sum in j order of a_j v_jd (each product rounded, then added).
// Each in-order sum is one lane's dependent chain.  Every hand-over inside a
// kernel is at a workgroup barrier; between kernels, at the launch boundary.
//   attn_qk   scores and per-64-position-tile maxima: a workgroup per (tile,
//             kv head, up to QK_TPW tokens), the K tile and the queries in
//             LDS, a lane per (query head, position);
//   attn_hv   one token: a workgroup per (query head, HV_CH columns): the
//             head's maximum, then e_j in blocks while one lane runs the
//             softmax sum over the block before, then a_j, then the products
//             a_j v_jd in blocks (V streamed from HBM a few blocks ahead)
//             while the chain wave adds the block before;
//   attn_sm + attn_avm   several tokens, or a context longer than attn_hv's
//             LDS holds: the softmax per (head, token), a_j written over the
//             scores, then the value chains of MT tokens per workgroup fed by
//             the same block pipeline as attn_hv.

#define SC_TILE 64
#define QK_TPW 4            // tokens per scores workgroup (the K tile is read once for them)
#define ATT_LDS_MAX (159 * 1024)
#define ATT_EXACT_MAX_CTX 32768     // attn_sm holds a head's weights in LDS

// A workgroup of 256 threads per (64-position tile, kv head, QK_TPW tokens):
// the tile's K rows (plain loads, row stride padded by one quad against bank
// conflicts) and the G query heads of QR tokens at a time in LDS, QR = 4 / G
// for G <= 2 (so that every thread has an item), else 1; item i = (token
// i / (64 G), query head (i / 64) % G, position i % 64), so the lanes of a
// wave share one query (its reads are broadcasts).  Positions at or past a
// token's end are neither computed nor written.
template <int G, int NCK>
__global__ __launch_bounds__(256) void attn_qk(const float *__restrict__ q, size_t q_stride,
                                               const float *__restrict__ kc, int n_head_kv,
                                               int hd, const uint32_t *__restrict__ pos,
                                               int n_ctx, size_t att_stride,
                                               float *__restrict__ att, float *__restrict__ tmax,
                                               int n_tiles, int M)
{
    // NCK > 0: hd = 32 NCK, the K tile arrives in NCK chunks of 32
    // dimensions (eight quads of every row) and the first round adds each
    // chunk as soon as it is in LDS while the later chunks are still in
    // flight; NCK = 0: any hd, the whole tile first
    constexpr int QR = G == 1 ? 4 : G == 2 ? 2 : 1;  // tokens per round
    constexpr int NQ = QR * G;                        // queries per round (<= 8)
    constexpr int NIT = (NQ * SC_TILE + 255) / 256;   // items per thread
    extern __shared__ float4 qk_lds[];
    const int hd4 = hd >> 2, ks = hd4 + 1;
    float4 *Ks = qk_lds;                           // [SC_TILE][ks]
    float4 *Qs = qk_lds + SC_TILE * ks;           // [NQ][hd4]: query (token, head)
    const int tid = threadIdx.x, lane = tid & 63;
    const int tile = blockIdx.x, p0 = tile * SC_TILE, kvh = blockIdx.y;
    const int n_head = n_head_kv * G, kvd = n_head_kv * hd;
    const size_t pz = pos[0];
    auto upto_of = [&](int t) { return (int)min(pz + (size_t)t + 1, (size_t)n_ctx); };
    const int tz = (int)blockIdx.z * QK_TPW, t_end = min(tz + QK_TPW, M);
    const int upto_last = upto_of(t_end - 1);
    if (p0 >= upto_last) return;                   // (uniform)
    const int rows = min(SC_TILE, upto_last - p0);
    int t0 = tz;
    while (upto_of(t0) <= p0) t0++;                // (uniform) the first token reaching the tile
    // the queries of a round's tokens: quad f of the round is query f / hd4
    // (token t + f / (G hd4), head (f / hd4) % G), dimension quad f % hd4; at
    // most 512 quads (NQ <= 8, hd <= 256); tokens past t_end re-read the last
    // one.  The first round's are requested with the K tile.
    auto q_quad = [&](int t, int f) {
        const int qi = f / hd4, tt = min(t + qi / G, t_end - 1);
        return ((const float4 *)(q + (size_t)tt * q_stride + (size_t)kvh * G * hd))
            [(qi % G) * hd4 + f % hd4];
    };
    float4 qr[2];
    qr[0] = q_quad(t0, min(tid, NQ * hd4 - 1));
    qr[1] = q_quad(t0, min(tid + 256, NQ * hd4 - 1));
    const float4 *kb = (const float4 *)(kc + (size_t)p0 * kvd + (size_t)kvh * hd);
    // NCK > 0: thread tid's quads of chunk c are idx = tid + 256 u: row
    // idx / 8, quad 8 c + idx % 8 (a wave's load is eight 128-byte row pieces)
    // (native 4-vectors: an array of float4 structs stays in scratch memory)
    typedef float f4v __attribute__((ext_vector_type(4)));
    f4v kr[NCK > 0 ? NCK : 1][2];
    if constexpr (NCK > 0) {
#pragma unroll
        for (int c = 0; c < NCK; c++)
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int idx = tid + 256 * u, row = min(idx >> 3, rows - 1);
                kr[c][u] = ((const f4v *)kb)[(size_t)row * (kvd / 4) + 8 * c + (idx & 7)];
            }
    } else {
        // the whole K tile: float4 f is (row f / hd4, quad f % hd4); eight
        // loads in flight per thread before they go to LDS
        const int nf = rows * hd4;
        for (int f0 = 0; f0 < nf; f0 += 8 * 256) {
            float4 r[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int f = min(f0 + k * 256 + tid, nf - 1);
                r[k] = kb[(size_t)(f / hd4) * (kvd / 4) + f % hd4];
            }
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int f = f0 + k * 256 + tid;
                if (f < nf) Ks[(f / hd4) * ks + f % hd4] = r[k];
            }
        }
    }
    const float scale = fox_div(1.0f, fox_sqrtf((float)hd));
    // the products of quads d0 .. d1 - 1 added to acc in dimension order,
    // eight quads' reads issued before their adds
    auto dots = [&](float acc, const float4 *kq, const float4 *qv4, int d0, int d1) {
        int d = d0;
        for (; d + 8 <= d1; d += 8) {
            float4 kv[8], qv[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                kv[u] = kq[d + u];
                qv[u] = qv4[d + u];
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                acc = acc + qv[u].x * kv[u].x;
                acc = acc + qv[u].y * kv[u].y;
                acc = acc + qv[u].z * kv[u].z;
                acc = acc + qv[u].w * kv[u].w;
            }
        }
        for (; d < d1; d++) {
            const float4 kv = kq[d], qv = qv4[d];
            acc = acc + qv.x * kv.x;
            acc = acc + qv.y * kv.y;
            acc = acc + qv.z * kv.z;
            acc = acc + qv.w * kv.w;
        }
        return acc;
    };
    for (int t = t0; t < t_end; t += QR) {
        if (t > t0) {
            __syncthreads();                      // every item of the previous round is done
            qr[0] = q_quad(t, min(tid, NQ * hd4 - 1));
            qr[1] = q_quad(t, min(tid + 256, NQ * hd4 - 1));
        }
        if (tid < NQ * hd4) Qs[tid] = qr[0];
        if (tid + 256 < NQ * hd4) Qs[tid + 256] = qr[1];
        // item it of this thread: query qi = item / 64 (token tt, head g),
        // position p
        float acc[NIT];
#pragma unroll
        for (int it = 0; it < NIT; it++) acc[it] = 0.0f;
        auto item_of = [&](int it, int &qi, int &pl, int &tt, bool &ok) {
            const int item = it * 256 + tid;
            qi = item >> 6;
            pl = item & 63;
            tt = t + qi / G;
            ok = item < NQ * SC_TILE && tt < t_end && p0 + pl < upto_of(tt);
        };
        if constexpr (NCK > 0) {
#pragma unroll
            for (int c = 0; c < NCK; c++) {
                if (t == t0) {
#pragma unroll
                    for (int u = 0; u < 2; u++) {
                        const int idx = tid + 256 * u;
                        ((f4v *)Ks)[(idx >> 3) * ks + 8 * c + (idx & 7)] = kr[c][u];
                    }
                }
                if (t == t0 || c == 0) __syncthreads();
#pragma unroll
                for (int it = 0; it < NIT; it++) {
                    int qi, pl, tt;
                    bool ok;
                    item_of(it, qi, pl, tt, ok);
                    if (ok) acc[it] = dots(acc[it], Ks + pl * ks, Qs + qi * hd4, 8 * c, 8 * c + 8);
                }
            }
        } else {
            __syncthreads();
#pragma unroll
            for (int it = 0; it < NIT; it++) {
                int qi, pl, tt;
                bool ok;
                item_of(it, qi, pl, tt, ok);
                if (ok) acc[it] = dots(acc[it], Ks + pl * ks, Qs + qi * hd4, 0, hd4);
            }
        }
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            int qi, pl, tt;
            bool ok;
            item_of(it, qi, pl, tt, ok);
            if (it * 256 >= NQ * SC_TILE) break;  // (uniform: no items)
            const int g = qi % G;
            const float sc = acc[it] * scale;
            if (ok) att[((size_t)tt * n_head + (size_t)kvh * G + g) * att_stride + p0 + pl] = sc;
            // the tile maximum, NaN never taken (a wave is one query: its
            // lanes' tokens are the same)
            const float m = wave_reduce((ok && sc == sc) ? sc : -INFINITY, -INFINITY,
                                        [](float x, float y) { return y > x ? y : x; });
            if (lane == 0 && tt < t_end)
                tmax[((size_t)tt * n_head + (size_t)kvh * G + g) * n_tiles + tile] = m;
        }
    }
}

// Dependent add chains of the value and softmax sums.  AV_CH chains per
// value workgroup of several tokens (attn_avm), AV_VD blocks of V in flight
// per producer lane; a workgroup of the value kernels takes more than half
// of a compute unit's LDS (AV_LDS_MIN), so that its chain wave has SIMD 0 to
// itself.
#define AV_CH 16
#define AV_VD 4
#define AV_LDS_MIN (81 * 1024)

// The softmax sum over block [j0, j1) of e (j0 a multiple of 4), by the
// whole wave: blocks that start from position SUM_FAST_FROM on through
// sum_in_order, earlier ones through the plain chain (there the running sum
// still climbs a binade every few hundred elements or less, and each climb
// is an event that costs sum_in_order as much as a run).  e must be
// readable up to SUM_CHUNK floats past j1.  (4B-class decode at 2048+ rows:
// from 512 on, the blocks from 960, 517.3 tok/s; from 1024 on 515.5; from
// 2048 on 512.3-514.2; no block 508.8.)
#ifndef SUM_FAST_FROM
#define SUM_FAST_FROM 512
#endif
__device__ __forceinline__ float softmax_sum_block(float sum, const float *e, int j0, int j1)
{
    if (j0 >= SUM_FAST_FROM) return sum_in_order(sum, e + j0, j1 - j0);
    const int nq = (j1 - j0) >> 2;
    sum = chain_quads(sum, (const float4 *)(e + j0), nq);
    for (int j = j0 + 4 * nq; j < j1; j++) sum = sum + e[j];
    return sum;
}

// ---- one token: softmax and values of one query head per workgroup, for
// HV_CH of its columns (256 threads).  Wave 0 runs the chains: lane 0 the
// softmax sum, then lanes 0 .. HV_CH - 1 the value sums of columns
// c0 .. c0 + HV_CH - 1; waves 1-3 produce their operands.
//   1. the head's maximum from its tile maxima (wave 0);
//   2. exp blocks (HV_B0 positions, then HV_EB): waves 1-3 write e_j =
//      expf(s_j - max) of block k to LDS while wave 0 adds block k - 1 to
//      the sum (softmax_sum_block); a barrier between blocks;
//   3. 1 / sum;
//   4. value blocks of VB quads: waves 1-3 multiply block b's V quads
//      (loaded VD blocks ahead) by a_j = e_j * (1/sum) into one of two
//      product buffers while wave 0 adds block b - 1's products to its
//      chains; a barrier between blocks.
// The exps of a head are computed by the hd / HV_CH workgroups of its column
// groups only (each is a run of double-precision operations); the G query
// heads that read the same V columns have the same blockIdx.x % 8, so that
// they run on one XCD and V comes from its L2 once.
#ifndef HV_CH
#define HV_CH 16            // value chains (columns) per workgroup
#endif
#define HV_B0 192           // positions of the first exp block (one per producer lane)
#define HV_EB 768           // positions of a later exp block (four per producer lane)
// value blocks (VB quads, VD of them of V in flight per producer lane, a
// product buffer of VB + 1 quads per chain: one quad of padding): 192 quads
// (768 positions, half the chain restarts of 96) where a head's weights
// leave room for their product buffers, else 96
#define HV_VB_BIG 192
#define HV_VD_BIG 2
#define HV_VB 96
#define HV_VD 4
__host__ __device__ constexpr size_t hv_lds_bytes(int estr, int vb)
{
    return (size_t)estr * 4 + 2 * HV_CH * (size_t)(vb + 1) * 16;
}

template <int VB, int VD>
__global__ __launch_bounds__(256) void attn_hv(const float *__restrict__ att, size_t att_stride,
                                               const float *__restrict__ tmax, int n_tiles,
                                               const float *__restrict__ vc, int n_head,
                                               int n_head_kv, int hd,
                                               const uint32_t *__restrict__ pos, int n_ctx,
                                               float *__restrict__ out, int estr)
{
    typedef float f4v __attribute__((ext_vector_type(4)));
    constexpr int PS = VB + 1;                     // quads per chain in a product buffer
    constexpr int NP = HV_CH * VB / 192;           // (column, quad) pairs per producer lane and block
    constexpr int QS = 192 / HV_CH;                // quad step of a producer lane's pairs
    static_assert(192 % HV_CH == 0 && NP * 192 == HV_CH * VB && VB % QS == 0,
                  "producer lane L takes column L % HV_CH and quads L / HV_CH + QS k");
    extern __shared__ float4 hv_lds[];
    float *e = (float *)hv_lds;                    // [estr]: e_j
    float4 *prod = hv_lds + estr / 4;              // [2][HV_CH][PS]
    __shared__ float mx_s, inv_s;
    __shared__ uint64_t tab[32];
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_index();
    // workgroup -> (kv head, column group, query head of the group): u =
    // kvh * ncg + cg keeps blockIdx.x % 8 for all G query heads
    const int G = n_head / n_head_kv, ncg = (hd + HV_CH - 1) / HV_CH;
    const int bx = blockIdx.x, rest = bx >> 3;
    const int g = rest % G, u = (bx & 7) + 8 * (rest / G);
    if (u >= n_head_kv * ncg) return;              // (uniform: the grid's padding)
    const int kvh = u / ncg, c0 = (u - kvh * ncg) * HV_CH, h = kvh * G + g;
    const int kvd = n_head_kv * hd;
    const int upto = (int)min((size_t)pos[0] + 1, (size_t)n_ctx);
    const int nq = upto >> 2, rem = upto & 3, nq_all = (upto + 3) >> 2;
    const float *srow = att + (size_t)h * att_stride;
    const bool producer = wave > 0;
    const int L = tid - 64;                        // producer lane 0 .. 191

    // the scores of the producer's positions of exp block k: block 0 is
    // [0, HV_B0), block k >= 1 [HV_B0 + (k - 1) HV_EB, + HV_EB); lane L takes
    // start + L + 192 i (one position in block 0, four later)
    auto blk0 = [&](int k) { return k == 0 ? 0 : HV_B0 + (k - 1) * HV_EB; };
    const int neb = upto <= HV_B0 ? 1 : 1 + (upto - HV_B0 + HV_EB - 1) / HV_EB;
    const int neb2 = (neb + 1) & ~1;               // (barriers after block 0: an even number)
    auto s_load = [&](int k, float *s) {
#pragma unroll
        for (int i = 0; i < 4; i++) s[i] = srow[min(blk0(k) + L + 192 * i, upto - 1)];
    };
    float sc[4];
    if (producer) s_load(0, sc);

    // 1. the head's maximum (src/ops.c:26-30: a NaN first score stays)
    if (wave == 0) {
        const float *tm = tmax + (size_t)h * n_tiles;
        const int used = (upto + SC_TILE - 1) / SC_TILE;
        float m = -INFINITY;
        for (int i = lane; i < used; i += 64) {
            const float v = tm[i];
            m = v > m ? v : m;
        }
        m = wave_reduce(m, -INFINITY, [](float x, float y) { return y > x ? y : x; });
        const float s0 = srow[0];
        if (lane == 0) mx_s = s0 != s0 ? s0 : m;
    }
    if (tid < 32) tab[tid] = fox_exp2_tab[tid];
    __syncthreads();

    // V of value blocks 0 .. VD - 1: producer lane L, pair k is column
    // c0 + L % HV_CH, quad L / HV_CH + QS k of the block (a wave's loads of
    // one k are runs of HV_CH consecutive quads).  Requested after exp blocks 0
    // and 1's scores, so that those do not wait for them; block b's V is in
    // vb[b % VD], the block loop unrolled by VD (every index known at
    // compile time, each slot reloaded in place).
    const f4v *v4 = (const f4v *)vc;
    const int vcol = kvh * hd + min(c0 + L % HV_CH, hd - 1);
    const int nvb = (nq_all + VB - 1) / VB;
    f4v vb[VD][NP];
    auto v_load = [&](int b, f4v *dst) {
#pragma unroll
        for (int k = 0; k < NP; k++) {
            const int jq = min(b * VB + L / HV_CH + QS * k, nq_all - 1);
            dst[k] = v4[(size_t)jq * kvd + vcol];
        }
    };

    // 2. exp blocks and the softmax sum (lane 0 of wave 0)
    float sum = 0.0f;
    if (producer) {
        const float m = mx_s;
        auto exps = [&](int k, const float *cur) {
            const int j0 = blk0(k), ni = k == 0 ? 1 : 4;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int j = j0 + L + 192 * i;
                if (i < ni && j < upto) e[j] = fox_expf_t(cur[i] - m, tab);
            }
        };
        // block 0 outside the loop: the V loads go out after block 1's
        // scores.  Then two blocks per iteration, their scores in two sets
        // of registers, each reloaded in place (a load into a temporary
        // moved into place would wait for the load at the move).
        float sb[4];
        s_load(min(1, neb - 1), sb);
#pragma unroll
        for (int d = 0; d < VD; d++) v_load(min(d, nvb - 1), vb[d]);
        exps(0, sc);
        __syncthreads();
        for (int k = 1; k <= neb2; k += 2) {
            s_load(min(k + 1, neb - 1), sc);
            if (k < neb) exps(k, sb);
            __syncthreads();
            s_load(min(k + 2, neb - 1), sb);
            if (k + 1 < neb) exps(k + 1, sc);
            __syncthreads();
        }
    } else {
        __syncthreads();
        for (int k = 1; k <= neb2; k++) {
            if (k <= neb) sum = softmax_sum_block(sum, e, blk0(k - 1), min(upto, blk0(k)));
            __syncthreads();
        }
    }

    // 3. a_j = e_j * (1/sum), or e_j where the sum is not positive
    // (src/ops.c:35-38); the producers apply it as they form the products
    if (wave == 0 && lane == 0) inv_s = sum > 0.0f ? fox_div(1.0f, sum) : 1.0f;
    __syncthreads();
    const float iv = inv_s;

    // 4. value blocks: products by waves 1-3, chains by wave 0 (lane c:
    // column c0 + c).  Indices are clamped, so steps past the last block
    // recompute the last quads into the buffer the chains are not reading.
    float acc = 0.0f;
    // (all of a step's e quads are read before the first product is
    // stored: a store to the product buffer may not be moved above a later
    // read of e, so reads interleaved with stores would pay the LDS latency
    // once per pair)
    auto produce = [&](int b, f4v *vs) {
        // (the unrolled loop runs to the next multiple of VD past nvb: those
        // steps are only their barriers)
        if (b > nvb) return;                               // (uniform)
        float4 *P = prod + (b & 1) * HV_CH * PS + (L % HV_CH) * PS;
        float4 a[NP];
#pragma unroll
        for (int k = 0; k < NP; k++)
            a[k] = ((const float4 *)e)[min(b * VB + L / HV_CH + QS * k, nq_all - 1)];
#pragma unroll
        for (int k = 0; k < NP; k++) {
            const float4 ak = make_float4(a[k].x * iv, a[k].y * iv, a[k].z * iv, a[k].w * iv);
            const f4v v = vs[k];
            float4 p;
            p.x = ak.x * v.x; p.y = ak.y * v.y; p.z = ak.z * v.z; p.w = ak.w * v.w;
            P[L / HV_CH + QS * k] = p;
        }
        v_load(min(b + VD, nvb - 1), vs);
    };
    // the chains over block b - 1: whole quads below upto, then the ragged
    // quad's first rem products
    auto chains = [&](int b) {
        if (b > 0 && b <= nvb && lane < HV_CH) {
            const float4 *P = prod + ((b - 1) & 1) * HV_CH * PS + lane * PS;
            const int nfull = min(VB, nq - (b - 1) * VB);
            acc = chain_quads(acc, P, nfull);
            if (b == nvb && rem) {
                const float4 v = P[nfull];
                acc = acc + v.x;
                if (rem > 1) acc = acc + v.y;
                if (rem > 2) acc = acc + v.z;
            }
        }
    };
    // (the block loop unrolled by VD: block b + d's V is in vb[d])
    if (producer) {
        for (int b = 0; b <= nvb; b += VD) {
#pragma unroll
            for (int d = 0; d < VD; d++) {
                produce(b + d, vb[d]);
                __syncthreads();
            }
        }
    } else {
        for (int b = 0; b <= nvb; b += VD) {
#pragma unroll
            for (int d = 0; d < VD; d++) {
                chains(b + d);
                __syncthreads();
            }
        }
        if (lane < HV_CH && c0 + lane < hd) out[(size_t)h * hd + c0 + lane] = acc;
    }
}

// ---- several tokens, or a context longer than attn_hv's LDS holds: the
// softmax and the values in two launches.
//   attn_sm   a workgroup per (query head, token): the maximum, then e_j in
//             blocks of SM_EB positions by waves 1-3 while lane 0 of wave 0
//             adds the block before, then a_j = e_j * (1/sum) written over
//             the scores;
//   attn_avm  a workgroup per (kv head, AV_CH / G columns, MT tokens): wave 0
//             runs the MT x AV_CH chains (lane = token * AV_CH + head * DC +
//             column); waves 1-3 stage block b + 1's a_j and V quads from
//             registers (loaded AV_VD blocks ahead) into LDS and multiply block
//             b's into one of two product buffers while wave 0 adds block
//             b - 1; a barrier between blocks.
#define SM_EB 768           // positions of a softmax exp block (four per producer lane)
#define MT 4                // tokens per attn_avm workgroup
#ifndef MV_VB
#define MV_VB 48            // quads of an attn_avm value block
#endif
#define MV_PS (MV_VB + 1)

__global__ __launch_bounds__(256) void attn_sm(float *__restrict__ att, size_t att_stride,
                                               const float *__restrict__ tmax, int n_tiles,
                                               int n_head, const uint32_t *__restrict__ pos,
                                               int n_ctx)
{
    extern __shared__ float4 sm_lds[];
    float *e = (float *)sm_lds;                    // [ceil4(upto)]
    __shared__ float mx_s, inv_s;
    __shared__ uint64_t tab[32];
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_index();
    const int h = blockIdx.x, t = blockIdx.y;
    const int upto = (int)min((size_t)pos[0] + (size_t)t + 1, (size_t)n_ctx);
    float *row = att + ((size_t)t * n_head + h) * att_stride;
    const bool producer = wave > 0;
    const int L = tid - 64;
    const int neb = (upto + SM_EB - 1) / SM_EB;
    auto s_load = [&](int k) {
        return *(const float4 *)(row + min(k * SM_EB + 4 * L, (upto - 1) & ~3));
    };
    float4 sc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (producer) sc = s_load(0);
    if (wave == 0) {
        // src/ops.c:26-30: a NaN first score stays the maximum
        const float *tm = tmax + ((size_t)t * n_head + h) * n_tiles;
        const int used = (upto + SC_TILE - 1) / SC_TILE;
        float m = -INFINITY;
        for (int i = lane; i < used; i += 64) {
            const float v = tm[i];
            m = v > m ? v : m;
        }
        m = wave_reduce(m, -INFINITY, [](float x, float y) { return y > x ? y : x; });
        const float s0 = row[0];
        if (lane == 0) mx_s = s0 != s0 ? s0 : m;
    }
    if (tid < 32) tab[tid] = fox_exp2_tab[tid];
    __syncthreads();
    float sum = 0.0f;
    if (producer) {
        const float m = mx_s;
        for (int k = 0; k <= neb; k++) {
            const float4 cur = sc;
            sc = s_load(min(k + 1, neb - 1));
            const int j = k * SM_EB + 4 * L;
            if (k < neb && j < upto) {
                float4 x;
                x.x = fox_expf_t(cur.x - m, tab);
                x.y = j + 1 < upto ? fox_expf_t(cur.y - m, tab) : 0.0f;
                x.z = j + 2 < upto ? fox_expf_t(cur.z - m, tab) : 0.0f;
                x.w = j + 3 < upto ? fox_expf_t(cur.w - m, tab) : 0.0f;
                *(float4 *)(e + j) = x;
            }
            __syncthreads();
        }
    } else {
        for (int k = 0; k <= neb; k++) {
            if (k > 0)
                sum = softmax_sum_block(sum, e, (k - 1) * SM_EB, min(upto, k * SM_EB));
            __syncthreads();
        }
    }
    // src/ops.c:35-38: a_j = e_j * (1/sum) when the sum is positive
    if (tid == 0) inv_s = sum > 0.0f ? fox_div(1.0f, sum) : 1.0f;
    __syncthreads();
    const float inv = inv_s;
    for (int jq = tid; jq < (upto + 3) >> 2; jq += 256) {
        float4 v = ((const float4 *)e)[jq];
        v.x = v.x * inv; v.y = v.y * inv; v.z = v.z * inv; v.w = v.w * inv;
        ((float4 *)row)[jq] = v;
    }
}

template <int G>
__global__ __launch_bounds__(256) void attn_avm(const float *__restrict__ att, size_t att_stride,
                                                const float *__restrict__ vc, int n_head_kv,
                                                int hd, int gq, const uint32_t *__restrict__ pos,
                                                int n_ctx, float *__restrict__ out,
                                                size_t out_stride, int M)
{
    // G: the query heads per kv head, gq, rounded up to a power of two (the
    // rows of heads gq .. G - 1 repeat head gq - 1 and are not written)
    constexpr int DC = AV_CH / G;                  // columns of the workgroup
    constexpr int NR = G * MT;                     // weight rows (token, head)
    constexpr int NA = (NR * MV_VB + 191) / 192;   // weight quads per producer lane and block
    constexpr int NV = (DC * MV_VB + 191) / 192;   // V quads per producer lane and block
    constexpr int NP = MT * AV_CH * MV_VB / 192;   // products per producer lane and block
    static_assert(MT * AV_CH == 64 && MT * AV_CH * MV_VB % 192 == 0, "attn_avm lane layout");
    // (slots and staging as native 4-vectors: a float4 struct copied into
    // an array slot is a memcpy the compiler keeps in scratch memory)
    typedef float f4v __attribute__((ext_vector_type(4)));
    __shared__ f4v A[2][NR * MV_VB], Vs[2][DC * MV_VB];
    extern __shared__ float4 prod[];               // [2][64][MV_PS]
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_index();
    const int n_cg = (hd + DC - 1) / DC;           // (columns past hd: V's last column, not written)
    const int kvh = blockIdx.x / n_cg, c0 = (blockIdx.x - kvh * n_cg) * DC;
    const int n_head = n_head_kv * gq, kvd = n_head_kv * hd;
    const int t0 = (int)blockIdx.y * MT, nt = min(MT, M - t0);
    auto upto_of = [&](int tl) { return (int)min((size_t)pos[0] + (size_t)(t0 + tl) + 1, (size_t)n_ctx); };
    const int upto_max = upto_of(nt - 1), nq_max = (upto_max + 3) >> 2;
    const int nvb = (nq_max + MV_VB - 1) / MV_VB;
    const bool producer = wave > 0;
    const int L = tid - 64;

    // a producer lane's loads of block b: weight quads (row r = token *
    // G + head, quad qq) and V quads (column c, quad qq); indices clamped, so
    // every load is inside the buffers (rows of tokens past nt and quads past
    // a token's end are loaded and multiplied, never added)
    struct Slot { f4v a[NA], v[NV]; };
    auto load = [&](int b, Slot &sl) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < NA; k++) {
            const int pa = min(L + 192 * k, NR * MV_VB - 1), r = pa / MV_VB;
            const int tl = min(r / G, nt - 1), g = min(r - (r / G) * G, gq - 1);
            const int jq = min(b * MV_VB + (pa - r * MV_VB), nq_max - 1);
            sl.a[k] = ((const f4v *)(att + ((size_t)(t0 + tl) * n_head + (size_t)kvh * gq + g) *
                                               att_stride))[jq];
        }
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const int pv = min(L + 192 * k, DC * MV_VB - 1), c = pv / MV_VB;
            const int jq = min(b * MV_VB + (pv - c * MV_VB), nq_max - 1);
            sl.v[k] = ((const f4v *)vc)[(size_t)jq * kvd + (size_t)kvh * hd + min(c0 + c, hd - 1)];
        }
    };
    auto stage = [&](int b, const Slot &sl) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < NA; k++) {
            const int pa = L + 192 * k;
            if (pa < NR * MV_VB) A[b & 1][pa] = sl.a[k];
        }
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const int pv = L + 192 * k;
            if (pv < DC * MV_VB) Vs[b & 1][pv] = sl.v[k];
        }
    };
    // the products of block b from the staged quads: product pi = L + 192 k
    // is chain pi / MV_VB (token, head, column), quad pi % MV_VB
    // (eight products' operands are read before the first of them is
    // stored: a store to the product buffer may not be moved above a later
    // read of the staging buffers, so reads interleaved with stores would
    // pay the LDS latency once per product)
    auto products = [&](int b) __attribute__((always_inline)) {
        float4 *P = prod + (b & 1) * 64 * MV_PS;
        static_assert(NP % 8 == 0, "products in groups of eight");
#pragma unroll
        for (int k0 = 0; k0 < NP; k0 += 8) {
            f4v a[8], v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int pi = L + 192 * (k0 + k), ch = pi / MV_VB, qq = pi - ch * MV_VB;
                const int tl = ch / AV_CH, rm = ch - tl * AV_CH, g = rm / DC, c = rm - g * DC;
                a[k] = A[b & 1][(tl * G + g) * MV_VB + qq];
                v[k] = Vs[b & 1][c * MV_VB + qq];
            }
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int pi = L + 192 * (k0 + k), ch = pi / MV_VB, qq = pi - ch * MV_VB;
                float4 p;
                p.x = a[k].x * v[k].x; p.y = a[k].y * v[k].y;
                p.z = a[k].z * v[k].z; p.w = a[k].w * v[k].w;
                P[ch * MV_PS + qq] = p;
            }
        }
    };
    // wave 0: chain lane = (token tl, head g, column c); its token's whole
    // quads of block b - 1, then its ragged quad's first rem products
    const int tl = lane / AV_CH, rm = lane - tl * AV_CH;
    const int my_upto = upto_of(min(tl, nt - 1)), my_nq = my_upto >> 2, my_rem = my_upto & 3;
    const int nq_min = upto_of(0) >> 2;            // (the shortest token's whole quads)
    float acc = 0.0f;
    auto chains = [&](int b) __attribute__((always_inline)) {
        // groups of 16 quads whole for every token: one wave-uniform asm
        // chain; then the lane's own rest
        const int q0 = (b - 1) * MV_VB;
        const int ng = __builtin_amdgcn_readfirstlane(max(0, min(MV_VB, nq_min - q0)) >> 4);
        if (b > 0 && b <= nvb && tl < nt) {
            const float4 *P = prod + ((b - 1) & 1) * 64 * MV_PS + lane * MV_PS;
            if (ng > 0) acc = chain_lds16(acc, P, ng);
            const int nfull = min(MV_VB, my_nq - q0);
            for (int i = ng << 4; i < nfull; i++) {
                const float4 v = P[i];
                acc = acc + v.x; acc = acc + v.y; acc = acc + v.z; acc = acc + v.w;
            }
            if (my_rem && nfull >= 0 && nfull < MV_VB) {
                const float4 v = P[nfull];
                acc = acc + v.x;
                if (my_rem > 1) acc = acc + v.y;
                if (my_rem > 2) acc = acc + v.z;
            }
        }
    };
    static_assert(AV_VD == 4, "the block loop is unrolled by AV_VD");
    if (producer) {
        // slot s holds block b with b % AV_VD == s; step b stages block b + 1
        // and multiplies block b
        Slot sl[AV_VD];
#pragma unroll
        for (int d = 0; d < AV_VD; d++) load(min(d, nvb - 1), sl[d]);
        stage(0, sl[0]);
        load(min(AV_VD, nvb - 1), sl[0]);
        __syncthreads();
        // (steps past nvb, to the next multiple of AV_VD: only their
        // barriers)
        auto step = [&](int b, Slot &s1) __attribute__((always_inline)) {
            if (b <= nvb) {                                // (uniform)
                stage(b + 1, s1);
                load(min(b + 1 + AV_VD, nvb - 1), s1);
                products(b);
            }
            __syncthreads();
        };
        for (int b = 0; b <= nvb; b += AV_VD) {
            step(b, sl[1]);
            step(b + 1, sl[2]);
            step(b + 2, sl[3]);
            step(b + 3, sl[0]);
        }
    } else {
        __syncthreads();
        for (int b = 0; b <= nvb; b += AV_VD) {
#pragma unroll
            for (int d = 0; d < AV_VD; d++) {
                chains(b + d);
                __syncthreads();
            }
        }
        const int g = rm / DC, c = rm - g * DC;
        if (tl < nt && g < gq && c0 + c < hd)
            out[(size_t)(t0 + tl) * out_stride + (size_t)(kvh * gq + g) * hd + c0 + c] = acc;
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
        if (n_ctx > ATT_EXACT_MAX_CTX)
            return fox_fail(FOX_GPU_ERR_UNSUPPORTED,
                            "attention: exact mode keeps a head's %zu weights in LDS; at most "
                            "%d positions", n_ctx, ATT_EXACT_MAX_CTX);
        const size_t att_stride = (n_ctx + 3) & ~(size_t)3;
        const int n_tiles = (int)((n_ctx + SC_TILE - 1) / SC_TILE);
        const size_t att_bytes = M * n_head * att_stride * sizeof(float);
        const size_t bytes = att_bytes + M * n_head * (size_t)n_tiles * sizeof(float);
        fox_gpu_status st = fox_ws_reserve(ctx, bytes);
        if (st) return st;
        float *att = (float *)ctx->ws;
        float *tmax = (float *)(ctx->ws + att_bytes);
        const size_t gqa = n_head / n_head_kv;
        const int ikv = (int)n_head_kv, ihd = (int)head_dim, ictx = (int)n_ctx;
        {
            // scores: the K tile (a padding quad per row) and G query heads
            const size_t nq = gqa <= 2 ? 4 : gqa;          // (queries of a round: attn_qk's QR G)
            const size_t lds = ((size_t)SC_TILE * (head_dim / 4 + 1) + nq * head_dim / 4) * 16;
            // (head_dim 128: the K tile in four chunks, the first round's
            // adds overlapping the later chunks' loads)
            const bool ck = head_dim == 128;
#define FOX_QK(g) (ck ? (const void *)attn_qk<g, 4> : (const void *)attn_qk<g, 0>)
            const void *qk = gqa == 1 ? FOX_QK(1) : gqa == 2 ? FOX_QK(2) : gqa == 3 ? FOX_QK(3)
                           : gqa == 4 ? FOX_QK(4) : gqa == 5 ? FOX_QK(5) : gqa == 6 ? FOX_QK(6)
                           : gqa == 7 ? FOX_QK(7) : FOX_QK(8);
#undef FOX_QK
            if (lds > 64 * 1024) {
                hipError_t e = hipFuncSetAttribute(qk, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   (int)lds);
                if (e != hipSuccess) return fox_hip_fail(e, "attention: LDS size");
            }
            const int iM = (int)M;
            void *args[] = {(void *)&q, (void *)&qs, (void *)&k_cache, (void *)&ikv, (void *)&ihd,
                            (void *)&pos, (void *)&ictx, (void *)&att_stride, (void *)&att,
                            (void *)&tmax, (void *)&n_tiles, (void *)&iM};
            hipError_t e = hipLaunchKernel(qk, dim3((unsigned)n_tiles, (unsigned)n_head_kv,
                                                    (unsigned)((M + QK_TPW - 1) / QK_TPW)),
                                           dim3(256), args, lds, ctx->stream);
            if (e != hipSuccess) return fox_hip_fail(e, "attention scores");
            FOX_LAUNCHED("attention scores");
        }
        // one token: softmax and values in one launch, when the head's
        // weights fit in LDS beside the product buffers
        const int estr = (int)((n_ctx + 31) & ~(size_t)31);
        // (at least AV_LDS_MIN: more than half of a compute unit's LDS, so
        // that no two workgroups share a compute unit, whose chain waves
        // would share SIMD 0's instruction issue)
#ifndef HV_BIG_OFF
        const bool big = hv_lds_bytes(estr, HV_VB_BIG) <= ATT_LDS_MAX;
#else
        const bool big = false;
#endif
        size_t hv_lds = hv_lds_bytes(estr, big ? HV_VB_BIG : HV_VB);
        if (hv_lds < AV_LDS_MIN) hv_lds = AV_LDS_MIN;
        if (M == 1 && hv_lds <= ATT_LDS_MAX) {
            const void *hv = big ? (const void *)attn_hv<HV_VB_BIG, HV_VD_BIG>
                                 : (const void *)attn_hv<HV_VB, HV_VD>;
            hipError_t e = hipFuncSetAttribute(hv, hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)hv_lds);
            if (e != hipSuccess) return fox_hip_fail(e, "attention: LDS size");
            const size_t ncg = (head_dim + HV_CH - 1) / HV_CH;
            const size_t nwg = (n_head_kv * ncg + 7) / 8 * 8 * gqa;
            const int in_head = (int)n_head;
            void *args[] = {(void *)&att, (void *)&att_stride, (void *)&tmax, (void *)&n_tiles,
                            (void *)&v_cache, (void *)&in_head, (void *)&ikv, (void *)&ihd,
                            (void *)&pos, (void *)&ictx, (void *)&out, (void *)&estr};
            e = hipLaunchKernel(hv, dim3((unsigned)nwg), dim3(256), args, hv_lds, ctx->stream);
            if (e != hipSuccess) return fox_hip_fail(e, "attention softmax+values");
            FOX_LAUNCHED("attention softmax+values");
            return FOX_GPU_OK;
        }
        // softmax per (head, token), then the values of MT tokens per
        // workgroup
        const int gp = gqa == 1 ? 1 : gqa == 2 ? 2 : gqa <= 4 ? 4 : 8;
        const size_t dcm = AV_CH / gp;
        {
            // (SUM_CHUNK floats past the weights: softmax_sum_block reads
            // whole chunks of SUM_CHUNK)
            const size_t sm_lds = (att_stride + SUM_CHUNK) * sizeof(float);
            if (sm_lds > 64 * 1024) {
                hipError_t e = hipFuncSetAttribute((const void *)attn_sm,
                                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   (int)sm_lds);
                if (e != hipSuccess) return fox_hip_fail(e, "attention: LDS size");
            }
            hipLaunchKernelGGL(attn_sm, dim3((unsigned)n_head, (unsigned)M), dim3(256), sm_lds,
                               ctx->stream, att, att_stride, tmax, n_tiles, (int)n_head, pos,
                               (int)n_ctx);
            FOX_LAUNCHED("attention softmax");
        }
        const void *avm = gp == 1 ? (const void *)attn_avm<1> : gp == 2 ? (const void *)attn_avm<2>
                        : gp == 4 ? (const void *)attn_avm<4> : (const void *)attn_avm<8>;
        const size_t avm_lds = 2 * 64 * MV_PS * 16;
        hipError_t e = hipFuncSetAttribute(avm, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)avm_lds);
        if (e != hipSuccess) return fox_hip_fail(e, "attention: LDS size");
        const int iM = (int)M, igq = (int)gqa;
        void *args[] = {(void *)&att, (void *)&att_stride, (void *)&v_cache, (void *)&ikv,
                        (void *)&ihd, (void *)&igq, (void *)&pos, (void *)&ictx, (void *)&out,
                        (void *)&os, (void *)&iM};
        e = hipLaunchKernel(avm, dim3((unsigned)(n_head_kv * ((head_dim + dcm - 1) / dcm)),
                                      (unsigned)((M + MT - 1) / MT)),
                            dim3(256), args, avm_lds, ctx->stream);
        if (e != hipSuccess) return fox_hip_fail(e, "attention values");
        FOX_LAUNCHED("attention values");
        return FOX_GPU_OK;
    }
    if (mode != FOX_GPU_ATTN_SPLIT) return fox_fail(FOX_GPU_ERR_ARG, "attention: unknown mode %d", mode);
    const int split = head_dim == 128 ? FD_SPLIT_W : FD_SPLIT;
    const int n_splits = (int)((n_ctx + split - 1) / split);
    if (n_splits > FD_MAXS)
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "attention: split mode takes at most %d positions",
                        FD_MAXS * split);
    const size_t bytes = M * n_head * (size_t)n_splits * (4 + head_dim) * sizeof(float);
    fox_gpu_status st = fox_ws_reserve(ctx, bytes);
    if (st) return st;
    float *part = (float *)ctx->ws;
    const size_t gqa = n_head / n_head_kv, hd4 = head_dim / 4;
    const size_t lds = ((size_t)FD_SPLIT * (hd4 + 1) + gqa * hd4 + (FD_SPLIT / 4) * head_dim) * 16 +
                       gqa * FD_SPLIT * 4;
    const void *fd = gqa == 1 ? (const void *)attn_fd<1> : gqa == 2 ? (const void *)attn_fd<2>
                   : gqa == 3 ? (const void *)attn_fd<3> : gqa == 4 ? (const void *)attn_fd<4>
                   : gqa == 5 ? (const void *)attn_fd<5> : gqa == 6 ? (const void *)attn_fd<6>
                   : gqa == 7 ? (const void *)attn_fd<7> : (const void *)attn_fd<8>;
    const int ikv = (int)n_head_kv, ihd = (int)head_dim, ictx = (int)n_ctx;
    hipError_t e;
    if (head_dim == 128) {
        const void *f1 = gqa == 1 ? (const void *)attn_fd128<1> : gqa == 2 ? (const void *)attn_fd128<2>
                       : gqa == 3 ? (const void *)attn_fd128<3> : gqa == 4 ? (const void *)attn_fd128<4>
                       : gqa == 5 ? (const void *)attn_fd128<5> : gqa == 6 ? (const void *)attn_fd128<6>
                       : gqa == 7 ? (const void *)attn_fd128<7> : (const void *)attn_fd128<8>;
        void *args[] = {(void *)&q, (void *)&qs, (void *)&k_cache, (void *)&v_cache, (void *)&ikv,
                        (void *)&pos, (void *)&ictx, (void *)&n_splits, (void *)&part};
        e = hipLaunchKernel(f1, dim3((unsigned)n_splits, (unsigned)n_head_kv, (unsigned)M),
                            dim3(512), args, 0, ctx->stream);
    } else {
        if (lds > 64 * 1024) {
            e = hipFuncSetAttribute(fd, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return fox_hip_fail(e, "attention: LDS size");
        }
        void *args[] = {(void *)&q, (void *)&qs, (void *)&k_cache, (void *)&v_cache, (void *)&ikv,
                        (void *)&ihd, (void *)&pos, (void *)&ictx, (void *)&n_splits, (void *)&part};
        e = hipLaunchKernel(fd, dim3((unsigned)n_splits, (unsigned)n_head_kv, (unsigned)M),
                            dim3(256), args, lds, ctx->stream);
    }
    if (e != hipSuccess) return fox_hip_fail(e, "attention partial");
    FOX_LAUNCHED("attention partial");
    hipLaunchKernelGGL(attn_fdm, dim3((unsigned)n_head, (unsigned)M), dim3(256), 0, ctx->stream,
                       part, pos, ictx, (int)n_head, (int)head_dim, split, n_splits, out, os);
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
