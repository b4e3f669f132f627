// fox_ops.hip -- bandwidth-bound decode ops: row gather, RMSNorm, RoPE + KV
// store, split-position GQA attention, SwiGLU, residual add, argmax.
// Built with -ffp-contract=off like the rest of the library: every float op
// rounds once, in the reference's order where the reference fixes an order.
#include "fox_internal.h"
#include "fox_math.h"

#include <cmath>

// ------------------------------------------------------------------ rows

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
    const WT *row = src + (size_t)r * K;
    for (uint64_t k = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; k < K;
         k += (uint64_t)gridDim.x * blockDim.x)
        out[(size_t)i * out_stride + k] = (float)row[k];
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

__global__ __launch_bounds__(256) void rmsnorm_k(float *__restrict__ out, size_t out_stride,
                                                 const float *__restrict__ x, size_t x_stride,
                                                 const float *__restrict__ w, int n, float eps)
{
    __shared__ double red[4];
    __shared__ float sc;
    const int t = blockIdx.x, tid = threadIdx.x;
    const float *xt = x + (size_t)t * x_stride;
    double s = 0.0;
    for (int i = tid; i < n; i += 256) s += (double)xt[i] * (double)xt[i];
    s = wave_sum_d(s);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    if (tid == 0) {
        const double tot = (red[0] + red[1]) + (red[2] + red[3]);
        const double rel = (double)(n + 64) * 0x1p-52;
        const double y_hi = rms_scale_d(tot * (1.0 - rel), n, eps) * (1.0 + 0x1p-50);
        const double y_lo = rms_scale_d(tot * (1.0 + rel), n, eps) * (1.0 - 0x1p-50);
        float f_hi = (float)y_hi, f_lo = (float)y_lo;
        if (f_hi == f_lo) {
            sc = f_hi;
        } else {
            double seq = 0.0;
            for (int i = 0; i < n; i++) seq += (double)xt[i] * (double)xt[i];
            sc = (float)rms_scale_d(seq, n, eps);
        }
    }
    __syncthreads();
    const float scale = sc;
    float *ot = out + (size_t)t * out_stride;
    for (int i = tid; i < n; i += 256) {
        float v = xt[i] * scale;
        ot[i] = w ? v * w[i] : v;
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
    hipLaunchKernelGGL(rmsnorm_k, dim3((unsigned)M), dim3(256), 0, ctx->stream, out,
                       M > 1 ? out_stride : n, x, M > 1 ? x_stride : n, w, (int)n, eps);
    FOX_LAUNCHED("rmsnorm");
    return FOX_GPU_OK;
}

// ------------------------------------------------------------ rope+store

// src/ops.c:56-73 on q and k of token t at position pos[0]+t, then the
// src/forward.c:427-443 copies of k and v into cache row pos[0]+t.
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
        vc[p * kvd + i] = vt[i];
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

// -------------------------------------------------------------- attention

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
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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
    // o = sum_p e_p v_p, one (head, dim) per thread, rows read coalesced in d
    for (int i = tid; i < gqa * hd; i += 256) {
        const int g = i / hd, d = i % hd;
        float o = 0.0f;
        for (int pp = 0; pp < pn; pp++)
            o += sc[g * ATT_SPLIT + pp] * vc[(size_t)(p0 + pp) * kvd + (size_t)kvh * hd + d];
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


// ---- attention in the reference's order (src/forward.c:303-338,
// src/ops.c:24-39, 75-81), bit for bit:
//   score_j = (sum_d q_d k_jd, summed in d order) * (1 / sqrtf(hd));
//   softmax: max, e_j = expf(score_j - max), sum in j order, e_j * (1/sum);
//   out_d = sum in j order of a_j v_jd.
// Each in-order sum is one lane's chain; work is spread over lanes by
// position (scores), head (softmax) and head x dimension (values).

#define EX_TILE 32

__global__ __launch_bounds__(256) void attn_scores_exact(const float *__restrict__ q,
                                                         size_t q_stride,
                                                         const float *__restrict__ kc,
                                                         int n_head, int n_head_kv, int hd,
                                                         const uint32_t *__restrict__ pos,
                                                         int n_ctx, float *__restrict__ att)
{
    __shared__ float ks[EX_TILE * (ATT_MAXHD + 1)];
    __shared__ float qs[ATT_MAXG * ATT_MAXHD];
    const int p0 = blockIdx.x * EX_TILE, kvh = blockIdx.y, t = blockIdx.z, tid = threadIdx.x;
    const int gqa = n_head / n_head_kv, kvd = n_head_kv * hd, ks_stride = hd + 1;
    const int upto = (int)min((size_t)pos[0] + (size_t)t + 1, (size_t)n_ctx);
    if (p0 >= upto) return;
    const int pn = upto - p0 < EX_TILE ? upto - p0 : EX_TILE;
    for (int i = tid; i < pn * hd; i += 256) {
        const int j = i / hd, d = i % hd;
        ks[j * ks_stride + d] = kc[(size_t)(p0 + j) * kvd + (size_t)kvh * hd + d];
    }
    for (int i = tid; i < gqa * hd; i += 256)
        qs[i] = q[(size_t)t * q_stride + (size_t)kvh * gqa * hd + i];
    __syncthreads();
    const float scale = fox_div(1.0f, fox_sqrtf((float)hd));
    for (int i = tid; i < gqa * EX_TILE; i += 256) {
        const int g = i / EX_TILE, j = i % EX_TILE;
        if (j >= pn) continue;
        const float *qr = qs + g * hd, *kr = ks + j * ks_stride;
        float a = 0.0f;
        for (int d = 0; d < hd; d++) a = a + qr[d] * kr[d];
        att[((size_t)t * n_head + (size_t)kvh * gqa + g) * n_ctx + p0 + j] = a * scale;
    }
}

__global__ __launch_bounds__(256) void attn_softmax_exact(float *__restrict__ att, int n_head,
                                                          const uint32_t *__restrict__ pos,
                                                          int n_ctx)
{
    extern __shared__ float e[];
    __shared__ float red[4];
    __shared__ float inv_s;
    __shared__ int norm;
    const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    const int upto = (int)min((size_t)pos[0] + (size_t)t + 1, (size_t)n_ctx);
    float *row = att + ((size_t)t * n_head + h) * n_ctx;
    float m = -INFINITY;
    for (int j = tid; j < upto; j += 256) m = fmaxf(m, row[j]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    // src/ops.c:26-30: the maximum in index order from x[0]; with no NaN
    // this is the plain maximum
    const float mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int j = tid; j < upto; j += 256) e[j] = fox_expf(row[j] - mx);
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        int j = 0;
        for (; j + 8 <= upto; j += 8) {
            sum = sum + e[j];
            sum = sum + e[j + 1];
            sum = sum + e[j + 2];
            sum = sum + e[j + 3];
            sum = sum + e[j + 4];
            sum = sum + e[j + 5];
            sum = sum + e[j + 6];
            sum = sum + e[j + 7];
        }
        for (; j < upto; j++) sum = sum + e[j];
        norm = sum > 0.0f;
        inv_s = norm ? fox_div(1.0f, sum) : 1.0f;
    }
    __syncthreads();
    const float inv = inv_s;
    for (int j = tid; j < upto; j += 256) row[j] = norm ? e[j] * inv : e[j];
}

__global__ __launch_bounds__(64) void attn_values_exact(const float *__restrict__ att,
                                                        const float *__restrict__ vc,
                                                        int n_head, int n_head_kv, int hd,
                                                        const uint32_t *__restrict__ pos,
                                                        int n_ctx, float *__restrict__ out,
                                                        size_t out_stride)
{
    const int h = blockIdx.x, t = blockIdx.y, d = blockIdx.z * 64 + threadIdx.x;
    if (d >= hd) return;
    const int gqa = n_head / n_head_kv, kvh = h / gqa, kvd = n_head_kv * hd;
    const int upto = (int)min((size_t)pos[0] + (size_t)t + 1, (size_t)n_ctx);
    const float *a = att + ((size_t)t * n_head + h) * n_ctx;
    const float *v = vc + (size_t)kvh * hd + d;
    float acc = 0.0f;
    int j = 0;
    for (; j + 8 <= upto; j += 8) {
        float vv[8], aa[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            vv[u] = v[(size_t)(j + u) * kvd];
            aa[u] = a[j + u];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) acc = acc + aa[u] * vv[u];
    }
    for (; j < upto; j++) acc = acc + a[j] * v[(size_t)j * kvd];
    out[(size_t)t * out_stride + (size_t)h * hd + d] = acc;
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
    if (n_head / n_head_kv > ATT_MAXG || head_dim > ATT_MAXHD)
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED,
                        "attention: at most %d query heads per kv head and head_dim %d",
                        ATT_MAXG, ATT_MAXHD);
    if (M > FOX_GPU_MAX_TOKENS) return fox_fail(FOX_GPU_ERR_ARG, "attention: too many tokens");
    if (mode == FOX_GPU_ATTN_EXACT) {
        const size_t bytes = M * n_head * n_ctx * sizeof(float);
        if (n_ctx * sizeof(float) > 60 * 1024)
            return fox_fail(FOX_GPU_ERR_UNSUPPORTED,
                            "attention: exact mode keeps a head's %zu scores in LDS; at most "
                            "15360 positions", n_ctx);
        fox_gpu_status st = fox_ws_reserve(ctx, bytes);
        if (st) return st;
        float *att = (float *)ctx->ws;
        const size_t qs = M > 1 ? q_stride : n_head * head_dim;
        hipLaunchKernelGGL(attn_scores_exact,
                           dim3((unsigned)((n_ctx + EX_TILE - 1) / EX_TILE), (unsigned)n_head_kv,
                                (unsigned)M), dim3(256), 0, ctx->stream, q, qs, k_cache,
                           (int)n_head, (int)n_head_kv, (int)head_dim, pos, (int)n_ctx, att);
        FOX_LAUNCHED("attention scores");
        hipLaunchKernelGGL(attn_softmax_exact, dim3((unsigned)n_head, (unsigned)M), dim3(256),
                           n_ctx * sizeof(float), ctx->stream, att, (int)n_head, pos, (int)n_ctx);
        FOX_LAUNCHED("attention softmax");
        hipLaunchKernelGGL(attn_values_exact,
                           dim3((unsigned)n_head, (unsigned)M, (unsigned)((head_dim + 63) / 64)),
                           dim3(64), 0, ctx->stream, att, v_cache, (int)n_head, (int)n_head_kv,
                           (int)head_dim, pos, (int)n_ctx, out,
                           M > 1 ? out_stride : n_head * head_dim);
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
                       dim3(256), 0, ctx->stream, q, M > 1 ? q_stride : n_head * head_dim,
                       k_cache, v_cache, (int)n_head, (int)n_head_kv, (int)head_dim, pos,
                       (int)n_ctx, n_splits, part);
    FOX_LAUNCHED("attention partial");
    hipLaunchKernelGGL(attn_merge, dim3((unsigned)n_head, (unsigned)M), dim3(128), 0, ctx->stream,
                       part, (int)n_head, (int)head_dim, n_splits, out,
                       M > 1 ? out_stride : n_head * head_dim);
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
__global__ __launch_bounds__(1024) void argmax_k(const float *__restrict__ x, int n,
                                                 uint32_t *__restrict__ idx,
                                                 uint32_t *__restrict__ pos, uint32_t advance,
                                                 uint32_t *__restrict__ history)
{
    __shared__ float bv[16];
    __shared__ int bi[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float best = -INFINITY;
    int bidx = 0x7fffffff;
    for (int i = tid; i < n; i += 1024) {
        float v = x[i];
        if (v > best) { best = v; bidx = i; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(best, o);
        int oi = __shfl_xor(bidx, o);
        if (ov > best || (ov == best && oi < bidx)) { best = ov; bidx = oi; }
    }
    if (lane == 0) { bv[wave] = best; bi[wave] = bidx; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 16; w++)
            if (bv[w] > best || (bv[w] == best && bi[w] < bidx)) { best = bv[w]; bidx = bi[w]; }
        // index 0 wins unless something is strictly greater than x[0]
        float x0 = x[0];
        uint32_t r = (x0 != x0 || !(best > x0)) ? 0u : (uint32_t)bidx;
        *idx = r;
        if (pos) {
            if (history) history[*pos] = r;
            *pos += advance;
        }
    }
}

extern "C" fox_gpu_status fox_gpu_argmax(fox_gpu_ctx *ctx, const float *logits, size_t n,
                                         uint32_t *idx, uint32_t *pos, uint32_t advance,
                                         uint32_t *history)
{
    if (!ctx || !logits || !idx || n == 0 || n > 0x7fffffff)
        return fox_fail(FOX_GPU_ERR_ARG, "argmax: bad argument");
    hipLaunchKernelGGL(argmax_k, dim3(1), dim3(1024), 0, ctx->stream, logits, (int)n, idx, pos,
                       advance, history);
    FOX_LAUNCHED("argmax");
    return FOX_GPU_OK;
}
