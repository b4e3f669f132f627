// fox_fused.hip -- one-launch GEMV stages of a decode layer: the activation
// input stage runs inside the GEMV.
//
// Ternary formats (TQ1_0, TQ2_0; TQ1_0 tensors are held as TQ2_0 blocks of
// the same trits), 1..8 tokens: for one or two tokens every workgroup takes
// the f32 input (optionally RMS-normalised first), quantises it to int8
// exactly as src/gemv.c:11-42 does, and lays it out in LDS as the MFMA B
// operand; the weight loads of its waves are already in flight while it
// does so.  From three tokens on fused_prep does that once per launch (one
// workgroup per token) into workspace memory, and every GEMV workgroup copies
// the result into LDS.  The per-block integer sums, the block-order float
// combine and the final activation-scale multiply are those of gemv_blocks
// (fox_gemv.hip), so results are bit-identical to it and to the reference.
//
// K-quants (Q4_K, Q6_K), one token: the input is quantised per 256-element
// block as src/kernels.c:722-754 does, into LDS in element order with its
// block scales and sub-block sums; each lane of a weight block takes one row
// and one quarter of the block and forms its integer dot products with
// v_dot4_i32_i8 (a token of one column would use 1/16 of an MFMA), then the
// float terms of src/kernels.c:571-661 (8 per block for Q4_K, 4 for Q6_K),
// which the ordered combine adds in the reference's order.  Epilogues:
//   STORE  y (or out + y with FOX_GPU_GEMV_ACCUMULATE: the residual add of
//          src/forward.c:374-377, 393-396);
//   ROPE   segments q, k, v of one projection: RoPE on q and k
//          (src/ops.c:56-73) at position pos[0] + t, q to its buffer, k and
//          v into the layer's caches (src/forward.c:346-362);
//   SILU   segments gate and up, one tile of each per workgroup:
//          h = silu(gate) * up (src/ops.c:41-48);
//   SUMS   per-block integer sums only (fox_gpu_block_sums).
#include "fox_gemv_dev.h"
#include "fox_math.h"

#include <cstring>
#include <type_traits>

#define FW 8                    // waves per workgroup
#define FWG (FW * 64)
// weight blocks in flight per wave, several tokens: one item's units (R4
// blocks, 2 R4 for gate/up pairs), at least 4 and at most 8.  One token
// keeps three (PF_ONE): the loads of every workgroup go out at once, so
// fewer in flight per wave leave the input's loads less traffic to queue
// behind (the 4B layer's four ternary GEMVs 26.3 -> 25.5 us, 14336 x 4096
// 7.2 -> 6.8 us; two, four and six in flight were slower)
#ifndef PF_ONE
#define PF_ONE 3
#endif
__host__ __device__ constexpr int pf_of(int R4, int epi2)
{
    return epi2 * R4 < 4 ? 4 : epi2 * R4 > 8 ? 8 : epi2 * R4;
}
// LDS per workgroup: two workgroups share a compute unit up to two tokens,
// one has it alone from three on (fused_go_r).  The bound is on the dynamic
// carve-up (fused_lds); the kernel's static arrays (reduction slots of up to
// four tokens per wave and the token scales, checked against this figure in
// the kernel) come on top of it.
#define FUSED_STATIC_LDS 512
__host__ __device__ constexpr int fused_lds_max(size_t M)
{
    return (M > 2 ? 160 * 1024 : 96 * 1024) - FUSED_STATIC_LDS;
}

// IN_B: the B operand, block corrections and token scales prepared by
// fused_prep (several tokens, f32 or RMS-normed input), copied into LDS
enum { IN_Q = 0, IN_F32 = 1, IN_NORM = 2, IN_B = 3 };
enum { EPI_STORE = 0, EPI_ROPE = 1, EPI_SILU = 2, EPI_SUMS = 3 };

struct FusedArgs {
    const uint8_t *w[MAX_SEGS];
    float *out[MAX_SEGS];
    int out_stride[MAX_SEGS];
    int n_rows[MAX_SEGS];
    int tile_start[MAX_SEGS + 1];
    int nseg, nb, M, n_work;
    int n_per, n_rem;           // items per workgroup: n_per, plus one below n_rem
    unsigned flags;
    const float *x;
    int x_stride;
    const float *norm_w;
    float eps;
    const int8_t *q_in;
    const float *scale_in;
    int32_t *sums;
    const float *rope_cos, *rope_sin;
    const uint32_t *pos;
    int head_dim, kv_dim, n_ctx;
    int role0;                  // ROPE: the role (0 q, 1 k, 2 v) of segment 0
    int q6_mask;                // FMT_KQMIX: bit s set when segment s is Q6_K (else Q4_K)
    float *k_cache, *v_cache;
};

// LDS carve-up (bytes), identical on host and device.  B: the MFMA B
// operand (ternary formats) or the int8 input in element order (K-quants,
// one token); aux: per-block corrections (ternary) or sub-block sums
// (K-quants: [block][8] for Q4_K, [block][4 quarters][4 groups] for Q6_K);
// bs: the K-quants' per-block activation scales; terms: two buffers of
// [slab][16 rows][token][ntp] float terms, ntp = terms per row (blocks times
// terms per block) padded to a multiple of 4.
struct FusedLds {
    int B, aux, bs, terms, y, total;
};

__host__ __device__ constexpr int fused_ntp(int fmt, int nb)
{
    return (nb * terms_per_block(fmt) + 3) & ~3;
}

__host__ __device__ inline FusedLds fused_lds(int fmt, int K, int M, int nslab)
{
    const int nb = K / 256;
    FusedLds L;
    int off = 0;
    L.B = off;     off += nb * M * (fmt == FMT_TQ2 ? b_bytes_per_block_tok(fmt) : 256);
    L.aux = off;   off += ((nb * M * aux_per_block_tok(fmt) * 4) + 15) & ~15;
    L.bs = off;    off += fmt == FMT_TQ2 ? 0 : ((nb * 4 + 15) & ~15);
    L.terms = off; off += 2 * nslab * 16 * M * fused_ntp(fmt, nb) * 4;
    L.y = off;     off += FWG * 4;
    L.total = off;
    return L;
}

// ------------------------------------------------------------ input stage

__device__ __forceinline__ double wave_sum_dd(double v)
{
    return wave_reduce(v, 0.0, [](double x, double y) { return x + y; });
}

// wave sums of N values at once (the steps of wave_reduce, interleaved);
// every lane receives the sums
template <int N>
__device__ __forceinline__ void wave_sum_n(int (&v)[N])
{
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp_t<0xB1, 0xF>(0, v[i]);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp_t<0x4E, 0xF>(0, v[i]);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp_t<0x141, 0xF>(0, v[i]);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp_t<0x140, 0xF>(0, v[i]);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp_t<0x142, 0xA>(0, v[i]);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += dpp_t<0x143, 0xC>(0, v[i]);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = read_lane(v[i], 63);
}

#define R4_LIMIT 11             // input dwords per thread: K <= 4 * R4_LIMIT * FWG
#define R4_LIMIT_NORM 8         // with the RMSNorm weights also held: K <= 16384

// Where lane dl's int8 dword (block-local elements 4 dl .. 4 dl + 3) goes in
// a block's B operand for one token, as a byte offset from the block's
// token-t base: the TQ2_0 layout of act_prep (fox_gemv.hip), which mirrors
// the A bytes of the block decode.  Elements e0 = 4 dl ..: half (g >> 1),
// level l, offset 16 (g & 1) + 4 u.
__device__ __forceinline__ int b_lane_off(int dl, int M)
{
    const int e0 = 4 * dl;
    const int half = e0 >> 7, l = (e0 >> 5) & 3, o = e0 & 31;
    const int g = 2 * half + (o >> 4), u = (o & 15) >> 2;
    return ((u * 4 + g) * M) * 16 + l * 4;
}

// Token t of the input: optional RMSNorm (src/ops.c:7-22), per-vector int8
// quantisation (src/gemv.c:11-42) and the B operand and per-block
// corrections in LDS, in one pass over the input.  Thread tid owns input
// dwords m = tid + FWG r; dword m lies in block m / 64, so a wave owns the
// 64 dwords of a block and block sums are wave sums.  Returns amax / 127.
// a thread's input dwords of one token, loaded before anything else
template <int R4MAX>
struct InRegs {
    float4 xv[R4MAX], wv[R4MAX];
    uint32_t qd[R4MAX];
};

// (the pointers come in as separate kernel arguments, which the hardware
// loads into scalar registers before the wave starts: the first input loads
// need not wait for a kernel-argument read)
template <int IN, int R4MAX>
__device__ __forceinline__ void load_input(const float *x, const float *norm_w, const int8_t *q_in,
                                           int x_stride, int t, int K, InRegs<R4MAX> &in)
{
    const int tid = threadIdx.x, nd = K >> 2;
    // Every lane loads (past the end it re-reads dword nd - 1; in_mask drops
    // the value at its first use): a load under a condition leaves the
    // compiler unsure how many loads follow this one, and a register
    // overwritten here waits for its load, so either would make the weight
    // blocks issued next wait for the input.
    if (IN == IN_Q) {
        const uint32_t *q4 = (const uint32_t *)(q_in + (size_t)t * K);
#pragma unroll
        for (int r = 0; r < R4MAX; r++) {
            const int m = tid + r * FWG;
            in.qd[r] = q4[m < nd ? m : nd - 1];
        }
        return;
    }
    const float4 *x4 = (const float4 *)(x + (size_t)t * x_stride);
#pragma unroll
    for (int r = 0; r < R4MAX; r++) {
        const int m = tid + r * FWG;
        in.xv[r] = x4[m < nd ? m : nd - 1];
    }
    if (IN == IN_NORM) {
        const float4 *w4 = (const float4 *)norm_w;
#pragma unroll
        for (int r = 0; r < R4MAX; r++) {
            const int m = tid + r * FWG;
            in.wv[r] = w4[m < nd ? m : nd - 1];
        }
    }
}

// zero the input dwords past the end (at their first use; selects on the
// values: a select between two float4 objects would put them in memory)
__device__ __forceinline__ float4 keep4(bool ok, float4 v)
{
    return make_float4(ok ? v.x : 0.0f, ok ? v.y : 0.0f, ok ? v.z : 0.0f, ok ? v.w : 0.0f);
}

template <int IN, int R4MAX>
__device__ __forceinline__ void in_mask(int K, InRegs<R4MAX> &in)
{
    const int tid = threadIdx.x, nd = K >> 2;
#pragma unroll
    for (int r = 0; r < R4MAX; r++) {
        const bool ok = tid + r * FWG < nd;
        if (IN == IN_Q) {
            in.qd[r] = ok ? in.qd[r] : 0u;
        } else {
            in.xv[r] = keep4(ok, in.xv[r]);
            if (IN == IN_NORM) in.wv[r] = keep4(ok, in.wv[r]);
        }
    }
}

// RMSNorm of token t held in the input registers (src/ops.c:7-22)
template <int R4MAX>
__device__ __forceinline__ void rms_apply(const FusedArgs &a, int t, int K, double *dred,
                                          InRegs<R4MAX> &in)
{
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    float4 *xv = in.xv;
    const float4 *wv = in.wv;
    double ss = 0.0;
#pragma unroll
    for (int r = 0; r < R4MAX; r++) {
        const double x0 = xv[r].x, x1 = xv[r].y, x2 = xv[r].z, x3 = xv[r].w;
        ss = __builtin_fma(x0, x0, ss);
        ss = __builtin_fma(x1, x1, ss);
        ss = __builtin_fma(x2, x2, ss);
        ss = __builtin_fma(x3, x3, ss);
    }
    ss = wave_sum_dd(ss);
    if (lane == 0) dred[wave] = ss;
    __syncthreads();
    // Every wave derives the scale itself (no second barrier).  The tree sum
    // certifies the float scale of the reference's index-order double sum
    // (it lies within (K + 64) 2^-52 tot, and the scale is monotone in the
    // sum): even lanes evaluate the low end of that interval, odd lanes the
    // high end; equal floats are the reference's.
    double tot = 0.0;
    for (int w = 0; w < FW; w++) tot += dred[w];
    const double rel = (double)(K + 64) * 0x1p-52;
    const double sgn = (lane & 1) ? 1.0 : -1.0;
    const double y = 1.0 / __builtin_sqrt(tot * (1.0 + sgn * rel) / (double)K +
                                          (double)a.eps) * (1.0 - sgn * 0x1p-50);
    const float f = (float)y;
    float rs = read_lane(f, 0);
    if (rs != read_lane(f, 1)) {
        // undecided: the sequential sum, by every lane (wave-uniform)
        const float *xt = a.x + (size_t)t * a.x_stride;
        double seq = 0.0;
        for (int i = 0; i < K; i++) seq += (double)xt[i] * (double)xt[i];
        rs = (float)(1.0 / __builtin_sqrt(seq / (double)K + (double)a.eps));
    }
#pragma unroll
    for (int r = 0; r < R4MAX; r++) {           // src/ops.c:18: x * scale * w
        xv[r].x = xv[r].x * rs * wv[r].x;
        xv[r].y = xv[r].y * rs * wv[r].y;
        xv[r].z = xv[r].z * rs * wv[r].z;
        xv[r].w = xv[r].w * rs * wv[r].w;
    }
}

template <int FMT, int IN, int R4MAX>
__device__ __forceinline__ float quantise_to_b(const FusedArgs &a, int t, int K, uint8_t *B, int32_t *aux,
                                               double *dred, uint32_t *ured, InRegs<R4MAX> &in)
{
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = a.M, nb = K >> 8;
    in_mask<IN, R4MAX>(K, in);
    uint32_t *qd = in.qd;
    float act = 0.0f;
    if (IN != IN_Q) {
        float4 *xv = in.xv;
        if (IN == IN_NORM) rms_apply<R4MAX>(a, t, K, dred, in);
        // amax (src/gemv.c:20-23) as the largest |x| bit pattern: for x >= 0
        // the integer order is the float order, and NaN lies above inf
        uint32_t mb = 0;
#pragma unroll
        for (int r = 0; r < R4MAX; r++) {
            mb = max(mb, __float_as_uint(xv[r].x) & 0x7fffffffu);
            mb = max(mb, __float_as_uint(xv[r].y) & 0x7fffffffu);
            mb = max(mb, __float_as_uint(xv[r].z) & 0x7fffffffu);
            mb = max(mb, __float_as_uint(xv[r].w) & 0x7fffffffu);
        }
        mb = wave_reduce(mb, 0u, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
        if (lane == 0) ured[wave] = mb;
        __syncthreads();
        uint32_t am = 0;
        for (int w = 0; w < FW; w++) am = max(am, ured[w]);
        if (am >= 0x03800000u && am < 0x7f800000u) {
            // amax in [2^-120, inf), no NaN: quant_fast applies
            const float amax = __uint_as_float(am);
            const float inv = fox_div(127.0f, amax);
#pragma unroll
            for (int r = 0; r < R4MAX; r++)
                qd[r] = pack_lo_bytes(quant_fast(xv[r].x, inv), quant_fast(xv[r].y, inv),
                                      quant_fast(xv[r].z, inv), quant_fast(xv[r].w, inv));
            act = fox_div(amax, 127.0f);
        } else if (am == 0) {
#pragma unroll
            for (int r = 0; r < R4MAX; r++) qd[r] = 0u;
        } else {
            // NaN, inf or a tiny amax (wave-uniform): the float amax of the
            // non-NaN values (src/gemv.c:20-23), then the exact quantiser
            float m = 0.0f;
#pragma unroll
            for (int r = 0; r < R4MAX; r++) {
                const float v4[4] = {xv[r].x, xv[r].y, xv[r].z, xv[r].w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float av = fabsf(v4[e]);
                    if (av > m) m = av;
                }
            }
            m = wave_max(m);
            __syncthreads();
            if (lane == 0) ured[wave] = __float_as_uint(m);
            __syncthreads();
            float amax = 0.0f;
            for (int w = 0; w < FW; w++) amax = max(amax, __uint_as_float(ured[w]));
            if (amax > 0.0f) {
                const float inv = fox_div(127.0f, amax);
#pragma unroll
                for (int r = 0; r < R4MAX; r++)
                    qd[r] = pack_lo_bytes(quant_one(xv[r].x, inv), quant_one(xv[r].y, inv),
                                          quant_one(xv[r].z, inv), quant_one(xv[r].w, inv));
                act = fox_div(amax, 127.0f);
            } else {
#pragma unroll
                for (int r = 0; r < R4MAX; r++) qd[r] = 0u;
            }
        }
    }
    // B operand and per-block corrections (-(block sum)); a wave's 64 lanes
    // are one block.  The block sums of all the wave's blocks reduce
    // together, their steps interleaved.
    const int boff = b_lane_off(lane, M);
    const int bbytes = b_bytes_per_block_tok(FMT) * M;
    int part[R4MAX];
#pragma unroll
    for (int r = 0; r < R4MAX; r++) {
        const int b = wave + FW * r;
        if (b < nb) *(uint32_t *)(B + b * bbytes + t * 16 + boff) = qd[r];   // (uniform)
        part[r] = __builtin_amdgcn_sdot4((int)qd[r], 0x01010101, 0, false);
    }
    wave_sum_n<R4MAX>(part);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R4MAX; r++) {
            const int b = wave + FW * r;
            if (b >= nb) break;
            aux[b * M + t] = -part[r];
        }
    }
    if (IN == IN_Q) act = a.scale_in ? a.scale_in[t] : 0.0f;   // block sums come without a scale
    __syncthreads();
    return act;
}

// N wave maxima at once (the steps of wave_reduce, interleaved); every lane
// receives them
template <int N>
__device__ __forceinline__ void wave_max_n(uint32_t (&v)[N])
{
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = max(v[i], dpp_t<0xB1, 0xF>(0u, v[i]));
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = max(v[i], dpp_t<0x4E, 0xF>(0u, v[i]));
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = max(v[i], dpp_t<0x141, 0xF>(0u, v[i]));
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = max(v[i], dpp_t<0x140, 0xF>(0u, v[i]));
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = max(v[i], dpp_t<0x142, 0xA>(0u, v[i]));
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = max(v[i], dpp_t<0x143, 0xC>(0u, v[i]));
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = read_lane(v[i], 63);
}

// ---- several tokens (the ternary formats, M > 1): tokens in groups of
// TG, a group's tokens loaded together and taken through each step of
// quantise_to_b side by side, so that a group costs the barriers of one
// token (three) instead of three per token.  TG keeps a group's input
// registers at 16 float4 per thread.
__host__ __device__ constexpr int tg_of(int R4)
{
    return R4 <= 2 ? 2 : 1;
}

// from three tokens on a workgroup has its compute unit alone (two waves per
// SIMD), so a group may hold more tokens, loaded once per group instead of
// double-buffered: up to four tokens, 8 float4 of input per thread (16, up
// to eight tokens, spilled in the norm-input kernels and ran slower at three
// and four tokens)
__host__ __device__ constexpr int tg_big(int R4)
{
    return 8 / R4 > 4 ? 4 : 8 / R4 < 1 ? 1 : 8 / R4;
}

template <int R4MAX, int TG>
struct InGrp {
    float4 xv[TG][R4MAX];
    float4 wv[R4MAX];                      // the RMSNorm weights (one copy for all tokens)
    uint32_t qd[TG][R4MAX];
};

// the dwords of tokens t0 .. t0 + nt - 1 (nt <= TG; the rows past the
// group's last token re-read it, so that the count of loads is fixed), and
// with wv the norm weights
template <int IN, int R4MAX, int TG>
__device__ __forceinline__ void load_group(const float *x, const float *norm_w, const int8_t *q_in,
                                           int x_stride, int t0, int nt, int K, bool wv,
                                           InGrp<R4MAX, TG> &g)
{
    const int tid = threadIdx.x, nd = K >> 2;
#pragma unroll
    for (int j = 0; j < TG; j++) {
        const int t = t0 + (j < nt ? j : nt - 1);
        if (IN == IN_Q) {
            const uint32_t *q4 = (const uint32_t *)(q_in + (size_t)t * K);
#pragma unroll
            for (int r = 0; r < R4MAX; r++) {
                const int m = tid + r * FWG;
                g.qd[j][r] = q4[m < nd ? m : nd - 1];
            }
        } else {
            const float4 *x4 = (const float4 *)(x + (size_t)t * x_stride);
#pragma unroll
            for (int r = 0; r < R4MAX; r++) {
                const int m = tid + r * FWG;
                g.xv[j][r] = x4[m < nd ? m : nd - 1];
            }
        }
    }
    if (IN == IN_NORM && wv) {
        const float4 *w4 = (const float4 *)norm_w;
#pragma unroll
        for (int r = 0; r < R4MAX; r++) {
            const int m = tid + r * FWG;
            g.wv[r] = w4[m < nd ? m : nd - 1];
        }
    }
}

// quantise_to_b for the group's tokens: the same operations per token, in
// the same order (RMSNorm with the certified scale, amax, quantiser, B
// operand, block corrections); dred and ured hold TG x FW partials.  Writes
// ascale[t] and ends with a barrier.
template <int FMT, int IN, int R4MAX, int TG>
__device__ __forceinline__ void quantise_group(const FusedArgs &a, int t0, int nt, int K,
                                               uint8_t *B, int32_t *aux, double *dred,
                                               uint32_t *ured, float *ascale,
                                               InGrp<R4MAX, TG> &g)
{
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = a.M, nb = K >> 8, nd = K >> 2;
#pragma unroll
    for (int r = 0; r < R4MAX; r++) {
        const bool ok = tid + r * FWG < nd;
#pragma unroll
        for (int j = 0; j < TG; j++) {
            if (IN == IN_Q) g.qd[j][r] = ok ? g.qd[j][r] : 0u;
            else g.xv[j][r] = keep4(ok, g.xv[j][r]);
        }
        if (IN == IN_NORM) g.wv[r] = keep4(ok, g.wv[r]);
    }
    float act[TG];
#pragma unroll
    for (int j = 0; j < TG; j++) act[j] = 0.0f;
    if (IN == IN_NORM) {
        // rms_apply per token, the partial sums of all tokens through one barrier
        double ss[TG];
#pragma unroll
        for (int j = 0; j < TG; j++) {
            ss[j] = 0.0;
#pragma unroll
            for (int r = 0; r < R4MAX; r++) {
                const double x0 = g.xv[j][r].x, x1 = g.xv[j][r].y;
                const double x2 = g.xv[j][r].z, x3 = g.xv[j][r].w;
                ss[j] = __builtin_fma(x0, x0, ss[j]);
                ss[j] = __builtin_fma(x1, x1, ss[j]);
                ss[j] = __builtin_fma(x2, x2, ss[j]);
                ss[j] = __builtin_fma(x3, x3, ss[j]);
            }
        }
#pragma unroll
        for (int j = 0; j < TG; j++) ss[j] = wave_sum_dd(ss[j]);
        if (lane == 0) {
#pragma unroll
            for (int j = 0; j < TG; j++) dred[j * FW + wave] = ss[j];
        }
        __syncthreads();
        const double rel = (double)(K + 64) * 0x1p-52;
        const double sgn = (lane & 1) ? 1.0 : -1.0;
#pragma unroll
        for (int j = 0; j < TG; j++) {
            if (j >= nt) break;                                   // (uniform)
            double tot = 0.0;
            for (int w = 0; w < FW; w++) tot += dred[j * FW + w];
            const double y = 1.0 / __builtin_sqrt(tot * (1.0 + sgn * rel) / (double)K +
                                                  (double)a.eps) * (1.0 - sgn * 0x1p-50);
            const float f = (float)y;
            float rs = read_lane(f, 0);
            if (rs != read_lane(f, 1)) {
                const float *xt = a.x + (size_t)(t0 + j) * a.x_stride;
                double seq = 0.0;
                for (int i = 0; i < K; i++) seq += (double)xt[i] * (double)xt[i];
                rs = (float)(1.0 / __builtin_sqrt(seq / (double)K + (double)a.eps));
            }
#pragma unroll
            for (int r = 0; r < R4MAX; r++) {
                g.xv[j][r].x = g.xv[j][r].x * rs * g.wv[r].x;
                g.xv[j][r].y = g.xv[j][r].y * rs * g.wv[r].y;
                g.xv[j][r].z = g.xv[j][r].z * rs * g.wv[r].z;
                g.xv[j][r].w = g.xv[j][r].w * rs * g.wv[r].w;
            }
        }
    }
    if (IN != IN_Q) {
        // amax per token as the largest |x| bit pattern, all tokens' wave
        // maxima together
        uint32_t mb[TG];
#pragma unroll
        for (int j = 0; j < TG; j++) {
            uint32_t m = 0;
#pragma unroll
            for (int r = 0; r < R4MAX; r++) {
                m = max(m, __float_as_uint(g.xv[j][r].x) & 0x7fffffffu);
                m = max(m, __float_as_uint(g.xv[j][r].y) & 0x7fffffffu);
                m = max(m, __float_as_uint(g.xv[j][r].z) & 0x7fffffffu);
                m = max(m, __float_as_uint(g.xv[j][r].w) & 0x7fffffffu);
            }
            mb[j] = m;
        }
        wave_max_n<TG>(mb);
        if (lane == 0) {
#pragma unroll
            for (int j = 0; j < TG; j++) ured[j * FW + wave] = mb[j];
        }
        __syncthreads();
        uint32_t am[TG];
#pragma unroll
        for (int j = 0; j < TG; j++) {
            am[j] = 0;
            for (int w = 0; w < FW; w++) am[j] = max(am[j], ured[j * FW + w]);
        }
#pragma unroll
        for (int j = 0; j < TG; j++) {
            if (j >= nt) break;                                   // (uniform)
            if (am[j] >= 0x03800000u && am[j] < 0x7f800000u) {
                const float amax = __uint_as_float(am[j]);
                const float inv = fox_div(127.0f, amax);
#pragma unroll
                for (int r = 0; r < R4MAX; r++)
                    g.qd[j][r] = pack_lo_bytes(quant_fast(g.xv[j][r].x, inv),
                                               quant_fast(g.xv[j][r].y, inv),
                                               quant_fast(g.xv[j][r].z, inv),
                                               quant_fast(g.xv[j][r].w, inv));
                act[j] = fox_div(amax, 127.0f);
            } else if (am[j] == 0) {
#pragma unroll
                for (int r = 0; r < R4MAX; r++) g.qd[j][r] = 0u;
            } else {
                // NaN, inf or a tiny amax (uniform): the float amax of the
                // non-NaN values, then the exact quantiser.  (Every thread
                // has read all of the group's maxima before the first
                // barrier here, so the slot can be reused.)
                float m = 0.0f;
#pragma unroll
                for (int r = 0; r < R4MAX; r++) {
                    const float v4[4] = {g.xv[j][r].x, g.xv[j][r].y, g.xv[j][r].z, g.xv[j][r].w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float av = fabsf(v4[e]);
                        if (av > m) m = av;
                    }
                }
                m = wave_max(m);
                __syncthreads();
                if (lane == 0) ured[j * FW + wave] = __float_as_uint(m);
                __syncthreads();
                float amax = 0.0f;
                for (int w = 0; w < FW; w++) amax = max(amax, __uint_as_float(ured[j * FW + w]));
                if (amax > 0.0f) {
                    const float inv = fox_div(127.0f, amax);
#pragma unroll
                    for (int r = 0; r < R4MAX; r++)
                        g.qd[j][r] = pack_lo_bytes(quant_one(g.xv[j][r].x, inv),
                                                   quant_one(g.xv[j][r].y, inv),
                                                   quant_one(g.xv[j][r].z, inv),
                                                   quant_one(g.xv[j][r].w, inv));
                    act[j] = fox_div(amax, 127.0f);
                } else {
#pragma unroll
                    for (int r = 0; r < R4MAX; r++) g.qd[j][r] = 0u;
                }
            }
        }
    }
    // B operand and the per-block corrections of all the group's tokens
    const int boff = b_lane_off(lane, M);
    const int bbytes = b_bytes_per_block_tok(FMT) * M;
    int part[TG * R4MAX];
#pragma unroll
    for (int j = 0; j < TG; j++) {
#pragma unroll
        for (int r = 0; r < R4MAX; r++) {
            const int b = wave + FW * r;
            if (j < nt && b < nb)                                  // (uniform)
                *(uint32_t *)(B + b * bbytes + (t0 + j) * 16 + boff) = g.qd[j][r];
            part[j * R4MAX + r] = __builtin_amdgcn_sdot4((int)g.qd[j][r], 0x01010101, 0, false);
        }
    }
    wave_sum_n<TG * R4MAX>(part);
    if (lane == 0) {
#pragma unroll
        for (int j = 0; j < TG; j++) {
            if (j >= nt) break;
#pragma unroll
            for (int r = 0; r < R4MAX; r++) {
                const int b = wave + FW * r;
                if (b >= nb) break;
                aux[b * M + t0 + j] = -part[j * R4MAX + r];
            }
        }
    }
    if (tid == 0) {
#pragma unroll
        for (int j = 0; j < TG; j++) {
            if (j >= nt) break;
            ascale[t0 + j] = IN == IN_Q ? (a.scale_in ? a.scale_in[t0 + j] : 0.0f) : act[j];
        }
    }
    __syncthreads();
}

// K-quant input stage, one token: RMSNorm (IN_NORM), then every 256-element
// block quantised with its own scale (src/kernels.c:722-754) into xq in
// element order, its scale into bs and the sums of its sub-blocks (32
// elements for Q4_K, 16 for Q6_K) into aux.  Thread tid holds input dwords
// m = tid + FWG r, so wave w holds blocks w + FW r and a block's amax is one
// wave maximum; the amaxes of all the wave's blocks reduce together.
template <int FMT, int IN, int R4MAX>
__device__ __forceinline__ void quantise_kq(const FusedArgs &a, int K, int8_t *xq, int32_t *aux,
                                            float *bs, double *dred, InRegs<R4MAX> &in)
{
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb = K >> 8;
    in_mask<IN, R4MAX>(K, in);
    float4 *xv = in.xv;
    if (IN == IN_NORM) rms_apply<R4MAX>(a, 0, K, dred, in);
    // per-block amax as the largest |x| bit pattern (for x >= 0 the integer
    // order is the float order, and NaN lies above inf)
    uint32_t mb[R4MAX];
#pragma unroll
    for (int r = 0; r < R4MAX; r++) {
        uint32_t m = __float_as_uint(xv[r].x) & 0x7fffffffu;
        m = max(m, __float_as_uint(xv[r].y) & 0x7fffffffu);
        m = max(m, __float_as_uint(xv[r].z) & 0x7fffffffu);
        m = max(m, __float_as_uint(xv[r].w) & 0x7fffffffu);
        mb[r] = m;
    }
    wave_max_n<R4MAX>(mb);
    // the blocks' 127/amax and amax/127 in one double division: lane r
    // (r < R4MAX) divides for block r, lane 32 + r the other way (the same
    // operations as per block; a double division is a long dependent
    // sequence at the FP64 rate, two per block otherwise)
    static_assert(R4MAX <= 32, "one lane per block in each half of the wave");
    float dq;
    {
        uint32_t amr = mb[0];
#pragma unroll
        for (int r = 1; r < R4MAX; r++) amr = (lane & 31) == r ? mb[r] : amr;
        const float amx = __uint_as_float(amr);
        dq = lane < 32 ? fox_div(127.0f, amx) : fox_div(amx, 127.0f);
    }
    int part[R4MAX];
#pragma unroll
    for (int r = 0; r < R4MAX; r++) {
        const int b = wave + FW * r;
        const uint32_t am = mb[r];
        uint32_t q = 0u;
        float s = 0.0f;
        if (am >= 0x03800000u && am < 0x7f800000u) {           // (uniform)
            // amax in [2^-120, inf), no NaN: quant_fast applies
            const float inv = read_lane(dq, r);                 // 127 / amax
            q = pack_lo_bytes(quant_fast(xv[r].x, inv), quant_fast(xv[r].y, inv),
                              quant_fast(xv[r].z, inv), quant_fast(xv[r].w, inv));
            s = read_lane(dq, 32 + r);                          // amax / 127
        } else if (am != 0u) {
            // NaN, inf or a tiny amax: the float amax of the non-NaN values
            // (src/kernels.c:734-737), then the exact quantiser
            const float v4[4] = {xv[r].x, xv[r].y, xv[r].z, xv[r].w};
            float m = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float av = fabsf(v4[e]);
                if (av > m) m = av;
            }
            m = wave_max(m);
            if (m > 0.0f) {
                const float inv = fox_div(127.0f, m);
                q = pack_lo_bytes(quant_one(v4[0], inv), quant_one(v4[1], inv),
                                  quant_one(v4[2], inv), quant_one(v4[3], inv));
                s = fox_div(m, 127.0f);
            }
        }
        if (b < nb) {                                           // (uniform)
            *(uint32_t *)(xq + b * 256 + 4 * lane) = q;
            if (lane == 0) bs[b] = s;
        }
        part[r] = __builtin_amdgcn_sdot4((int)q, 0x01010101, 0, false);
    }
    // sub-block sums: quads of lanes (16 elements), then eights (32)
#pragma unroll
    for (int r = 0; r < R4MAX; r++) part[r] += dpp_t<0xB1, 0xF>(0, part[r]);
#pragma unroll
    for (int r = 0; r < R4MAX; r++) part[r] += dpp_t<0x4E, 0xF>(0, part[r]);
    // (both formats: the sixteen-element sums first, at aux + 8 nb, then
    // their pairs)
    constexpr bool S16 = FMT == FMT_Q6K || FMT == FMT_KQMIX;
    constexpr bool S32 = FMT == FMT_Q4K || FMT == FMT_KQMIX;
    if constexpr (S16) {
        int32_t *a16 = aux + (FMT == FMT_KQMIX ? 8 * nb : 0);
#pragma unroll
        for (int r = 0; r < R4MAX; r++) {
            const int b = wave + FW * r;
            if (b >= nb) break;                                 // (uniform)
            if ((lane & 3) == 0) {
                // lane l holds elements 4l ..: half h = l >> 5, group g =
                // (l >> 3) & 3, sixteen s = (l >> 2) & 1; stored at
                // [block][quarter 2h + s][group g]
                const int h = lane >> 5, g = (lane >> 3) & 3, s = (lane >> 2) & 1;
                a16[b * 16 + (2 * h + s) * 4 + g] = part[r];
            }
        }
    }
    if constexpr (S32) {
#pragma unroll
        for (int r = 0; r < R4MAX; r++) part[r] += dpp_t<0x141, 0xF>(0, part[r]);
#pragma unroll
        for (int r = 0; r < R4MAX; r++) {
            const int b = wave + FW * r;
            if (b >= nb) break;                                 // (uniform)
            if ((lane & 7) == 0) aux[b * 8 + (lane >> 3)] = part[r];
        }
    }
    __syncthreads();
}

// ------------------------------------------------------------ weights

// one lane's bytes of one (tile, block) chunk
template <int FMT>
struct RawBlk {
    uint32_t d0, d1, d2, d3;   // the lane's 16 bytes of 2-bit codes
    uint2 dd;                  // f16 scales of rows 4g .. 4g+3
};

// Q4_K lane (row r = lane & 15, part p = lane >> 4): qs[32p .. 32p + 31] of
// its row (eight bytes from each of the lanes r + 16 g of the chunk layout)
// and the row's d, dmin and 12 scale bytes
template <>
struct RawBlk<FMT_Q4K> {
    uint2 q0, q1, q2, q3;
    uint4 hd;
};

// Q6_K lane (row r = lane & 15, quarter v = lane >> 4 = 2 h + s): the
// row's ql[64h + 16s ..] and ql[64h + 32 + 16s ..] (16 bytes each),
// qh[32h + 16s ..] (16), scales 8h .. 8h + 7 and d
template <>
struct RawBlk<FMT_Q6K> {
    uint4 l0, l1, h;
    uint2 sc;
    uint32_t d;
};

// either K-quant's lane bytes (FMT_KQMIX: the format is the segment's):
// Q6_K's l0, l1, h, sc, d as a, b, c, sc, d; Q4_K's q0 .. q3 in a and b and
// its hd in c
template <>
struct RawBlk<FMT_KQMIX> {
    uint4 a, b, c;
    uint2 sc;
    uint32_t d;
};

__device__ __forceinline__ RawBlk<FMT_Q4K> q4k_view(const RawBlk<FMT_KQMIX> &m)
{
    RawBlk<FMT_Q4K> r;
    r.q0 = make_uint2(m.a.x, m.a.y);
    r.q1 = make_uint2(m.a.z, m.a.w);
    r.q2 = make_uint2(m.b.x, m.b.y);
    r.q3 = make_uint2(m.b.z, m.b.w);
    r.hd = m.c;
    return r;
}

__device__ __forceinline__ RawBlk<FMT_Q6K> q6k_view(const RawBlk<FMT_KQMIX> &m)
{
    RawBlk<FMT_Q6K> r;
    r.l0 = m.a;
    r.l1 = m.b;
    r.h = m.c;
    r.sc = m.sc;
    r.d = m.d;
    return r;
}

template <int FMT>
__device__ __forceinline__ RawBlk<FMT> load_raw(const uint8_t *__restrict__ ch, int lane);

// a chunk of either K-quant (q6: the segment is Q6_K)
__device__ __forceinline__ RawBlk<FMT_KQMIX> load_raw_mix(const uint8_t *__restrict__ ch,
                                                         int lane, bool q6);

template <int FMT>
__device__ __forceinline__ RawBlk<FMT> load_raw(const uint8_t *__restrict__ ch, int lane)
{
    RawBlk<FMT> r;
    if constexpr (FMT == FMT_TQ2) {
        const int g = lane >> 4;
        const uint4 v = *(const uint4 *)(ch + 16 * lane);
        r.d0 = v.x;
        r.d1 = v.y;
        r.d2 = v.z;
        r.d3 = v.w;
        r.dd = *(const uint2 *)(ch + 1024 + 8 * g);
    } else if constexpr (FMT == FMT_Q4K) {
        const int row = lane & 15, p = lane >> 4;
        const uint8_t *q = ch + 32 * row + 8 * p;   // lane r + 16 g: + 512 g
        r.q0 = *(const uint2 *)q;
        r.q1 = *(const uint2 *)(q + 512);
        r.q2 = *(const uint2 *)(q + 1024);
        r.q3 = *(const uint2 *)(q + 1536);
        r.hd = *(const uint4 *)(ch + 2048 + 16 * row);
    } else {
        const int row = lane & 15, h = lane >> 5, s = (lane >> 4) & 1;
        const uint8_t *ql = ch + 128 * row + 64 * h + 16 * s;
        r.l0 = *(const uint4 *)ql;
        r.l1 = *(const uint4 *)(ql + 32);
        r.h = *(const uint4 *)(ch + 2048 + 64 * row + 32 * h + 16 * s);
        r.sc = *(const uint2 *)(ch + 3072 + 16 * row + 8 * h);
        r.d = *(const unsigned short *)(ch + 3328 + 2 * row);
    }
    return r;
}

// The same seven loads for either format, only their addresses chosen by
// the format: with a branch around the loads, the two paths leave different
// numbers of loads in flight, and where they join the compiler waits for
// every load (the blocks in flight included) on each unit.  A Q4_K chunk
// reads its sc and d slots from the chunk's first bytes (unused).
__device__ __forceinline__ RawBlk<FMT_KQMIX> load_raw_mix(const uint8_t *__restrict__ ch,
                                                         int lane, bool q6)
{
    const int row = lane & 15, h = lane >> 5, s = (lane >> 4) & 1;
    const int l6 = 128 * row + 64 * h + 16 * s;                 // Q6_K ql (as load_raw)
    const int q4 = 32 * row + 8 * (lane >> 4);                  // Q4_K qs (as load_raw)
    const int o0 = q6 ? l6 : q4, o1 = q6 ? l6 + 8 : q4 + 512;
    const int o2 = q6 ? l6 + 32 : q4 + 1024, o3 = q6 ? l6 + 40 : q4 + 1536;
    const int oc = 2048 + (q6 ? 64 * row + 32 * h + 16 * s : 16 * row);
    const int os = q6 ? 3072 + 16 * row + 8 * h : 0;
    const int od = q6 ? 3328 + 2 * row : 0;
    const uint2 v0 = *(const uint2 *)(ch + o0), v1 = *(const uint2 *)(ch + o1);
    const uint2 v2 = *(const uint2 *)(ch + o2), v3 = *(const uint2 *)(ch + o3);
    RawBlk<FMT_KQMIX> m;
    m.a = make_uint4(v0.x, v0.y, v1.x, v1.y);
    m.b = make_uint4(v2.x, v2.y, v3.x, v3.y);
    m.c = *(const uint4 *)(ch + oc);
    m.sc = *(const uint2 *)(ch + os);
    m.d = *(const unsigned short *)(ch + od);
    return m;
}

// Q4_K terms of sub-blocks 2p and 2p + 1 of one block and row
// (src/kernels.c:585-599): xb the block's int8 input, sx its sub-block sums,
// as its activation scale
__device__ __forceinline__ void q4k_terms(const RawBlk<FMT_Q4K> &w, const int8_t *xb,
                                          const int32_t *sx, float as, int p, float &t0,
                                          float &t1)
{
    const uint4 *x4 = (const uint4 *)(xb + 64 * p);
    const uint4 xa = x4[0], xb1 = x4[1], xc = x4[2], xd = x4[3];
    // dword k of the lane holds qs[32p + 4k ..]: low nibbles with inputs
    // 64p + 4k .., high nibbles with 64p + 32 + 4k ..
    const uint32_t q[8] = {w.q0.x, w.q0.y, w.q1.x, w.q1.y, w.q2.x, w.q2.y, w.q3.x, w.q3.y};
    const uint32_t xl[8] = {xa.x, xa.y, xa.z, xa.w, xb1.x, xb1.y, xb1.z, xb1.w};
    const uint32_t xh[8] = {xc.x, xc.y, xc.z, xc.w, xd.x, xd.y, xd.z, xd.w};
    int D0 = 0, D1 = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        D0 = __builtin_amdgcn_sdot4((int)(q[k] & 0x0F0F0F0Fu), (int)xl[k], D0, false);
        D1 = __builtin_amdgcn_sdot4((int)((q[k] >> 4) & 0x0F0F0F0Fu), (int)xh[k], D1, false);
    }
    const int2 sq = *(const int2 *)(sx + 2 * p);
    const float d = half_bits_to_float(w.hd.x & 0xFFFFu);
    const float dmin = half_bits_to_float(w.hd.x >> 16);
    // scale and min of sub-blocks j = 2p, 2p + 1 (src/kernels.c:246-255):
    // bytes (j & 3) of the three scale dwords
    const int sh = 16 * (p & 1);
    const uint32_t S0 = w.hd.y >> sh, S1 = w.hd.z >> sh, S2 = w.hd.w >> sh;
    int sc0, mn0, sc1, mn1;
    if (p < 2) {
        sc0 = S0 & 63;
        mn0 = S1 & 63;
        sc1 = (S0 >> 8) & 63;
        mn1 = (S1 >> 8) & 63;
    } else {
        sc0 = (S2 & 0x0F) | (((S0 >> 6) & 3) << 4);
        mn0 = ((S2 >> 4) & 0x0F) | (((S1 >> 6) & 3) << 4);
        sc1 = ((S2 >> 8) & 0x0F) | (((S0 >> 14) & 3) << 4);
        mn1 = ((S2 >> 12) & 0x0F) | (((S1 >> 14) & 3) << 4);
    }
    t0 = as * (d * (float)sc0 * (float)D0 - dmin * (float)mn0 * (float)sq.x);
    t1 = as * (d * (float)sc1 * (float)D1 - dmin * (float)mn1 * (float)sq.y);
}

// Q6_K term of quarter v = 2h + s of one block and row: the group dot of
// src/kernels.c:531-569 (sub = s of half h), scaled as src/kernels.c:655-657
__device__ __forceinline__ float q6k_term(const RawBlk<FMT_Q6K> &w, const int8_t *xb,
                                          const int32_t *sx, float as, int lane)
{
    const int h = lane >> 5, s = (lane >> 4) & 1;
    const int8_t *xs = xb + 128 * h + 16 * s;
    const int4 sg = *(const int4 *)(sx + 4 * (lane >> 4));
    const int sgv[4] = {sg.x, sg.y, sg.z, sg.w};
    const uint32_t L0[4] = {w.l0.x, w.l0.y, w.l0.z, w.l0.w};
    const uint32_t L1[4] = {w.l1.x, w.l1.y, w.l1.z, w.l1.w};
    const uint32_t H[4] = {w.h.x, w.h.y, w.h.z, w.h.w};
    int part = 0;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        // group g: inputs 128h + 32g + 16s .., weights (ql low / high nibble
        // of the first or second 32 bytes) | (qh bits 2g, 2g + 1) << 4
        const uint4 x4 = *(const uint4 *)(xs + 32 * g);
        const uint32_t xw[4] = {x4.x, x4.y, x4.z, x4.w};
        int dot = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t src = (g & 1) ? L1[k] : L0[k];
            const uint32_t q6 = ((src >> (4 * (g >> 1))) & 0x0F0F0F0Fu) |
                                (((H[k] >> (2 * g)) & 0x03030303u) << 4);
            dot = __builtin_amdgcn_sdot4((int)q6, (int)xw[k], dot, false);
        }
        // scale byte s + 2g of the row's scales 8h ..
        const int sc = __builtin_amdgcn_sbfe((int)(g < 2 ? w.sc.x : w.sc.y), 8 * (s + 2 * (g & 1)), 8);
        part += sc * (dot - 32 * sgv[g]);
    }
    const float d = half_bits_to_float(w.d & 0xFFFFu);
    return as * d * (float)part;
}

// integer block sums of rows 4g .. 4g+3 for the lane's B column; returns
// S in acc[r] for lanes with j < M (each 2-bit code is one A byte; corr
// carries the -1 of every code).  Lanes past the M tokens read the last
// token's column (their MFMA columns are not used): with no lane-dependent
// branch the four B reads issue together.
template <int FMT>
__device__ __forceinline__ void block_mfma(const RawBlk<FMT> &r, const uint8_t *__restrict__ Bb,
                                           int M, int lane, int corr, int S[4])
{
    const int g = lane >> 4, j = lane & 15, jc = j < M ? j : M - 1;
    v4i bv[4];
#pragma unroll
    for (int u = 0; u < 4; u++) bv[u] = *(const v4i *)(Bb + (((u * 4 + g) * M) + jc) * 16);
    v4i acc = {0, 0, 0, 0};
    const uint32_t dw[4] = {r.d0, r.d1, r.d2, r.d3};
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const uint32_t d = dw[u];
        acc = mfma(d & 0x03030303u, (d >> 2) & 0x03030303u, (d >> 4) & 0x03030303u,
                   (d >> 6) & 0x03030303u, bv[u], acc);
    }
#pragma unroll
    for (int q = 0; q < 4; q++) S[q] = acc[q] + corr;
}

// One token, the MFMA transposed: the activations as the A operand (every
// A row the token's, read from the same B-operand bytes) and the codes as
// the B operand (column n = row n of the tile, the lane layout of the codes
// is the same), so lane l receives row l % 16's integer sum in every
// element of acc, and lanes 0-15 form one float term each instead of four
// lanes four terms.  The chunk's codes as load_raw, and the f16 scale of the
// lane's row l % 16.
__device__ __forceinline__ RawBlk<FMT_TQ2> load_raw_t1(const uint8_t *__restrict__ ch, int lane)
{
    RawBlk<FMT_TQ2> r;
    const uint4 v = *(const uint4 *)(ch + 16 * lane);
    r.d0 = v.x;
    r.d1 = v.y;
    r.d2 = v.z;
    r.d3 = v.w;
    r.dd = make_uint2(*(const unsigned short *)(ch + 1024 + 2 * (lane & 15)), 0u);
    return r;
}

__device__ __forceinline__ int block_mfma_t1(const RawBlk<FMT_TQ2> &r,
                                             const uint8_t *__restrict__ Bb, int lane, int corr)
{
    const int g = lane >> 4;
    v4i bv[4];
#pragma unroll
    for (int u = 0; u < 4; u++) bv[u] = *(const v4i *)(Bb + (u * 4 + g) * 16);
    v4i acc = {0, 0, 0, 0};
    const uint32_t dw[4] = {r.d0, r.d1, r.d2, r.d3};
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const uint32_t d = dw[u];
        const v4i w = {(int)(d & 0x03030303u), (int)((d >> 2) & 0x03030303u),
                       (int)((d >> 4) & 0x03030303u), (int)((d >> 6) & 0x03030303u)};
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(bv[u], w, acc, 0, 0, 0);
    }
    return acc[0] + corr;
}

// ------------------------------------------------------------ kernel

// a wave-uniform value pinned in scalar registers: the compiler may no longer
// re-derive it from memory (pointers stay global-memory pointers, so that
// loads through them remain global loads)
template <typename T>
__device__ __forceinline__ T in_sgpr(T v)
{
    asm volatile("" : "+s"(v));
    return v;
}

template <typename T>
__device__ __forceinline__ T *in_sgpr(T *p)
{
    auto g = (__attribute__((address_space(1))) T *)p;
    asm volatile("" : "+s"(g));
    return (T *)g;
}

// v[s] of a kernel-argument array: flat selects (a nested choice becomes
// branches) among values pinned in registers (a select among the loads
// themselves compiles to a load at a computed offset followed by a wait, at
// every use: once per weight block)
template <typename T>
__device__ __forceinline__ T pick4(const T *v, int s)
{
    const T v0 = in_sgpr(v[0]), v1 = in_sgpr(v[1]), v2 = in_sgpr(v[2]), v3 = in_sgpr(v[3]);
    T r = v0;
    r = s >= 1 ? v1 : r;
    r = s >= 2 ? v2 : r;
    r = s >= 3 ? v3 : r;
    return r;
}

// MT: 0 one token; 1 two tokens (input in pairs, the next pair in flight);
// 2 three or more (one workgroup per compute unit, larger groups).  Separate
// instantiations keep the one-token kernels' registers as they are.
template <int FMT, int IN, int EPI, int R4, int MT>
__global__ __launch_bounds__(FWG) void gemv_fused(const float *x_in, const float *norm_in,
                                                 const int8_t *q_in, int nb_in, FusedArgs a)
{
    extern __shared__ uint4 fused_lds4[];
    uint8_t *lds = (uint8_t *)fused_lds4;
    constexpr bool KQ = FMT != FMT_TQ2;                    // a K-quant (one token)
    constexpr int TG = KQ ? 1 : MT == 2 ? tg_big(R4) : MT == 1 ? tg_of(R4) : 1;   // tokens per input group
    __shared__ double dred[FW * TG];
    __shared__ uint32_t ured[FW * TG];
    __shared__ float ascale[FOX_GPU_MAX_TOKENS];
    static_assert(sizeof(dred) + sizeof(ured) + sizeof(ascale) <= FUSED_STATIC_LDS,
                  "static LDS beyond the bound fused_lds_max leaves for it");

    constexpr int CHUNK = FMT == FMT_TQ2 ? TQ2_CHUNK : FMT == FMT_Q4K ? Q4K_CHUNK : Q6K_CHUNK;
    // the K-quant of segment sg (FMT_KQMIX: per segment) and its chunk bytes
    auto seg_q6 = [&](int sg) -> bool {
        return FMT == FMT_Q6K || (FMT == FMT_KQMIX && ((a.q6_mask >> sg) & 1));
    };
    auto chunk_of = [&](int sg) -> int {
        return FMT == FMT_KQMIX ? (seg_q6(sg) ? Q6K_CHUNK : Q4K_CHUNK) : CHUNK;
    };
    constexpr int T = terms_per_block(FMT);
    // (the wave index as a wave-uniform value: everything per wave below,
    // the units, items and weight addresses, is then scalar work)
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb = nb_in, M = MT && !KQ ? a.M : 1, K = nb * 256;
    constexpr int nslab = EPI == EPI_SILU ? 2 : 1;
    const FusedLds L = fused_lds(FMT, K, M, nslab);
    uint8_t *B = lds + L.B;
    int32_t *aux = (int32_t *)(lds + L.aux);
    float *bsc = (float *)(lds + L.bs);
    // block terms [2][nslab][16 rows][M][nbp]: a row's terms (T per block)
    // are contiguous, padded with zeros to nbp, a multiple of 4 (adding
    // +0.0f changes no sum: the ordered sum starts at +0.0f and so is never
    // -0.0f)
    float *terms = (float *)(lds + L.terms);
    float *ybuf = (float *)(lds + L.y);
    const int nbp = fused_ntp(FMT, nb);
    const int nbp6 = FMT == FMT_KQMIX ? fused_ntp(FMT_Q6K, nb) : nbp;   // (Q6_K segments' rows)
    const int tstride = nslab * 16 * M * nbp;              // floats per terms buffer

    // ---- work: items bx, bx + gridDim.x, ... (a 16-row tile of one segment,
    // or with SILU a tile of gate and the same tile of up).  Arguments are
    // read with constant indices only, so that they arrive in one batch of
    // scalar loads (an argument indexed at run time is a chain of loads).
    const int bx = blockIdx.x, nwg = gridDim.x;
    // the input of token 0 (several tokens: of the first group) first:
    // nothing ahead of its loads but the argument reads they need
    using InT = std::conditional_t<MT && !KQ, InGrp<R4, TG>, InRegs<R4>>;
    InT in;
    // IN_B: the prepared operand into registers ahead of the weight loads
    // (loads complete in order); its nb M 16 + nb M / 4 words are at most
    // 2 R4 + 1 per thread (nb <= 8 R4, M <= 8)
    // (native 4-vectors: an array of uint4 structs stays in scratch memory)
    typedef unsigned int u4v __attribute__((ext_vector_type(4)));
    constexpr int NWB = IN == IN_B ? 2 * R4 + 1 : 1;
    u4v opw[NWB];
    float opsc = 0.0f;
    const int nwb = (L.terms - L.B) >> 4;
    if constexpr (IN == IN_B) {
        const u4v *src = (const u4v *)q_in;
#pragma unroll
        for (int k = 0; k < NWB; k++) opw[k] = src[min(tid + k * FWG, nwb - 1)];
        opsc = a.scale_in[min(tid, M - 1)];
    } else if constexpr (MT && !KQ) {
        load_group<IN, R4, TG>(x_in, norm_in, q_in, a.x_stride, 0, min(M, TG), K, true, in);
    } else {
        load_input<IN, R4>(x_in, norm_in, q_in, a.x_stride, 0, K, in);
    }
    const int ntl = a.n_per + (bx < a.n_rem);              // items of this workgroup (>= 1)
    const int ts1 = a.tile_start[1], ts2 = a.tile_start[2], ts3 = a.tile_start[3];
    // (integer arithmetic only: comparisons turned into 0/1 values and
    // branches would split the scalar work of the prologue into many small
    // blocks; tile_start entries past the last segment are INT_MAX)
    auto item = [&](int ti, int sl, int &sg, int &tl) {
        const int w = bx + ti * nwg;
        if (EPI == EPI_SILU) {
            sg = sl;
            tl = w;
        } else {
            const int c1 = (int)((unsigned)(ts1 - 1 - w) >> 31);    // w >= ts1
            const int c2 = (int)((unsigned)(ts2 - 1 - w) >> 31);
            const int c3 = (int)((unsigned)(ts3 - 1 - w) >> 31);
            sg = c1 + c2 + c3;
            tl = w - (c1 * ts1 + c2 * (ts2 - ts1) + c3 * (ts3 - ts2));
        }
    };
    const int nunits = nslab * nb;
    const int nu = wave < nunits ? (nunits - 1 - wave) / FW + 1 : 0;   // units per item
    const int total = nu * ntl;
    // unit r (of nu) of item ti: block u = wave + FW r of the item's units
    // (clamped to the item's last one: a wave without units reads that)
    // The wave's weight cursor: unit r of item ti, its chunk, the chunk's
    // bytes and (FMT_KQMIX) whether its segment is Q6_K.
    struct Cur {
        int ti, r;
        const uint8_t *p;
        int ch, q6;
    };
    auto unit_cur = [&](int ti, int r) -> Cur {
        // (one slab: sl = 0 written out, the compiler cannot see that u < nb)
        const int u = min(wave + FW * r, nunits - 1), sl = nslab == 1 ? 0 : u >= nb;
        const int b = u - sl * nb;
        int sg, tl;
        item(ti, sl, sg, tl);
        const int ch = chunk_of(sg);
        return Cur{ti, r, pick4(a.w, sg) + ((size_t)tl * nb + b) * ch, ch, (int)seg_q6(sg)};
    };
    // (item, unit) counters stepped one unit at a time (no divisions, no
    // branches)
    auto step = [&](int &ti, int &r) {
        const int wrap = r + 1 == nu;
        r = wrap ? 0 : r + 1;
        ti += wrap;
    };
    // The next unit of the same item and slab is FW chunks on; only a new
    // item, or the step from the gate blocks to the up blocks, recomputes
    // the address (the computation is scalar work every wave of the compute
    // unit shares one scalar unit for).  Called only when a next unit
    // exists.
    auto cur_next = [&](Cur c) -> Cur {
        const int u = wave + FW * c.r;
        if (c.r + 1 == nu || (EPI == EPI_SILU && u < nb && u + FW >= nb)) {   // (uniform)
            int ti = c.ti, r = c.r;
            step(ti, r);
            return unit_cur(ti, r);
        }
        return Cur{c.ti, c.r + 1, c.p + FW * (FMT == FMT_KQMIX ? c.ch : CHUNK), c.ch, c.q6};
    };
    // one token of a ternary format: the transposed block (block_mfma_t1)
    constexpr bool T1 = FMT == FMT_TQ2 && MT == 0;
    auto load_unit = [&](const Cur &c) -> RawBlk<FMT> {
        if constexpr (FMT == FMT_KQMIX) return load_raw_mix(c.p, lane, c.q6 != 0);
        else if constexpr (T1) return load_raw_t1(c.p, lane);
        else return load_raw<FMT>(c.p, lane);
    };

    // ---- loads in the order they are used (they complete in order): the
    // input of token 0 (above), the first weight blocks, the epilogue's
    // operands.
    //
    // The K-quant kernels keep one block per wave in flight: with more,
    // tens of MB of weights queue ahead of the input's and the epilogue's
    // loads (8B-class Q4_K/Q6_K decode at 4096 rows, alternating runs: 376.6
    // tok/s with one, 353.3 with four (three for the mixed q/k/v), 369.5 with
    // one but three for the mix, 366.6 with two, 322.3 with six).  The
    // ternary kernels keep three (two or four: 4B-class decode 501.8 and
    // 503.9 against 510.1 tok/s).
    constexpr int PF = KQ ? 1 : MT ? pf_of(R4, EPI == EPI_SILU ? 2 : 1) : PF_ONE;
    // (every wave issues PF block loads before the input stage, past its
    // last unit re-reading that one, so that the input's first use waits for
    // the input only)
    RawBlk<FMT> raw[PF];
    Cur fc = unit_cur(0, 0);                               // unit k (then PF) of the wave
#pragma unroll
    for (int k = 0; k < PF; k++) {
        raw[k] = load_unit(fc);
        if (k + 1 < total) fc = cur_next(fc);              // past the last unit: reload it
    }

    // combiner threads: (slab, token, row) of an item's outputs.  A
    // workgroup with exactly two items ends them together: the waves from
    // hbase on take the second item, so that its blocks follow the first
    // item's with no barrier between, and one barrier and one combine serve
    // both (whole waves, so that the item index stays wave-uniform).
    const int nthr = nslab * 16 * M, hbase = (nthr + 63) & ~63;
    const bool pair = !KQ && EPI != EPI_SUMS && ntl == 2 && hbase + nthr <= FWG;   // (uniform)
    const int hb = pair && wave >= (hbase >> 6) ? 1 : 0;   // the wave's item of the pair
    const int ltid = tid - hb * hbase;
    const bool comb = ltid < nthr;
    const int csl = ltid / (16 * M), crem = ltid - csl * 16 * M;
    const int ct = crem >> 4, crow = crem & 15;
    // the position through the scalar cache: its wait does not wait for the
    // vector loads above
    size_t rp = 0;
    if (EPI == EPI_ROPE)
        rp = (size_t)*(const __attribute__((address_space(4))) uint32_t *)a.pos + (size_t)ct;
    // epilogue operands of item ti for this thread (old output, RoPE table)
    // (loads at clamped in-range addresses, values dropped where unused: a
    // fixed number of loads keeps the compiler's waits exact)
    auto epi_load = [&](int ti, float &p0, float &p1) {
        int sg, tl;
        item(ti < ntl ? ti : ntl - 1, csl < nslab ? csl : 0, sg, tl);
        const int nr = pick4(a.n_rows, sg);
        int orow = tl * 16 + crow;
        orow = orow < nr ? orow : nr - 1;
        if (EPI == EPI_STORE && (a.flags & FOX_GPU_GEMV_ACCUMULATE))   // (uniform)
            p0 = pick4(a.out, sg)[(size_t)ct * pick4(a.out_stride, sg) + orow];
        if (EPI == EPI_ROPE) {
            const int half = a.head_dim / 2, i = (orow % a.head_dim) >> 1;
            const size_t rc = rp < (size_t)a.n_ctx ? rp : (size_t)a.n_ctx - 1;
            p0 = a.rope_cos[rc * half + i];
            p1 = a.rope_sin[rc * half + i];
        }
    };
    float pre0 = 0.0f, pre1 = 0.0f;
    // (the first item's old outputs or RoPE table entries: in flight during
    // the input stage)
    if (EPI == EPI_STORE || EPI == EPI_ROPE) epi_load(hb, pre0, pre1);
    // (nothing that uses the input may be scheduled above the weight loads)
    __builtin_amdgcn_sched_barrier(0);
    // the zero padding of the term rows (read after the input stage's
    // barriers)
    if (nbp != nb * T) {
        const int used = nb * T, pad = nbp - used;
        for (int i = tid; i < 2 * nslab * 16 * M * pad; i += FWG) {
            const int row = i / pad;
            terms[row * nbp + used + (i - row * pad)] = 0.0f;
        }
    }

    // ---- input stage: int8 activations straight into the B operand in LDS
    // (token 0 outside the loop: its waits then count the loads above)
    if constexpr (IN == IN_B) {
        // fused_prep's output has the LDS carve-up of B and the corrections
        // (one run of 16-byte words), then the token scales
        u4v *dst = (u4v *)(lds + L.B);
#pragma unroll
        for (int k = 0; k < NWB; k++)
            if (tid + k * FWG < nwb) dst[tid + k * FWG] = opw[k];
        if (tid < M) ascale[tid] = opsc;
    } else if constexpr (KQ) {
        quantise_kq<FMT, IN, R4>(a, K, (int8_t *)B, aux, bsc, dred, in);
    } else if constexpr (MT == 2) {
        // the groups in turn (the first in flight since the start; a later
        // group's loads go out once the group before is quantised)
        for (int t0 = 0; t0 < M; t0 += TG) {
            if (t0 > 0)
                load_group<IN, R4, TG>(x_in, norm_in, q_in, a.x_stride, t0, min(M - t0, TG), K,
                                       false, in);
            quantise_group<FMT, IN, R4, TG>(a, t0, min(M - t0, TG), K, B, aux, dred, ured,
                                            ascale, in);
        }
    } else if constexpr (MT == 1) {
        // the groups in turn, the next one's input in flight while a group
        // is quantised (the first is in flight since the start)
        for (int t0 = 0; t0 < M; t0 += TG) {
            InT cur = in;
            if (t0 + TG < M)
                load_group<IN, R4, TG>(x_in, norm_in, q_in, a.x_stride, t0 + TG,
                                       min(M - t0 - TG, TG), K, false, in);
            quantise_group<FMT, IN, R4, TG>(a, t0, min(M - t0, TG), K, B, aux, dred, ured,
                                            ascale, cur);
        }
    } else {
        const float s = quantise_to_b<FMT, IN, R4>(a, 0, K, B, aux, dred, ured, in);
        if (tid == 0) ascale[0] = s;
    }
    __syncthreads();

    // ---- end of item ti0 (with both: of items ti0 and ti0 + 1, the pair):
    // ordered combine, activation scale, epilogue
    auto item_end = [&](int ti0, bool both) {
        if (EPI == EPI_SUMS) return;
        __syncthreads();
        const int ti = ti0 + hb;
        const bool act = comb && (hb == 0 || both);
        int sg = 0, tl = 0;
        item(ti, csl, sg, tl);
        const int orow = tl * 16 + crow;
        const bool owns = act && orow < pick4(a.n_rows, sg);
        float y = 0.0f;
        if (act) {
            // The row's terms in block order, four at a time (chunk c holds
            // terms 4c .. 4c + 3).  Four chunk slots rotate, each reloaded
            // with the chunk four ahead right after its adds (the
            // scheduling barriers keep that order), so that the reads
            // overlap the adds; with up to four chunks all reads go out at
            // once.
            const int nbpi = FMT == FMT_KQMIX && seg_q6(sg) ? nbp6 : nbp;
            const float4 *tq = (const float4 *)(terms + (ti & 1) * tstride +
                                                ((csl * 16 + crow) * M + ct) * nbpi);
            const int nq = nbpi >> 2, last = nq - 1;
            float acc = 0.0f;
            auto add4 = [&](const float4 &v) {
                acc = acc + v.x; acc = acc + v.y; acc = acc + v.z; acc = acc + v.w;
            };
            float4 S0 = tq[0], S1 = tq[min(1, last)], S2 = tq[min(2, last)], S3 = tq[min(3, last)];
            int c = 0;
            for (; c + 8 <= nq; c += 4) {
                add4(S0); S0 = tq[c + 4]; __builtin_amdgcn_sched_barrier(0);
                add4(S1); S1 = tq[c + 5]; __builtin_amdgcn_sched_barrier(0);
                add4(S2); S2 = tq[c + 6]; __builtin_amdgcn_sched_barrier(0);
                add4(S3); S3 = tq[c + 7]; __builtin_amdgcn_sched_barrier(0);
            }
            // the slots hold chunks c .. c + 3 (those below nq)
            add4(S0);
            if (c + 1 < nq) add4(S1);
            if (c + 2 < nq) add4(S2);
            if (c + 3 < nq) add4(S3);
            for (c += 4; c < nq; c++) add4(tq[c]);
            // (the ternary formats' per-vector scale: src/gemv.c:70; the
            // K-quants' per-block scales are inside the terms)
            y = KQ ? acc : acc * ascale[ct];
        }
        if (EPI == EPI_STORE) {
            if (owns) {
                float *o = pick4(a.out, sg) + (size_t)ct * pick4(a.out_stride, sg) + orow;
                *o = (a.flags & FOX_GPU_GEMV_ACCUMULATE) ? pre0 + y : y;
            }
        } else if (EPI == EPI_SILU) {
            if (act) ybuf[tid] = y;
            __syncthreads();
            if (owns && csl == 0) {
                const float gt = y, up = ybuf[hb * hbase + 16 * M + crem];
                a.out[0][(size_t)ct * a.out_stride[0] + orow] =
                    fox_div(gt, 1.0f + fox_expf(-gt)) * up; // src/ops.c:45-46
            }
        } else {  // EPI_ROPE: roles 0 q, 1 k, 2 v (segment sg has role role0 + sg)
            const float partner = lane_xor1(y);
            const int role = sg + a.role0;
            if (owns) {
                const bool inside = rp < (size_t)a.n_ctx;
                float v = y;
                if (role < 2 && inside) {
                    // src/ops.c:64-69 on the pair (row & ~1, row | 1)
                    v = (orow & 1) ? partner * pre1 + y * pre0 : y * pre0 - partner * pre1;
                }
                if (role == 0) {
                    a.out[0][(size_t)ct * a.out_stride[0] + orow] = v;
                } else if (inside) {
                    const size_t kvd = (size_t)a.kv_dim;
                    if (role == 1) a.k_cache[rp * kvd + orow] = v;
                    else a.v_cache[((rp >> 2) * kvd + orow) * 4 + (rp & 3)] = v;
                }
            }
        }
        // the next item's operands, loaded into the registers just read (no
        // copy: a copy would wait here for the load); they are used at that
        // item's end, after its blocks
        if ((EPI == EPI_STORE || EPI == EPI_ROPE) && !pair && ti + 1 < ntl)
            epi_load(ti + 1, pre0, pre1);
    };

    // ---- blocks: integer sums, then one float term per row and token (T
    // per row for the K-quants).  A wave's units run through all its items;
    // PF blocks stay in flight.
    const int g = lane >> 4, j = lane & 15;

    const int bbytes = b_bytes_per_block_tok(FMT) * M;
    const bool lead = j < M;
    const int tok = j;
    // a lead lane's terms: rows 4g .. 4g + 3 of token tok, row after row
    // M * nbp floats apart, the up slab 16 M nbp floats on
    const int rstep = M * nbp, tlane = (4 * g * M + tok) * nbp;
    // (the end of item ti; the pair's first item ends with its second)
    auto item_done = [&](int ti) {
        if (pair && ti == 0) return;
        item_end(pair ? 0 : ti, pair);
    };
    if (nu == 0) {
        for (int ti = 0; ti < ntl; ti++) item_done(ti);
        return;
    }
    int ti = 0, r = 0;                                     // unit n of the wave
    for (int n0 = 0; n0 < total; n0 += PF) {
#pragma unroll
        for (int k = 0; k < PF; k++) {
            const int n = n0 + k;
            if (n >= total) break;
            const int u = wave + FW * r, sl = nslab == 1 ? 0 : u >= nb, b = u - sl * nb;
            if constexpr (KQ) {
                // lane (row j, part g): T / 4 terms of its row
                const RawBlk<FMT> rk = raw[k];
                if (n + PF < total) {
                    raw[k] = load_unit(fc);
                    if (n + PF + 1 < total) fc = cur_next(fc);
                }
                const int8_t *xb = (const int8_t *)B + b * 256;
                const float as = bsc[b];
                if constexpr (FMT == FMT_KQMIX) {
                    int sg, tl;
                    item(ti, sl, sg, tl);
                    if (seg_q6(sg)) {                                        // (uniform)
                        float *tp = terms + (ti & 1) * tstride + (sl * 16 + j) * nbp6 + b * 4;
                        tp[g] = q6k_term(q6k_view(rk), xb, aux + 8 * nb + b * 16, as, lane);
                    } else {
                        float *tp = terms + (ti & 1) * tstride + (sl * 16 + j) * nbp + b * 8;
                        float t0, t1;
                        q4k_terms(q4k_view(rk), xb, aux + b * 8, as, g, t0, t1);
                        *(float2 *)(tp + 2 * g) = make_float2(t0, t1);
                    }
                } else if constexpr (FMT == FMT_Q4K) {
                    float *tp = terms + (ti & 1) * tstride + (sl * 16 + j) * nbp + b * T;
                    float t0, t1;
                    q4k_terms(rk, xb, aux + b * 8, as, g, t0, t1);
                    *(float2 *)(tp + 2 * g) = make_float2(t0, t1);
                } else {
                    float *tp = terms + (ti & 1) * tstride + (sl * 16 + j) * nbp + b * T;
                    tp[g] = q6k_term(rk, xb, aux + b * 16, as, lane);
                }
            } else if constexpr (T1) {
                const int S = block_mfma_t1(raw[k], B + b * bbytes, lane, aux[b]);
                const RawBlk<FMT> rk = raw[k];
                if (n + PF < total) {
                    raw[k] = load_unit(fc);
                    if (n + PF + 1 < total) fc = cur_next(fc);
                }
                if (lane < 16) {                    // row lane of the tile
                    if (EPI == EPI_SUMS) {
                        int sg, tl;
                        item(ti, sl, sg, tl);
                        const int nrows = pick4(a.n_rows, sg), grow = tl * 16 + lane;
                        if (grow < nrows) a.sums[(size_t)grow * nb + b] = S;
                    } else {
                        const float d = half_bits_to_float(rk.dd.x & 0xFFFFu);
                        terms[(ti & 1) * tstride + (sl * 16 + lane) * nbp + b] = d * (float)S;
                    }
                }
            } else {
                const int corr = aux[b * M + (lead ? tok : M - 1)];   // (used by lead lanes)
                int S[4];
                block_mfma<FMT>(raw[k], B + b * bbytes, M, lane, corr, S);
                const RawBlk<FMT> rk = raw[k];
                if (n + PF < total) {
                    raw[k] = load_unit(fc);
                    if (n + PF + 1 < total) fc = cur_next(fc);
                }
                if (lead) {
                    const uint32_t hw[2] = {rk.dd.x, rk.dd.y};
                    int sg, tl;
                    item(ti, sl, sg, tl);
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const int row = 4 * g + q;
                        if (EPI == EPI_SUMS) {
                            const int nrows = pick4(a.n_rows, sg), grow = tl * 16 + row;
                            if (grow < nrows) a.sums[((size_t)tok * nrows + grow) * nb + b] = S[q];
                        } else {
                            const float d = half_bits_to_float((hw[q >> 1] >> (16 * (q & 1))) & 0xFFFFu);
                            terms[(ti & 1) * tstride + sl * 16 * rstep + tlane + q * rstep + b] =
                                d * (float)S[q];
                        }
                    }
                }
            }
            if (r == nu - 1) item_done(ti);
            step(ti, r);
        }
    }
}

// Several tokens (f32 or RMS-normed input): the input stage once per launch
// instead of once per GEMV workgroup.  Workgroup t takes token t through
// quantise_to_b (RMSNorm, per-vector int8 quantisation of src/gemv.c:11-42,
// B operand and per-block corrections, the operations and order of the
// one-token kernels) into global memory laid out as the GEMV's LDS carve-up
// for all the tokens (B at 0, corrections at `aux`), and writes its
// activation scale; the GEMV copies the operand into LDS (IN_B).
template <int IN, int R4>
__global__ __launch_bounds__(FWG) void fused_prep(const float *x_in, const float *norm_in,
                                                  int nb_in, FusedArgs a, uint8_t *B,
                                                  int32_t *aux, float *scale)
{
    __shared__ double dred[FW];
    __shared__ uint32_t ured[FW];
    const int t = blockIdx.x, K = nb_in * 256;
    InRegs<R4> in;
    load_input<IN, R4>(x_in, norm_in, nullptr, a.x_stride, t, K, in);
    const float s = quantise_to_b<FMT_TQ2, IN, R4>(a, t, K, B, aux, dred, ured, in);
    if (threadIdx.x == 0) scale[t] = s;
}

// ------------------------------------------------------------ host

// Workgroups write output rows while others still read the input, so an
// output must not overlap the input (the unfused path has no such limit).
static bool out_overlaps(const void *in, size_t in_bytes, size_t n, float *const *outs,
                         const size_t *rows, const size_t *strides, size_t M)
{
    const uintptr_t i0 = (uintptr_t)in, i1 = i0 + in_bytes;
    for (size_t k = 0; k < n; k++) {
        if (!outs[k]) continue;
        const uintptr_t o0 = (uintptr_t)outs[k];
        const uintptr_t o1 = o0 + ((M - 1) * (M > 1 ? strides[k] : 0) + rows[k]) * sizeof(float);
        if (o0 < i1 && i0 < o1) return true;
    }
    return false;
}

// the input stage reads x (and the norm weights) as float4, q as int32
static bool fused_aligned(const void *x, size_t x_stride, size_t M, const void *w)
{
    return !((uintptr_t)x % 16) && !((uintptr_t)w % 16) && (M == 1 || x_stride % 4 == 0);
}

static fox_gpu_status fused_check(int type, size_t K, size_t M, int nslab, int *fmt,
                                  bool norm = false)
{
    if (norm && K > 4 * R4_LIMIT_NORM * FWG)
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "fused gemv: K = %zu exceeds the %d values "
                        "one workgroup holds beside the norm weights", K,
                        4 * R4_LIMIT_NORM * FWG);
    *fmt = fmt_of(type);
    if (*fmt < 0)
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "fused gemv: %s weights use the unfused path",
                        fox_type_name(type));
    if (*fmt != FMT_TQ2 && M != 1)
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "fused gemv: %s weights take the fused path "
                        "for one token only", fox_type_name(type));
    if (K % 256 || K == 0) return fox_fail(FOX_GPU_ERR_ARG, "fused gemv: K %% 256 != 0");
    if (K > 4 * R4_LIMIT * FWG)
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "fused gemv: K = %zu exceeds the %d values "
                        "one workgroup holds", K, 4 * R4_LIMIT * FWG);
    if (M == 0 || M > FOX_GPU_MAX_TOKENS)
        return fox_fail(FOX_GPU_ERR_ARG, "fused gemv: 1 to %d tokens", FOX_GPU_MAX_TOKENS);
    if (fused_lds(*fmt, (int)K, (int)M, nslab).total > fused_lds_max(M))
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "fused gemv: %zu x %zu activations exceed the "
                        "workgroup's LDS", M, K);
    return FOX_GPU_OK;
}

// n_work items (tiles, or gate/up tile pairs) over at most two persistent
// workgroups per compute unit, or one from three tokens on (every workgroup
// quantises all the tokens' input, and two on a compute unit would do that
// VALU work twice; 14336 x 4096 at 8 tokens: 16.3 -> 13.9 us, at 4 tokens
// 11.4 -> 10.7 us, at 2 tokens 8.9 -> 9.2 us)
template <int FMT, int IN, int EPI, int R4>
static fox_gpu_status fused_go_r(fox_gpu_ctx *ctx, FusedArgs a, int n_work, uint8_t *fixed)
{
    // (the K-quants have the one-token kernels only: fused_check)
    constexpr bool MT_OK = FMT == FMT_TQ2;
    const int mt = MT_OK ? (a.M > 2 ? 2 : a.M > 1 ? 1 : 0) : 0;
    // (the multi-token kernels exist for the ternary formats only; from
    // three tokens on, f32 and normed input is prepared once by fused_prep
    // and the GEMV reads it as IN_B)
    constexpr int MT1 = MT_OK ? 1 : 0, MT2 = MT_OK ? 2 : 0;
    constexpr bool PREP = MT_OK && (IN == IN_F32 || IN == IN_NORM) && EPI != EPI_SUMS;
    constexpr int IN2 = PREP ? IN_B : IN;
    const FusedLds L = fused_lds(FMT, a.nb * 256, a.M, EPI == EPI_SILU ? 2 : 1);
    const size_t lds = L.total;
    // workgroups per compute unit: two, or one from three tokens on unless
    // the input comes prepared and two fit the LDS and the registers (R4 <= 5:
    // at most 128 VGPRs)
    const int per_cu = mt == 2 ? (PREP && R4 <= 5 && lds <= 80 * 1024 ? 2 : 1) : 2;
    a.n_work = n_work;
    int cap = per_cu * (ctx->n_cu > 0 ? ctx->n_cu : 1);
    if (ctx->max_wg > 0 && ctx->max_wg < cap) cap = ctx->max_wg;
    const int grid = n_work < cap ? n_work : cap;
    a.n_per = n_work / grid;
    a.n_rem = n_work - a.n_per * grid;
    const void *k = mt == 2 ? (const void *)gemv_fused<FMT, IN2, EPI, R4, MT2>
                  : mt == 1 ? (const void *)gemv_fused<FMT, IN, EPI, R4, MT1>
                            : (const void *)gemv_fused<FMT, IN, EPI, R4, 0>;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return fox_hip_fail(e, "fused gemv: LDS size");
    }
    if (mt == 2) {
        if constexpr (PREP) {
            // the operand (B and corrections, L.terms bytes) then the token
            // scales, in the workspace or the caller's fixed scratch
            const size_t opb = (size_t)(L.terms - L.B);
            const size_t need = opb + FOX_GPU_MAX_TOKENS * sizeof(float);
            if (opb > (size_t)(2 * R4 + 1) * FWG * 16)      // (the kernel's registers for it)
                return fox_fail(FOX_GPU_ERR_INTERNAL, "fused gemv: %zu bytes of prepared input "
                                "for %d input dwords per thread", opb, R4);
            uint8_t *buf = fixed;
            if (fixed) {
                if (need > FOX_NOALLOC_SCRATCH)
                    return fox_fail(FOX_GPU_ERR_ARG, "fused gemv: %zu bytes of prepared input "
                                    "exceed the fixed scratch (%u)", need, FOX_NOALLOC_SCRATCH);
            } else {
                fox_gpu_status st = fox_ws_reserve(ctx, need);
                if (st) return st;
                buf = ctx->ws;
            }
            float *sc = (float *)(buf + opb);
            hipLaunchKernelGGL((fused_prep<IN, R4>), dim3((unsigned)a.M), dim3(FWG), 0,
                               ctx->stream, a.x, a.norm_w, a.nb, a, buf,
                               (int32_t *)(buf + (L.aux - L.B)), sc);
            FOX_LAUNCHED("fused_prep");
            FusedArgs b = a;
            b.q_in = (const int8_t *)buf;
            b.scale_in = sc;
            hipLaunchKernelGGL((gemv_fused<FMT, IN2, EPI, R4, MT2>), dim3((unsigned)grid),
                               dim3(FWG), lds, ctx->stream, nullptr, nullptr, b.q_in, b.nb, b);
        } else {
            hipLaunchKernelGGL((gemv_fused<FMT, IN, EPI, R4, MT2>), dim3((unsigned)grid),
                               dim3(FWG), lds, ctx->stream, a.x, a.norm_w, a.q_in, a.nb, a);
        }
    }
    else if (mt == 1)
        hipLaunchKernelGGL((gemv_fused<FMT, IN, EPI, R4, MT1>), dim3((unsigned)grid), dim3(FWG),
                           lds, ctx->stream, a.x, a.norm_w, a.q_in, a.nb, a);
    else
        hipLaunchKernelGGL((gemv_fused<FMT, IN, EPI, R4, 0>), dim3((unsigned)grid), dim3(FWG),
                           lds, ctx->stream, a.x, a.norm_w, a.q_in, a.nb, a);
    FOX_LAUNCHED("gemv_fused");
    return FOX_GPU_OK;
}

// the input registers per thread fit K: 1, 2, 3, 5, 8 or (without the
// norm weights beside the input) 11 dwords
template <int FMT, int IN, int EPI>
static fox_gpu_status fused_go(fox_gpu_ctx *ctx, const FusedArgs &a, int grid, uint8_t *fixed)
{
    const int per = (a.nb * 64 + FWG - 1) / FWG;
    if (per <= 1) return fused_go_r<FMT, IN, EPI, 1>(ctx, a, grid, fixed);
    if (per <= 2) return fused_go_r<FMT, IN, EPI, 2>(ctx, a, grid, fixed);
    if (per <= 3) return fused_go_r<FMT, IN, EPI, 3>(ctx, a, grid, fixed);
    if (per <= 5) return fused_go_r<FMT, IN, EPI, 5>(ctx, a, grid, fixed);
    if constexpr (IN == IN_NORM) {
        return fused_go_r<FMT, IN, EPI, 8>(ctx, a, grid, fixed);   // (fused_check: K <= 16384)
    } else {
        if (per <= 8) return fused_go_r<FMT, IN, EPI, 8>(ctx, a, grid, fixed);
        return fused_go_r<FMT, IN, EPI, 11>(ctx, a, grid, fixed);
    }
}

// (the K-quant kernels take f32 input and write outputs: int8 input with
// per-block scales and the block-sum requests take the unfused path)
// (fixed: the caller's scratch for fused_prep's output, or null for the
// context's workspace)
template <int IN, int EPI>
static fox_gpu_status fused_dispatch(fox_gpu_ctx *ctx, int fmt, const FusedArgs &a, int grid,
                                     uint8_t *fixed = nullptr)
{
    if constexpr (IN != IN_Q && EPI != EPI_SUMS) {
        if (fmt == FMT_Q4K) return fused_go<FMT_Q4K, IN, EPI>(ctx, a, grid, fixed);
        if (fmt == FMT_Q6K) return fused_go<FMT_Q6K, IN, EPI>(ctx, a, grid, fixed);
    }
    if constexpr (IN == IN_NORM && EPI == EPI_ROPE) {
        if (fmt == FMT_KQMIX) return fused_go<FMT_KQMIX, IN, EPI>(ctx, a, grid, fixed);
    }
    return fused_go<FMT_TQ2, IN, EPI>(ctx, a, grid, fixed);
}

static void fused_segments(FusedArgs &a, size_t n, const fox_gpu_tensor *const *ws,
                           float *const *outs, const size_t *strides, size_t M, int *tiles)
{
    int t = 0;
    for (size_t i = 0; i < n; i++) {
        a.w[i] = ws[i]->d;
        a.out[i] = outs ? outs[i] : nullptr;
        a.out_stride[i] = strides ? (int)(M > 1 ? strides[i] : ws[i]->ne1) : 0;
        a.n_rows[i] = (int)ws[i]->ne1;
        a.tile_start[i] = t;
        t += (int)ws[i]->n_tiles;
    }
    a.tile_start[n] = t;
    for (size_t i = n + 1; i <= MAX_SEGS; i++) a.tile_start[i] = 0x7fffffff;
    a.nseg = (int)n;
    *tiles = t;
}

// The fused entry for y_i = W_i x of the existing gemv calls (x f32 or int8);
// returns FOX_GPU_ERR_UNSUPPORTED when the unfused path must run instead.
fox_gpu_status fox_fused_gemv(fox_gpu_ctx *ctx, size_t n, const fox_gpu_tensor *const *ws,
                              const float *x, size_t x_stride, const int8_t *q,
                              const float *scale, size_t M, float *const *outs,
                              const size_t *out_strides, unsigned flags, int32_t *sums,
                              uint8_t *fixed_ws)
{
    int fmt;
    const size_t K = (size_t)ws[0]->ne0;
    const int f = fmt_of(ws[0]->type);
    if (f < 0 || (f != FMT_TQ2 && (M != 1 || q || sums)))
        return FOX_GPU_ERR_UNSUPPORTED;
    if (fused_lds(f, (int)K, (int)M, 1).total > fused_lds_max(M) ||
        K > 4 * R4_LIMIT * FWG || !fused_aligned(x ? (const void *)x : (const void *)q,
                                             x ? x_stride : K, M, nullptr))
        return FOX_GPU_ERR_UNSUPPORTED;
    fox_gpu_status st = fused_check(ws[0]->type, K, M, 1, &fmt);
    if (st) return st;
    if (outs) {
        size_t rows[MAX_SEGS];
        for (size_t i = 0; i < n; i++) rows[i] = (size_t)ws[i]->ne1;
        const size_t in_bytes = x ? ((M - 1) * (M > 1 ? x_stride : 0) + K) * sizeof(float) : M * K;
        if (out_overlaps(x ? (const void *)x : (const void *)q, in_bytes, n, outs, rows,
                         out_strides, M))
            return FOX_GPU_ERR_UNSUPPORTED;
    }
    FusedArgs a;
    memset(&a, 0, sizeof(a));
    int tiles;
    fused_segments(a, n, ws, outs, out_strides, M, &tiles);
    a.nb = (int)(K / 256);
    a.M = (int)M;
    a.flags = flags;
    a.x = x;
    a.x_stride = (int)(M > 1 ? x_stride : K);
    a.q_in = q;
    a.scale_in = scale;
    a.sums = sums;
    if ((!x && !q) || (!sums && (!outs || (q && !scale))))
        return fox_fail(FOX_GPU_ERR_ARG, "fused gemv: missing activations, scale or output");
    if (sums) return fused_dispatch<IN_Q, EPI_SUMS>(ctx, fmt, a, tiles);
    if (q) return fused_dispatch<IN_Q, EPI_STORE>(ctx, fmt, a, tiles);
    return fused_dispatch<IN_F32, EPI_STORE>(ctx, fmt, a, tiles, fixed_ws);
}

extern "C" fox_gpu_status fox_gpu_gemv_rmsnorm(fox_gpu_ctx *ctx, size_t n,
                                               const fox_gpu_tensor *const *ws, const float *x,
                                               size_t x_stride, size_t M, const float *norm_w,
                                               float eps, float *const *outs,
                                               const size_t *out_strides, unsigned flags)
{
    if (!ctx || !ws || !x || !norm_w || !outs || !out_strides || n == 0 || n > MAX_SEGS)
        return fox_fail(FOX_GPU_ERR_ARG, "gemv_rmsnorm: bad argument");
    for (size_t i = 0; i < n; i++) {
        if (!ws[i] || !outs[i]) return fox_fail(FOX_GPU_ERR_ARG, "gemv_rmsnorm: null tensor");
        if (ws[i]->type != ws[0]->type || ws[i]->ne0 != ws[0]->ne0)
            return fox_fail(FOX_GPU_ERR_ARG, "gemv_rmsnorm: matrices must share type and width");
        if (M > 1 && out_strides[i] < ws[i]->ne1)
            return fox_fail(FOX_GPU_ERR_ARG, "gemv_rmsnorm: output stride < rows");
    }
    const size_t K = (size_t)ws[0]->ne0;
    if (M > 1 && x_stride < K) return fox_fail(FOX_GPU_ERR_ARG, "gemv_rmsnorm: input stride < K");
    int fmt;
    fox_gpu_status st = fused_check(ws[0]->type, K, M, 1, &fmt, true);
    if (st) return st;
    if (!fused_aligned(x, x_stride, M, norm_w))
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "gemv_rmsnorm: x and norm_w must be 16-byte "
                        "aligned, the stride a multiple of 4");
    {
        size_t rows[MAX_SEGS];
        for (size_t i = 0; i < n; i++) rows[i] = (size_t)ws[i]->ne1;
        if (out_overlaps(x, ((M - 1) * (M > 1 ? x_stride : 0) + K) * sizeof(float), n, outs, rows,
                         out_strides, M))
            return fox_fail(FOX_GPU_ERR_ARG, "gemv_rmsnorm: an output overlaps the input");
    }
    FusedArgs a;
    memset(&a, 0, sizeof(a));
    int tiles;
    fused_segments(a, n, ws, outs, out_strides, M, &tiles);
    a.nb = (int)(K / 256);
    a.M = (int)M;
    a.flags = flags;
    a.x = x;
    a.x_stride = (int)(M > 1 ? x_stride : K);
    a.norm_w = norm_w;
    a.eps = eps;
    return fused_dispatch<IN_NORM, EPI_STORE>(ctx, fmt, a, tiles);
}

extern "C" fox_gpu_status fox_gpu_qkv_rope(fox_gpu_ctx *ctx, const fox_gpu_tensor *wq,
                                           const fox_gpu_tensor *wk, const fox_gpu_tensor *wv,
                                           const float *x, size_t x_stride, size_t M,
                                           const float *norm_w, float eps, float *q_out,
                                           size_t q_stride, const float *cos_t,
                                           const float *sin_t, const uint32_t *pos,
                                           size_t n_ctx, float *k_cache, float *v_cache,
                                           size_t head_dim)
{
    if (!ctx || !wq || !wk || !wv || !x || !norm_w || !q_out || !cos_t || !sin_t || !pos ||
        !k_cache || !v_cache || head_dim == 0 || n_ctx == 0)
        return fox_fail(FOX_GPU_ERR_ARG, "qkv_rope: bad argument");
    if (wq->ne0 != wk->ne0 || wk->ne0 != wv->ne0 || wk->ne1 != wv->ne1)
        return fox_fail(FOX_GPU_ERR_ARG, "qkv_rope: q, k, v must share their width, k and v "
                        "their rows");
    if (head_dim % 2 || wq->ne1 % head_dim || wk->ne1 % head_dim)
        return fox_fail(FOX_GPU_ERR_ARG, "qkv_rope: rows are not whole heads of even size");
    const size_t K = (size_t)wq->ne0;
    if (M > 1 && (x_stride < K || q_stride < wq->ne1))
        return fox_fail(FOX_GPU_ERR_ARG, "qkv_rope: stride too small");
    if (n_ctx > 0x7fffffff) return fox_fail(FOX_GPU_ERR_ARG, "qkv_rope: n_ctx too large");
    // Q4_K and Q6_K side by side (a Q4_K_M-style mix) run as one launch,
    // each segment in its own format; v of another type than q and k
    // otherwise runs as a second launch over the same input
    int fmt, fmt_k, fmt_v = -1;
    fox_gpu_status st = fused_check(wq->type, K, M, 1, &fmt, true);
    if (st) return st;
    if ((st = fused_check(wk->type, K, M, 1, &fmt_k, true))) return st;
    if ((st = fused_check(wv->type, K, M, 1, &fmt_v, true))) return st;
    auto kq = [](int f) { return f == FMT_Q4K || f == FMT_Q6K; };
    int q6_mask = 0;
    if (kq(fmt) && kq(fmt_k) && kq(fmt_v) && (fmt != fmt_k || fmt != fmt_v)) {
        if (fused_lds(FMT_KQMIX, (int)K, 1, 1).total > fused_lds_max(1))
            return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "qkv_rope: K too large for one launch");
        q6_mask = (fmt == FMT_Q6K) | (fmt_k == FMT_Q6K) << 1 | (fmt_v == FMT_Q6K) << 2;
        fmt = fmt_v = FMT_KQMIX;
    } else if (fmt_k != fmt) {
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "qkv_rope: q and k of different types take "
                        "the separate steps");
    }
    const bool split = fmt_v != fmt;
    if (!fused_aligned(x, x_stride, M, norm_w))
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "qkv_rope: x and norm_w must be 16-byte "
                        "aligned, the stride a multiple of 4");
    {
        float *o[1] = {q_out};
        size_t rows[1] = {(size_t)wq->ne1}, str[1] = {q_stride};
        if (out_overlaps(x, ((M - 1) * (M > 1 ? x_stride : 0) + K) * sizeof(float), 1, o, rows,
                         str, M))
            return fox_fail(FOX_GPU_ERR_ARG, "qkv_rope: q_out overlaps the input");
    }
    const fox_gpu_tensor *ws[3] = {wq, wk, wv};
    float *outs[3] = {q_out, nullptr, nullptr};
    size_t strides[3] = {q_stride, 0, 0};
    FusedArgs a;
    memset(&a, 0, sizeof(a));
    int tiles;
    fused_segments(a, split ? 2 : 3, ws, outs, strides, M, &tiles);
    a.out_stride[0] = (int)(M > 1 ? q_stride : wq->ne1);
    a.nb = (int)(K / 256);
    a.M = (int)M;
    a.x = x;
    a.x_stride = (int)(M > 1 ? x_stride : K);
    a.norm_w = norm_w;
    a.eps = eps;
    a.rope_cos = cos_t;
    a.rope_sin = sin_t;
    a.pos = pos;
    a.head_dim = (int)head_dim;
    a.kv_dim = (int)wk->ne1;
    a.n_ctx = (int)n_ctx;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.q6_mask = q6_mask;
    if ((st = fused_dispatch<IN_NORM, EPI_ROPE>(ctx, fmt, a, tiles)) || !split) return st;
    FusedArgs b = a;
    const fox_gpu_tensor *wsv[1] = {wv};
    float *outv[1] = {nullptr};
    size_t strv[1] = {0};
    fused_segments(b, 1, wsv, outv, strv, M, &tiles);
    b.role0 = 2;
    return fused_dispatch<IN_NORM, EPI_ROPE>(ctx, fmt_v, b, tiles);
}

extern "C" fox_gpu_status fox_gpu_gate_up_silu(fox_gpu_ctx *ctx, const fox_gpu_tensor *wg,
                                               const fox_gpu_tensor *wu, const float *x,
                                               size_t x_stride, size_t M, const float *norm_w,
                                               float eps, float *h_out, size_t h_stride)
{
    if (!ctx || !wg || !wu || !x || !norm_w || !h_out)
        return fox_fail(FOX_GPU_ERR_ARG, "gate_up_silu: bad argument");
    if (wg->ne0 != wu->ne0 || wg->ne1 != wu->ne1)
        return fox_fail(FOX_GPU_ERR_ARG, "gate_up_silu: gate and up must have one shape");
    if (wg->type != wu->type)
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "gate_up_silu: gate and up of different types "
                        "take the separate steps");
    const size_t K = (size_t)wg->ne0;
    if (M > 1 && (x_stride < K || h_stride < wg->ne1))
        return fox_fail(FOX_GPU_ERR_ARG, "gate_up_silu: stride too small");
    int fmt;
    fox_gpu_status st = fused_check(wg->type, K, M, 2, &fmt, true);
    if (st) return st;
    if (!fused_aligned(x, x_stride, M, norm_w))
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "gate_up_silu: x and norm_w must be 16-byte "
                        "aligned, the stride a multiple of 4");
    {
        float *o[1] = {h_out};
        size_t rows[1] = {(size_t)wg->ne1}, str[1] = {h_stride};
        if (out_overlaps(x, ((M - 1) * (M > 1 ? x_stride : 0) + K) * sizeof(float), 1, o, rows,
                         str, M))
            return fox_fail(FOX_GPU_ERR_ARG, "gate_up_silu: h_out overlaps the input");
    }
    const fox_gpu_tensor *ws[2] = {wg, wu};
    float *outs[2] = {h_out, nullptr};
    size_t strides[2] = {h_stride, h_stride};
    FusedArgs a;
    memset(&a, 0, sizeof(a));
    int tiles;
    fused_segments(a, 2, ws, outs, strides, M, &tiles);
    a.nb = (int)(K / 256);
    a.M = (int)M;
    a.x = x;
    a.x_stride = (int)(M > 1 ? x_stride : K);
    a.norm_w = norm_w;
    a.eps = eps;
    return fused_dispatch<IN_NORM, EPI_SILU>(ctx, fmt, a, (int)wg->n_tiles);
}
