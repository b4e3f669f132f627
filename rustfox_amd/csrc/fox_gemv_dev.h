// fox_gemv_dev.h -- device helpers shared by the GEMV kernels: the block
// formats' MFMA operand layouts, the exact int8 activation quantiser and
// wave reductions.  See fox_gemv.hip for the exactness contract.
#pragma once

#include "fox_internal.h"

#define MAX_SEGS 4

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));

// (FMT_KQMIX: the one-launch q/k/v of the fused path with Q4_K and Q6_K
// segments side by side, the format chosen per segment)
enum { FMT_TQ2 = 1, FMT_Q4K = 2, FMT_Q6K = 3, FMT_KQMIX = 4 };

// the kernel format of a tensor of `type` (of its layout in HBM: TQ1_0
// tensors are held as TQ2_0 blocks)
static inline int fmt_of(int type)
{
    switch (fox_device_type(type)) {
    case FOX_GPU_TQ2_0: return FMT_TQ2;
    case FOX_GPU_Q4_K: return FMT_Q4K;
    case FOX_GPU_Q6_K: return FMT_Q6K;
    default: return -1;
    }
}

// float terms per block and row in the ordered combine
__host__ __device__ constexpr int terms_per_block(int fmt)
{
    return fmt == FMT_Q4K || fmt == FMT_KQMIX ? 8 : fmt == FMT_Q6K ? 4 : 1;
}

// B-operand bytes per block and token, aux int32 per block and token
__host__ __device__ constexpr int b_bytes_per_block_tok(int fmt)
{
    return fmt == FMT_Q4K ? 512 : 256;
}

__host__ __device__ constexpr int aux_per_block_tok(int fmt)
{
    return fmt == FMT_Q4K ? 8 : fmt == FMT_Q6K ? 16 : fmt == FMT_KQMIX ? 24 : 1;
}

__device__ __forceinline__ float half_bits_to_float(unsigned h)
{
    return (float)__builtin_bit_cast(_Float16, (unsigned short)h);
}

// ---------------------------------------------------------------- reduce

// Lane movement through DPP (a VALU operand modifier, no LDS round trip).
// CTL: 0xB1 quad_perm [1,0,3,2] (lane ^ 1), 0x4E quad_perm [2,3,0,1]
// (lane ^ 2), 0x141 row_half_mirror (lane 7 - i within 8), 0x140 row_mirror
// (lane 15 - i within 16), 0x142 row_bcast:15 (lane 15 of row r to row r + 1),
// 0x143 row_bcast:31 (lane 31 to rows 2 and 3).  Rows outside RM keep `old`.
template <int CTL, int RM, typename T>
__device__ __forceinline__ T dpp_t(T old, T v)
{
    static_assert(sizeof(T) % 4 == 0, "32-bit words");
    constexpr int N = sizeof(T) / 4;
    struct W { int w[N]; };
    const W o = __builtin_bit_cast(W, old), s = __builtin_bit_cast(W, v);
    W r;
#pragma unroll
    for (int i = 0; i < N; i++) r.w[i] = __builtin_amdgcn_update_dpp(o.w[i], s.w[i], CTL, RM, 0xF, false);
    return __builtin_bit_cast(T, r);
}

template <typename T>
__device__ __forceinline__ T read_lane(T v, int l)
{
    constexpr int N = sizeof(T) / 4;
    struct W { int w[N]; };
    const W s = __builtin_bit_cast(W, v);
    W r;
#pragma unroll
    for (int i = 0; i < N; i++) r.w[i] = __builtin_amdgcn_readlane(s.w[i], l);
    return __builtin_bit_cast(T, r);
}

// v of lane ^ 1
template <typename T>
__device__ __forceinline__ T lane_xor1(T v)
{
    return dpp_t<0xB1, 0xF>(v, v);
}

// op over the 64 lanes (op associative and commutative, id its identity):
// quads, 8 lanes, rows, then rows 0+1 into row 1 and 0..3 into row 3; the
// result, read from lane 63, is wave-uniform
template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce(T v, T id, Op op)
{
    v = op(v, dpp_t<0xB1, 0xF>(id, v));
    v = op(v, dpp_t<0x4E, 0xF>(id, v));
    v = op(v, dpp_t<0x141, 0xF>(id, v));
    v = op(v, dpp_t<0x140, 0xF>(id, v));
    v = op(v, dpp_t<0x142, 0xA>(id, v));
    v = op(v, dpp_t<0x143, 0xC>(id, v));
    return read_lane(v, 63);
}

// max over the wave of values that are >= 0 and not NaN
__device__ __forceinline__ float wave_max(float v)
{
    return wave_reduce(v, 0.0f, [](float x, float y) { return y > x ? y : x; });
}

__device__ __forceinline__ int wave_sum_i(int v)
{
    return wave_reduce(v, 0, [](int x, int y) { return x + y; });
}

// src/gemv.c:31-38 and src/kernels.c:744-751 for one element.  The (int)
// conversion of the reference's x86 build (cvttss2si) gives INT_MIN for NaN
// and for values outside int range, which the clamp turns into -127; the
// GPU conversion would give 0 or a saturated value, so those cases are
// mapped explicitly.
__device__ __forceinline__ int8_t quant_one(float x, float inv)
{
    float v = x * inv;
    float t = v < 0.0f ? v - 0.5f : v + 0.5f;
    int r = (t >= -2147483648.0f && t < 2147483648.0f) ? (int)t : (int)0x80000000u;
    r = r > 127 ? 127 : r;
    r = r < -127 ? -127 : r;
    return (int8_t)r;
}

// quant_one when |x| <= amax with amax in [2^-120, inf) and inv = 127 / amax:
// inv is finite, |x * inv| < 127.5 so no clamp applies, and v +/- 0.5 is
// v + copysign(0.5, v) (for v = -0.0 both truncate to 0)
__device__ __forceinline__ int quant_fast(float x, float inv)
{
    const float v = x * inv;
    return (int)(v + __builtin_copysignf(0.5f, v));
}

// the low bytes of r0..r3 as one dword, byte k from r_k
__device__ __forceinline__ uint32_t pack_lo_bytes(int r0, int r1, int r2, int r3)
{
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)r1, (uint32_t)r0, 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)r3, (uint32_t)r2, 0x04000c0cu);
    return lo | hi;
}

__device__ __forceinline__ v4i mfma(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3,
                                    v4i b, v4i c)
{
    v4i a = {(int)a0, (int)a1, (int)a2, (int)a3};
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v4i load_b(const uint8_t *p, bool ok)
{
    v4i z = {0, 0, 0, 0};
    return ok ? *(const v4i *)p : z;
}


// the one-launch GEMV of fox_fused.hip for the ternary formats;
// FOX_GPU_ERR_UNSUPPORTED (no error recorded) when the unfused path applies.
// fixed_ws: scratch of FOX_NOALLOC_SCRATCH bytes for the prepared input of
// three or more tokens, or null for the context's workspace
fox_gpu_status fox_fused_gemv(fox_gpu_ctx *ctx, size_t n, const fox_gpu_tensor *const *ws,
                              const float *x, size_t x_stride, const int8_t *q,
                              const float *scale, size_t M, float *const *outs,
                              const size_t *out_strides, unsigned flags, int32_t *sums,
                              uint8_t *fixed_ws);
