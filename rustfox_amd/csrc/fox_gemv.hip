// fox_gemv.hip -- activation quantisation and the quantised GEMVs on gfx950.
//
// Exactness contract (RustFox src/gemv.c, src/ternary.c, src/kernels.c):
//   * int8 activations are bit-identical to fox_quantize_activations_i8
//     (gemv.c:11-42) / quantize_activations_k (kernels.c:722-754): this file
//     is built with -ffp-contract=off, 127/amax and amax/127 are correctly
//     rounded (computed in double, which rounds innocuously for a float
//     quotient), v +/- 0.5f is rounded once and truncated;
//   * per-block integer sums are exact (integer MFMA);
//   * every output row combines its per-block terms in block order into a
//     float accumulator starting at 0.0f with one rounding per operation, as
//     the reference's row loop does (ternary.c:226-246, 303-325, kernels.c:571-661),
//     so outputs equal the reference built without FMA contraction.
//
// Work split: one workgroup (4 waves) per 16-row tile and segment; waves take
// 256-element blocks round-robin; each block is one 16 x 256 slab reduced by
// four v_mfma_i32_16x16x64_i8, the token dimension (M <= 8) riding in the
// MFMA's 16 columns.  Per-block float terms go to LDS and 16*M lanes add them
// in block order.
//
// TQ1_0 tensors are held as TQ2_0 blocks of the same trits (the upload
// converts them), so they run the TQ2_0 kernels: each 2-bit code is one
// MFMA A byte, and the -1 of every trit is the block sum of activations.
#include "fox_gemv_dev.h"

#include <cstring>
#include <new>

// waves of the unfused block kernel: a wave's blocks run one after another,
// each waiting for its loads, so more waves per tile keep more loads in
// flight (8 tokens: TQ1_0 5376 x 21504 48.3 -> 35.7 us, 4096 x 14336 30.5 ->
// 21.7 us, Q6_K 4096 x 14336 151 -> 93 us with 8 waves against 4; 16 waves
// were slower at 21504).  Q4_K keeps 4 (14336 x 4096: 53.4 us, 56.8 with 8).
__host__ __device__ constexpr int blk_waves(int fmt)
{
    return fmt == FMT_Q4K ? 4 : 8;
}

// ---------------------------------------------------- activation prep

// Workgroup (x, t) takes blocks [x AP_BLOCKS, ...) of token t: quantise (or
// copy a given q) its slice, then lay the int8 values out as the MFMA B
// operand of format FMT plus per-block integer sums.  The per-256 scales of
// the K-quants depend on one block each; the per-vector scale of the ternary
// formats depends on the whole token, so every workgroup first takes the
// amax over all of it (a read of K floats, shared through L2).
#define AP_BLOCKS 8
template <int FMT>
__global__ __launch_bounds__(512) void act_prep(const float *__restrict__ x, int x_stride,
                                               int K, int M, const int8_t *__restrict__ q_in,
                                               const float *__restrict__ scale_in,
                                               int8_t *__restrict__ q_out,
                                               float *__restrict__ scale_out,
                                               uint8_t *__restrict__ B,
                                               int32_t *__restrict__ aux)
{
    __shared__ int8_t qall[AP_BLOCKS * 256];
    __shared__ float red[16];
    const int t = blockIdx.y, tid = threadIdx.x, nthr = blockDim.x;
    const int lane = tid & 63, wave = tid >> 6, nwaves = nthr >> 6;
    const int nb = K >> 8;
    const bool per_block = (FMT == FMT_Q4K || FMT == FMT_Q6K);
    // this workgroup's blocks and elements (a ragged tail of K belongs to the
    // last workgroup: it is quantised, and has no block to go into)
    const int b0 = blockIdx.x * AP_BLOCKS, b1 = min(nb, b0 + AP_BLOCKS);
    const int e0 = b0 * 256, e1 = blockIdx.x + 1 == gridDim.x ? K : b1 * 256;
    int8_t *qbuf = qall - e0;                      // indexed by absolute element, e0 <= i < e1

    if (q_in) {
        for (int i = e0 + tid; i < e1; i += nthr) qbuf[i] = q_in[(size_t)t * K + i];
        if (scale_in && per_block) {
            for (int b = b0 + tid; b < b1; b += nthr) scale_out[(size_t)t * nb + b] = scale_in[(size_t)t * nb + b];
        } else if (scale_in && tid == 0 && blockIdx.x == 0) {
            scale_out[t] = scale_in[t];
        }
    } else if (!per_block) {
        const float *xt = x + (size_t)t * x_stride;
        // (eight reads in flight per thread: one at a time, the K / 512
        // dependent round trips of a 21504-wide token took 14 us)
        float m = 0.0f;
        int i = tid;
        for (; i + 7 * nthr < K; i += 8 * nthr) {
            float a[8];
#pragma unroll
            for (int k = 0; k < 8; k++) a[k] = xt[i + k * nthr];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float v = fabsf(a[k]);
                if (v > m) m = v;
            }
        }
        for (; i < K; i += nthr) {
            float a = fabsf(xt[i]);
            if (a > m) m = a;
        }
        m = wave_max(m);
        if (lane == 0) red[wave] = m;
        __syncthreads();
        if (tid == 0) {
            float a = 0.0f;
            for (int w = 0; w < nwaves; w++) if (red[w] > a) a = red[w];
            red[15] = a;
        }
        __syncthreads();
        float amax = red[15];
        if (!(amax > 0.0f)) {
            for (int i = e0 + tid; i < e1; i += nthr) qbuf[i] = 0;
            if (tid == 0 && blockIdx.x == 0) scale_out[t] = 0.0f;
        } else {
            float inv = (float)(127.0 / (double)amax);
            for (int i = e0 + tid; i < e1; i += nthr) qbuf[i] = quant_one(xt[i], inv);
            if (tid == 0 && blockIdx.x == 0) scale_out[t] = (float)((double)amax / 127.0);
        }
    } else {
        const float *xt = x + (size_t)t * x_stride;
        for (int b = b0 + wave; b < b1; b += nwaves) {
            float v[4], m = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                v[e] = xt[b * 256 + e * 64 + lane];
                float a = fabsf(v[e]);
                if (a > m) m = a;
            }
            m = wave_max(m);
            if (!(m > 0.0f)) {
#pragma unroll
                for (int e = 0; e < 4; e++) qbuf[b * 256 + e * 64 + lane] = 0;
                if (lane == 0) scale_out[(size_t)t * nb + b] = 0.0f;
            } else {
                float inv = (float)(127.0 / (double)m);
#pragma unroll
                for (int e = 0; e < 4; e++) qbuf[b * 256 + e * 64 + lane] = quant_one(v[e], inv);
                if (lane == 0) scale_out[(size_t)t * nb + b] = (float)((double)m / 127.0);
            }
        }
    }
    __syncthreads();
    if (q_out && !q_in)
        for (int i = e0 + tid; i < e1; i += nthr) q_out[(size_t)t * K + i] = qbuf[i];

    // ---- B operand
    if (FMT == FMT_TQ2) {
        const int items = (b1 - b0) * 16;  // (b, u, g)
        for (int it = tid; it < items; it += nthr) {
            int g = it & 3, u = (it >> 2) & 3, b = b0 + (it >> 4);
            uint32_t w4[4];
#pragma unroll
            for (int l = 0; l < 4; l++) {
                uint32_t d = 0;
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    int m = 16 * g + 4 * u + p;
                    int e = (m >> 5) * 128 + l * 32 + (m & 31);
                    d |= (uint32_t)(uint8_t)qbuf[b * 256 + e] << (8 * p);
                }
                w4[l] = d;
            }
            size_t off = ((((size_t)b * 4 + u) * 4 + g) * M + t) * 16;
            *(uint4 *)(B + off) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        }
        for (int b = b0 + wave; b < b1; b += nwaves) {
            const int8_t *qb = qbuf + b * 256;
            int a = wave_sum_i(qb[lane] + qb[lane + 64] + qb[lane + 128] + qb[lane + 192]);
            if (lane == 0) aux[(size_t)b * M + t] = -a;
        }
    } else if (FMT == FMT_Q4K) {
        const int items = (b1 - b0) * 32;  // (b, p, g, c)
        for (int it = tid; it < items; it += nthr) {
            int c = it & 1, g = (it >> 1) & 3, p = (it >> 3) & 3, b = b0 + (it >> 5);
            const int8_t *src = qbuf + b * 256 + 64 * p + 32 * c + 8 * g;
            uint32_t lo0 = 0, lo1 = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                lo0 |= (uint32_t)(uint8_t)src[e] << (8 * e);
                lo1 |= (uint32_t)(uint8_t)src[4 + e] << (8 * e);
            }
            uint4 v = c == 0 ? make_uint4(lo0, lo1, 0u, 0u) : make_uint4(0u, 0u, lo0, lo1);
            size_t off = ((((size_t)b * 4 + p) * 4 + g) * (2 * M) + 2 * t + c) * 16;
            *(uint4 *)(B + off) = v;
        }
        for (int it = b0 * 8 + wave; it < b1 * 8; it += nwaves) {
            int b = it >> 3, j = it & 7;
            int a = lane < 32 ? qbuf[b * 256 + 32 * j + lane] : 0;
            a = wave_sum_i(a);
            if (lane == 0) aux[((size_t)b * 8 + j) * M + t] = a;
        }
    } else {  // FMT_Q6K: diagonal blocks only
        const int items = (b1 - b0) * 16;  // (b, v, g)
        for (int it = tid; it < items; it += nthr) {
            int g = it & 3, v = (it >> 2) & 3, b = b0 + (it >> 4);
            int h = v >> 1, s = v & 1;
            const int8_t *src = qbuf + b * 256 + 128 * h + 32 * g + 16 * s;
            uint32_t w4[4];
#pragma unroll
            for (int w = 0; w < 4; w++) {
                uint32_t d = 0;
#pragma unroll
                for (int p = 0; p < 4; p++) d |= (uint32_t)(uint8_t)src[4 * w + p] << (8 * p);
                w4[w] = d;
            }
            size_t off = ((((size_t)b * 4 + v) * 4 + g) * M + t) * 16;
            *(uint4 *)(B + off) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        }
        for (int it = b0 * 16 + wave; it < b1 * 16; it += nwaves) {
            int b = it >> 4, v = (it >> 2) & 3, g = it & 3;
            int h = v >> 1, s = v & 1;
            int a = lane < 16 ? qbuf[b * 256 + 128 * h + 32 * g + 16 * s + lane] : 0;
            a = wave_sum_i(a);
            if (lane == 0) aux[((((size_t)b * 4 + v) * 4) + g) * M + t] = a;
        }
    }
}

// ------------------------------------------------------------------ GEMV

struct Segs {
    const uint8_t *w[MAX_SEGS];
    float *out[MAX_SEGS];
    int out_stride[MAX_SEGS];
    int n_rows[MAX_SEGS];
    int tile_start[MAX_SEGS + 1];
    int n;
};

// Process block b of the tile at `ch` (its chunk) for one wave; writes the
// block's float terms (or integer sums) of rows 4g+r.
template <int FMT>
__device__ __forceinline__ void gemv_block(const uint8_t *__restrict__ ch, int b, int nb,
                                           int M, int lane, const uint8_t *__restrict__ B,
                                           const int32_t *__restrict__ aux,
                                           const float *__restrict__ scale,
                                           float *__restrict__ terms /* [T][16][M] */,
                                           int32_t *__restrict__ sums, int row0, int n_rows)
{
    const int g = lane >> 4, j = lane & 15;
    const v4i zero = {0, 0, 0, 0};

    if (FMT == FMT_TQ2) {
        uint4 qs = *(const uint4 *)(ch + 16 * lane);
        uint2 dd = *(const uint2 *)(ch + 1024 + 8 * g);
        const bool bok = j < M;
        // (lanes past the M tokens read the last token's column, unused:
        // with no lane-dependent branch the four B reads issue together)
        const int jc = bok ? j : M - 1;
        uint32_t dw[4] = {qs.x, qs.y, qs.z, qs.w};
        v4i acc = zero;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            v4i bv = *(const v4i *)(B + ((((size_t)b * 4 + u) * 4 + g) * M + jc) * 16);
            uint32_t d = dw[u];
            acc = mfma(d & 0x03030303u, (d >> 2) & 0x03030303u, (d >> 4) & 0x03030303u,
                       (d >> 6) & 0x03030303u, bv, acc);
        }
        if (bok) {
            int t = j;
            int corr = aux[(size_t)b * M + t];
            uint32_t hw[2] = {dd.x, dd.y};
#pragma unroll
            for (int r = 0; r < 4; r++) {
                int S = acc[r] + corr;
                int row = 4 * g + r;
                if (sums) {
                    if (row0 + row < n_rows) sums[((size_t)t * n_rows + row0 + row) * nb + b] = S;
                } else {
                    float d = half_bits_to_float((hw[r >> 1] >> (16 * (r & 1))) & 0xFFFFu);
                    terms[row * M + t] = d * (float)S;
                }
            }
        }
    } else if (FMT == FMT_Q4K) {
        const uint4 *qp = (const uint4 *)(ch + 32 * lane);
        uint4 q0 = qp[0], q1 = qp[1];
        uint32_t dw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const bool bok = j < 2 * M;
        const int jc = bok ? j : 2 * M - 1;                // (as for TQ2_0)
        v4i acc[4];
#pragma unroll
        for (int p = 0; p < 4; p++) {
            v4i bv = *(const v4i *)(B + ((((size_t)b * 4 + p) * 4 + g) * (2 * M) + jc) * 16);
            uint32_t a0 = dw[2 * p], a1 = dw[2 * p + 1];
            acc[p] = mfma(a0 & 0x0F0F0F0Fu, a1 & 0x0F0F0F0Fu, (a0 >> 4) & 0x0F0F0F0Fu,
                          (a1 >> 4) & 0x0F0F0F0Fu, bv, zero);
        }
        if (bok) {
            const int t = j >> 1, c = j & 1;
            const float as = sums ? 0.0f : scale[(size_t)t * nb + b];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = 4 * g + r;
                const uint8_t *hd = ch + 2048 + 16 * row;
                uint4 h4 = *(const uint4 *)hd;
                uint32_t hb[4] = {h4.x, h4.y, h4.z, h4.w};
                const uint8_t *sb = (const uint8_t *)hb + 4;  // scales[12]
                float d = half_bits_to_float(hb[0] & 0xFFFFu);
                float dmin = half_bits_to_float(hb[0] >> 16);
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    const int sj = 2 * p + c;  // src/kernels.c:246-255
                    int sc, mn;
                    if (sj < 4) {
                        sc = sb[sj] & 63;
                        mn = sb[sj + 4] & 63;
                    } else {
                        sc = (sb[sj + 4] & 0x0F) | ((sb[sj - 4] >> 6) << 4);
                        mn = (sb[sj + 4] >> 4) | ((sb[sj] >> 6) << 4);
                    }
                    int D = acc[p][r];
                    if (sums) {
                        if (row0 + row < n_rows)
                            sums[(((size_t)t * n_rows + row0 + row) * nb + b) * 8 + sj] = D;
                    } else {
                        int sq = aux[((size_t)b * 8 + sj) * M + t];
                        float tv = d * (float)sc * (float)D - dmin * (float)mn * (float)sq;
                        terms[(sj * 16 + row) * M + t] = as * tv;
                    }
                }
            }
        }
    } else {  // FMT_Q6K
        const int i = lane & 15;
        const uint8_t *ql = ch + 128 * i;
        const uint8_t *qh = ch + 2048 + 64 * i;
        uint32_t a[4][4];
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int h = v >> 1, s = v & 1;
            uint4 L4 = *(const uint4 *)(ql + 64 * h + 32 * (g & 1) + 16 * s);
            uint4 H4 = *(const uint4 *)(qh + 32 * h + 16 * s);
            uint32_t Lw[4] = {L4.x, L4.y, L4.z, L4.w}, Hw[4] = {H4.x, H4.y, H4.z, H4.w};
#pragma unroll
            for (int w = 0; w < 4; w++) {
                uint32_t nib = (g < 2 ? Lw[w] : Lw[w] >> 4) & 0x0F0F0F0Fu;
                uint32_t hi = ((Hw[w] >> (2 * g)) & 0x03030303u) << 4;
                a[v][w] = nib | hi;
            }
        }
        for (int t0 = 0; t0 < M; t0 += 4) {
            const int c = j & 3, t = t0 + (j >> 2);
            const bool bok = t < M && c == g;
            v4i acc[4];
#pragma unroll
            for (int v = 0; v < 4; v++) {
                v4i bv = load_b(B + ((((size_t)b * 4 + v) * 4 + g) * M + t) * 16, bok);
                acc[v] = mfma(a[v][0], a[v][1], a[v][2], a[v][3], bv, zero);
            }
            const bool tok = t < M;
            const float as = (!tok || sums) ? 0.0f : scale[(size_t)t * nb + b];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = 4 * g + r;
                uint4 s4 = *(const uint4 *)(ch + 3072 + 16 * row);
                uint32_t sw[4] = {s4.x, s4.y, s4.z, s4.w};
                const int8_t *sc = (const int8_t *)sw;
                float d = half_bits_to_float(*(const unsigned short *)(ch + 3328 + 2 * row));
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int h = v >> 1, s = v & 1;
                    int part = 0;
                    if (tok) {
                        int as16 = aux[((((size_t)b * 4 + v) * 4) + c) * M + t];
                        part = (int)sc[8 * h + s + 2 * c] * (acc[v][r] - 32 * as16);
                    }
                    part += __shfl_xor(part, 1);
                    part += __shfl_xor(part, 2);
                    if (tok && c == 0) {
                        if (sums) {
                            if (row0 + row < n_rows)
                                sums[(((size_t)t * n_rows + row0 + row) * nb + b) * 4 + v] = part;
                        } else {
                            terms[(v * 16 + row) * M + t] = as * d * (float)part;
                        }
                    }
                }
            }
        }
    }
}

template <int FMT>
__global__ __launch_bounds__(blk_waves(FMT) * 64) void gemv_blocks(
    Segs segs, int nb, int M, int chunk_blocks, const uint8_t *__restrict__ B,
    const int32_t *__restrict__ aux, const float *__restrict__ scale, unsigned flags,
    int32_t *__restrict__ sums)
{
    extern __shared__ float terms[];  // [chunk_blocks][T][16][M]
    constexpr int T = terms_per_block(FMT);
    constexpr int CHUNK = FMT == FMT_TQ2 ? TQ2_CHUNK : FMT == FMT_Q4K ? Q4K_CHUNK : Q6K_CHUNK;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    int s = 0;
    while (s + 1 < segs.n && (int)blockIdx.x >= segs.tile_start[s + 1]) s++;
    const int tile = blockIdx.x - segs.tile_start[s];
    const int n_rows = segs.n_rows[s];
    const uint8_t *wt = segs.w[s] + (size_t)tile * nb * CHUNK;

    const bool combiner = tid < 16 * M;
    const int crow = tid & 15, ct = tid >> 4;
    float acc = 0.0f;

    for (int c0 = 0; c0 < nb; c0 += chunk_blocks) {
        const int c1 = c0 + chunk_blocks < nb ? c0 + chunk_blocks : nb;
        for (int b = c0 + wave; b < c1; b += blk_waves(FMT))
            gemv_block<FMT>(wt + (size_t)b * CHUNK, b, nb, M, lane, B, aux, scale,
                            terms + (size_t)(b - c0) * T * 16 * M, sums, tile * 16, n_rows);
        if (sums) continue;
        __syncthreads();
        if (combiner) {
            for (int b = c0; b < c1; b++) {
                const float *tb = terms + (size_t)(b - c0) * T * 16 * M;
#pragma unroll
                for (int k = 0; k < T; k++) acc = acc + tb[(k * 16 + crow) * M + ct];
            }
        }
        __syncthreads();
    }
    if (sums || !combiner) return;
    const int row = tile * 16 + crow;
    if (row >= n_rows) return;
    float y = FMT == FMT_TQ2 ? acc * scale[ct] : acc;  // src/gemv.c:70
    float *o = segs.out[s] + (size_t)ct * segs.out_stride[s] + row;
    *o = (flags & FOX_GPU_GEMV_ACCUMULATE) ? *o + y : y;
}

// -------------------------------------------------------- float weights

// F16 / F32 rows (src/kernels.c:81-96): each lane owns one row and adds
// w[k] * x[k] sequentially in k, exactly the reference's order.  A
// workgroup owns one 256-row tile of the tiled float layout.  Its chunks
// (128 bytes of every row, 32 KB contiguous) stream through LDS in halves
// (64 bytes of every row per step; rows padded by a dword against bank
// conflicts), double buffered: the next step's loads are in flight while a
// step is summed.  The activations of a step ride along in the same
// buffers.  (Half steps keep a workgroup's LDS near 35 KB, so that every
// tile of a large head is resident at once: with whole chunks only two
// workgroups fit a CU and the last tiles run in a second, mostly idle
// round.)
#define FR 256      // rows per tile of the layout

// RW rows per workgroup (FR, or FR / 2: two workgroups per tile, each
// reading its half of every chunk, which spreads a large head's rows more
// evenly over the compute units)
template <typename WT, int MT, int RW>
__global__ __launch_bounds__(RW) void gemv_float(const WT *__restrict__ W, int K, int N,
                                                 const float *__restrict__ x, int x_stride,
                                                 int M, float *__restrict__ out,
                                                 int out_stride, unsigned flags)
{
    constexpr int FK = 64 / sizeof(WT);                // elements of a step (half a row chunk)
    constexpr int RDW = FK * sizeof(WT) / 4;           // dwords of a row per step
    constexpr int RSTR = RDW + 1;                       // padded row stride
    constexpr int PPR = RDW / 4;                        // 16-byte pieces per row and step
    constexpr int NP = PPR;                             // pieces per thread
    __shared__ uint32_t wl[2][RW * RSTR];
    __shared__ float xs[2][MT * FK];
    if (MT == 1) M = 1;
    const int tid = threadIdx.x;
    const int r0 = blockIdx.x * RW;
    const int nchunk = (K + FK - 1) / FK;               // steps
    const int nch128 = (K + 2 * FK - 1) / (2 * FK);     // 128-byte chunks of the layout
    // this tile's chunks, 32 KB each (rows and columns zero-padded)
    const uint4 *tw = (const uint4 *)W + (size_t)(blockIdx.x / (FR / RW)) * nch128 * (FR * 2 * PPR) +
                      (size_t)(blockIdx.x % (FR / RW)) * RW * 2 * PPR;

    constexpr int XPT = (MT * FK + RW - 1) / RW;        // activations staged per thread
    uint4 R[NP];
    float xr[XPT];
    // global -> registers for chunk c (rows past N and columns past K read 0)
    auto fetch = [&](int c) {
        const int k0 = c * FK, kn = K - k0 < FK ? K - k0 : FK;
        // half c & 1 of chunk c / 2: pieces (row, part) at row * 2 PPR + part
        const uint4 *cw = tw + (size_t)(c >> 1) * (FR * 2 * PPR) + (c & 1) * PPR;
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int pc = tid + i * RW, r = pc / PPR, part = pc - r * PPR;
            R[i] = cw[r * 2 * PPR + part];
        }
#pragma unroll
        for (int v = 0; v < XPT; v++) {
            const int e = tid + v * RW;
            xr[v] = 0.0f;
            if (e < M * FK) {
                const int t = e / FK, kk = e - t * FK;
                if (kk < kn) xr[v] = x[(size_t)t * x_stride + k0 + kk];
            }
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int pc = tid + i * RW, r = pc / PPR, part = pc - r * PPR;
            uint32_t *d = &wl[buf][r * RSTR + part * 4];
            d[0] = R[i].x;
            d[1] = R[i].y;
            d[2] = R[i].z;
            d[3] = R[i].w;
        }
#pragma unroll
        for (int v = 0; v < XPT; v++) {
            const int e = tid + v * RW;
            if (e < M * FK) xs[buf][e] = xr[v];
        }
    };

    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = 0.0f;

    fetch(0);
    stash(0);
    if (nchunk > 1) fetch(1);
    __syncthreads();
    for (int c = 0; c < nchunk; c++) {
        const int buf = c & 1;
        const int kn = K - c * FK < FK ? K - c * FK : FK;
        const uint32_t *myw = &wl[buf][tid * RSTR];
        const float *xb = xs[buf];
        if (kn == FK) {
#pragma unroll 8
            for (int kk = 0; kk < FK; kk++) {
                const uint32_t dword = myw[kk / (4 / (int)sizeof(WT))];
                float w;
                if (sizeof(WT) == 2)
                    w = half_bits_to_float((dword >> (16 * (kk & 1))) & 0xFFFFu);
                else
                    w = __builtin_bit_cast(float, dword);
#pragma unroll
                for (int t = 0; t < MT; t++)
                    if (t < M) acc[t] = acc[t] + w * xb[t * FK + kk];
            }
        } else {
            for (int kk = 0; kk < kn; kk++) {
                const uint32_t dword = myw[kk / (4 / (int)sizeof(WT))];
                float w;
                if (sizeof(WT) == 2)
                    w = half_bits_to_float((dword >> (16 * (kk & 1))) & 0xFFFFu);
                else
                    w = __builtin_bit_cast(float, dword);
#pragma unroll
                for (int t = 0; t < MT; t++)
                    if (t < M) acc[t] = acc[t] + w * xb[t * FK + kk];
            }
        }
        if (c + 1 < nchunk) {
            // the other buffer was last read before the previous barrier
            stash(buf ^ 1);
            if (c + 2 < nchunk) fetch(c + 2);
        }
        __syncthreads();
    }
    const int row = r0 + tid;
    if (row >= N) return;
#pragma unroll
    for (int t = 0; t < MT; t++) {
        if (t >= M) break;
        float *o = out + (size_t)t * out_stride + row;
        *o = (flags & FOX_GPU_GEMV_ACCUMULATE) ? *o + acc[t] : acc[t];
    }
}

// ----------------------------------------------------------------- host

static size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct Ws {
    int8_t *q;
    float *scale;
    uint8_t *B;
    int32_t *aux;
};

// layout of the activation buffers of one format; returns the byte count
static size_t act_layout(int fmt, size_t K, size_t M, uint8_t *base, Ws *w)
{
    const size_t nb = K / 256;
    size_t off = 0, oq, os, ob, oa;
    oq = off; off = align_up(off + M * K, 256);
    os = off; off = align_up(off + M * (nb ? nb : 1) * 4, 256);
    ob = off; off = align_up(off + nb * M * (size_t)b_bytes_per_block_tok(fmt), 256);
    oa = off; off = align_up(off + nb * M * (size_t)aux_per_block_tok(fmt) * 4, 256);
    if (w) {
        w->q = (int8_t *)(base + oq);
        w->scale = (float *)(base + os);
        w->B = base + ob;
        w->aux = (int32_t *)(base + oa);
    }
    return off;
}

static fox_gpu_status carve(fox_gpu_ctx *ctx, int fmt, size_t K, size_t M, Ws *w)
{
    fox_gpu_status st = fox_ws_reserve(ctx, act_layout(fmt, K, M, nullptr, nullptr));
    if (st) return st;
    act_layout(fmt, K, M, ctx->ws, w);
    return FOX_GPU_OK;
}

static fox_gpu_status launch_prep(fox_gpu_ctx *ctx, int fmt, const float *x, size_t x_stride,
                                  const int8_t *q_in, const float *scale_in, size_t K,
                                  size_t M, const Ws &w, int8_t *q_out, float *scale_out)
{
    // workgroups of AP_BLOCKS blocks (AP_BLOCKS * 256 values); a ragged tail
    // of K (values beyond the last whole block) is quantised by the last
    const size_t nwg = (K + AP_BLOCKS * 256 - 1) / (AP_BLOCKS * 256);
    if (K > (1u << 24)) return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "gemv: K = %zu too large", K);
    dim3 grid((unsigned)nwg, (unsigned)M), block(512);
    switch (fmt) {
    case FMT_TQ2:
        hipLaunchKernelGGL(act_prep<FMT_TQ2>, grid, block, 0, ctx->stream, x, (int)x_stride,
                           (int)K, (int)M, q_in, scale_in, q_out, scale_out, w.B, w.aux);
        break;
    case FMT_Q4K:
        hipLaunchKernelGGL(act_prep<FMT_Q4K>, grid, block, 0, ctx->stream, x, (int)x_stride,
                           (int)K, (int)M, q_in, scale_in, q_out, scale_out, w.B, w.aux);
        break;
    default:
        hipLaunchKernelGGL(act_prep<FMT_Q6K>, grid, block, 0, ctx->stream, x, (int)x_stride,
                           (int)K, (int)M, q_in, scale_in, q_out, scale_out, w.B, w.aux);
        break;
    }
    FOX_LAUNCHED("act_prep");
    return FOX_GPU_OK;
}

static fox_gpu_status launch_blocks(fox_gpu_ctx *ctx, int fmt, const Segs &sg, int tiles,
                                    int nb, int M, const Ws &w, unsigned flags, int32_t *sums)
{
    const int T = terms_per_block(fmt);
    int chunk_blocks = (int)(65536 / ((size_t)T * 16 * M * 4));
    const int waves = blk_waves(fmt);
    chunk_blocks = chunk_blocks / waves * waves;
    if (chunk_blocks < waves) chunk_blocks = waves;
    if (chunk_blocks > nb) chunk_blocks = nb;
    size_t lds = sums ? 0 : (size_t)chunk_blocks * T * 16 * M * 4;
    dim3 grid((unsigned)tiles), block(waves * 64);
    switch (fmt) {
    case FMT_TQ2:
        hipLaunchKernelGGL(gemv_blocks<FMT_TQ2>, grid, block, lds, ctx->stream, sg, nb, M,
                           chunk_blocks, w.B, w.aux, w.scale, flags, sums);
        break;
    case FMT_Q4K:
        hipLaunchKernelGGL(gemv_blocks<FMT_Q4K>, grid, block, lds, ctx->stream, sg, nb, M,
                           chunk_blocks, w.B, w.aux, w.scale, flags, sums);
        break;
    default:
        hipLaunchKernelGGL(gemv_blocks<FMT_Q6K>, grid, block, lds, ctx->stream, sg, nb, M,
                           chunk_blocks, w.B, w.aux, w.scale, flags, sums);
        break;
    }
    FOX_LAUNCHED("gemv_blocks");
    return FOX_GPU_OK;
}

static fox_gpu_status check_common(size_t n, const fox_gpu_tensor *const *ws, size_t M,
                                   int *type, size_t *K)
{
    if (!ws || n == 0 || n > MAX_SEGS)
        return fox_fail(FOX_GPU_ERR_ARG, "gemv: 1 to %d matrices per call", MAX_SEGS);
    if (M == 0 || M > FOX_GPU_MAX_TOKENS)
        return fox_fail(FOX_GPU_ERR_ARG, "gemv: %zu tokens; 1 to %d per call", M,
                        FOX_GPU_MAX_TOKENS);
    for (size_t i = 0; i < n; i++) {
        if (!ws[i]) return fox_fail(FOX_GPU_ERR_ARG, "gemv: null tensor");
        if (i && (ws[i]->type != ws[0]->type || ws[i]->ne0 != ws[0]->ne0))
            return fox_fail(FOX_GPU_ERR_ARG,
                            "gemv: matrices of one call must share type and width");
    }
    *type = ws[0]->type;
    *K = (size_t)ws[0]->ne0;
    if (*K > (1u << 20) || ws[0]->ne1 > (1u << 30))
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "gemv: matrix too large");
    return FOX_GPU_OK;
}

// fixed_ws: a caller-provided workspace of fixed_cap bytes used instead of
// the context's growable one (nullptr: the context's)
static fox_gpu_status gemv_launch_ws(fox_gpu_ctx *ctx, size_t n, const fox_gpu_tensor *const *ws,
                                     const float *x, size_t x_stride, const int8_t *q,
                                     const float *scale, size_t M, float *const *outs,
                                     const size_t *out_strides, unsigned flags, int32_t *sums,
                                     uint8_t *fixed_ws, size_t fixed_cap)
{
    int type;
    size_t K;
    fox_gpu_status st;

    if (!ctx) return fox_fail(FOX_GPU_ERR_ARG, "gemv: null context");
    if ((st = check_common(n, ws, M, &type, &K))) return st;
    if (!x && !q) return fox_fail(FOX_GPU_ERR_ARG, "gemv: null activations");
    if (!sums) {
        if (!outs || !out_strides) return fox_fail(FOX_GPU_ERR_ARG, "gemv: null output");
        for (size_t i = 0; i < n; i++) {
            if (!outs[i]) return fox_fail(FOX_GPU_ERR_ARG, "gemv: null output");
            if (M > 1 && out_strides[i] < ws[i]->ne1)
                return fox_fail(FOX_GPU_ERR_ARG, "gemv: output stride %zu < %llu rows",
                                out_strides[i], (unsigned long long)ws[i]->ne1);
        }
    }
    if (x && M > 1 && x_stride < K)
        return fox_fail(FOX_GPU_ERR_ARG, "gemv: input stride %zu < K = %zu", x_stride, K);

    if (type == FOX_GPU_F16 || type == FOX_GPU_F32) {
        if (!x || sums)
            return fox_fail(FOX_GPU_ERR_UNSUPPORTED,
                            "gemv: %s weights take float activations", fox_type_name(type));
        for (size_t i = 0; i < n; i++) {
            const int N = (int)ws[i]->ne1;
            // one token: half-tile workgroups (a 151936-row head is 1187 of
            // them: 4.6 per compute unit, against 2.3 whole tiles)
            constexpr int RH = FR / 2;
            dim3 grid((unsigned)((N + FR - 1) / FR)), block(FR);
            dim3 grid1((unsigned)((N + RH - 1) / RH)), block1(RH);
            const _Float16 *wh = (const _Float16 *)ws[i]->d;
            const float *wf = (const float *)ws[i]->d;
            if (type == FOX_GPU_F16 && M == 1)
                hipLaunchKernelGGL((gemv_float<_Float16, 1, RH>), grid1, block1, 0, ctx->stream, wh,
                                   (int)K, N, x, (int)x_stride, (int)M, outs[i],
                                   (int)out_strides[i], flags);
            else if (type == FOX_GPU_F16)
                hipLaunchKernelGGL((gemv_float<_Float16, FOX_GPU_MAX_TOKENS, FR>), grid, block, 0,
                                   ctx->stream, wh, (int)K, N, x, (int)x_stride, (int)M, outs[i],
                                   (int)out_strides[i], flags);
            else if (M == 1)
                hipLaunchKernelGGL((gemv_float<float, 1, RH>), grid1, block1, 0, ctx->stream, wf,
                                   (int)K, N, x, (int)x_stride, (int)M, outs[i],
                                   (int)out_strides[i], flags);
            else
                hipLaunchKernelGGL((gemv_float<float, FOX_GPU_MAX_TOKENS, FR>), grid, block, 0,
                                   ctx->stream, wf, (int)K, N, x, (int)x_stride, (int)M, outs[i],
                                   (int)out_strides[i], flags);
            FOX_LAUNCHED("gemv_float");
        }
        return FOX_GPU_OK;
    }

    const int fmt = fmt_of(type);
    if (fmt < 0)
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "gemv: no kernel for %s", fox_type_name(type));
    if (K % 256)
        return fox_fail(FOX_GPU_ERR_ARG,
                        "gemv: %zu columns is not a multiple of the 256-element block", K);
    st = fox_fused_gemv(ctx, n, ws, x, x_stride, q, scale, M, outs, out_strides, flags, sums,
                        fixed_ws);
    if (st != FOX_GPU_ERR_UNSUPPORTED) return st;
    Ws w;
    if (fixed_ws) {
        const size_t need = act_layout(fmt, K, M, nullptr, nullptr);
        if (need > fixed_cap)
            return fox_fail(FOX_GPU_ERR_ARG, "gemv: %zu x %zu %s activations need %zu bytes of "
                            "scratch; the fixed scratch holds %zu", M, K, fox_type_name(type),
                            need, fixed_cap);
        act_layout(fmt, K, M, fixed_ws, &w);
    } else if ((st = carve(ctx, fmt, K, M, &w))) {
        return st;
    }
    if ((st = launch_prep(ctx, fmt, x, x_stride, q, scale, K, M, w, w.q, w.scale))) return st;

    Segs sg;
    memset(&sg, 0, sizeof(sg));
    sg.n = (int)n;
    int tiles = 0;
    for (size_t i = 0; i < n; i++) {
        sg.w[i] = ws[i]->d;
        sg.out[i] = outs ? outs[i] : nullptr;
        sg.out_stride[i] = out_strides ? (int)out_strides[i] : 0;
        sg.n_rows[i] = (int)ws[i]->ne1;
        sg.tile_start[i] = tiles;
        tiles += (int)ws[i]->n_tiles;
    }
    sg.tile_start[n] = tiles;
    return launch_blocks(ctx, fmt, sg, tiles, (int)(K / 256), (int)M, w, flags, sums);
}

fox_gpu_status fox_gemv_launch(fox_gpu_ctx *ctx, size_t n, const fox_gpu_tensor *const *ws,
                               const float *x, size_t x_stride, const int8_t *q,
                               const float *scale, size_t M, float *const *outs,
                               const size_t *out_strides, unsigned flags, int32_t *sums)
{
    return gemv_launch_ws(ctx, n, ws, x, x_stride, q, scale, M, outs, out_strides, flags, sums,
                          nullptr, 0);
}

// ------------------------------------------------------ fixed scratch

// The workspace of fox_gpu_gemv_noalloc: a file-scope device array, one
// copy per GPU, alive until the process ends.  Host code never uses its
// name as an address (that is a host-side stand-in); fox_scratch_init
// resolves this device's copy with hipGetSymbolAddress once per context,
// with the device current, and the kernels receive that pointer.
static __device__ __align__(256) uint8_t scratch[FOX_NOALLOC_SCRATCH];

fox_gpu_status fox_scratch_init(fox_gpu_ctx *ctx)
{
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        ctx->scratch = nullptr;
        return fox_fail(FOX_GPU_ERR_INTERNAL, "init: the fixed scratch of device %d has no "
                        "address: %s", ctx->device, hipGetErrorString(e));
    }
    ctx->scratch = (uint8_t *)p;
    return FOX_GPU_OK;
}

// ----------------------------------------------------------- C entries

extern "C" fox_gpu_status fox_gpu_quantize(fox_gpu_ctx *ctx, int mode, const float *x, size_t K,
                                           size_t M, size_t x_stride, int8_t *q, float *scale)
{
    if (!ctx || !x || !q || !scale || K == 0 || M == 0)
        return fox_fail(FOX_GPU_ERR_ARG, "quantize: bad argument");
    if (M > FOX_GPU_MAX_TOKENS)
        return fox_fail(FOX_GPU_ERR_ARG, "quantize: %zu rows; at most %d", M, FOX_GPU_MAX_TOKENS);
    if (M > 1 && x_stride < K) return fox_fail(FOX_GPU_ERR_ARG, "quantize: stride < K");
    if (mode != FOX_GPU_ACT_PER_VECTOR && mode != FOX_GPU_ACT_PER_BLOCK)
        return fox_fail(FOX_GPU_ERR_ARG, "quantize: unknown mode %d", mode);
    if (mode == FOX_GPU_ACT_PER_BLOCK && K % 256)
        return fox_fail(FOX_GPU_ERR_ARG, "quantize: %zu values is not a whole number of "
                        "256-element blocks", K);
    const int fmt = mode == FOX_GPU_ACT_PER_BLOCK ? FMT_Q4K : FMT_TQ2;
    Ws w;
    fox_gpu_status st;
    // the B operand is laid out for whole blocks only; a ragged tail is
    // quantised with the rest but has no block to go into
    size_t Kb = K / 256 * 256;
    if ((st = carve(ctx, fmt, Kb ? Kb : 256, M, &w))) return st;
    return launch_prep(ctx, fmt, x, M > 1 ? x_stride : K, nullptr, nullptr, K, M, w, q, scale);
}

extern "C" fox_gpu_status fox_gpu_gemv(fox_gpu_ctx *ctx, const fox_gpu_tensor *w, const float *x,
                                       size_t x_stride, size_t M, float *out, size_t out_stride,
                                       unsigned flags)
{
    if (!x || !out) return fox_fail(FOX_GPU_ERR_ARG, "gemv: null pointer");
    const fox_gpu_tensor *ws[1] = {w};
    float *outs[1] = {out};
    size_t strides[1] = {M > 1 ? out_stride : (w ? (size_t)w->ne1 : 0)};
    return fox_gemv_launch(ctx, 1, ws, x, M > 1 ? x_stride : (w ? (size_t)w->ne0 : 0), nullptr,
                           nullptr, M, outs, strides, flags, nullptr);
}

// fox_gpu_gemv's computation, its activation workspace the fixed scratch:
// nothing is allocated.  Calls on one device share the scratch (each
// rewrites every byte it reads before reading it), so calls that overlap
// in time on one device race.
extern "C" fox_gpu_status fox_gpu_gemv_noalloc(fox_gpu_ctx *ctx, const fox_gpu_tensor *w,
                                               const float *x, size_t x_stride, size_t M,
                                               float *out, size_t out_stride, unsigned flags)
{
    if (!ctx || !x || !out) return fox_fail(FOX_GPU_ERR_ARG, "gemv_noalloc: null pointer");
    if (!ctx->scratch)
        return fox_fail(FOX_GPU_ERR_INTERNAL, "gemv_noalloc: the context has no fixed scratch");
    const fox_gpu_tensor *ws[1] = {w};
    float *outs[1] = {out};
    size_t strides[1] = {M > 1 ? out_stride : (w ? (size_t)w->ne1 : 0)};
    return gemv_launch_ws(ctx, 1, ws, x, M > 1 ? x_stride : (w ? (size_t)w->ne0 : 0), nullptr,
                          nullptr, M, outs, strides, flags, nullptr, ctx->scratch,
                          FOX_NOALLOC_SCRATCH);
}

extern "C" fox_gpu_status fox_gpu_gemv_multi(fox_gpu_ctx *ctx, size_t n,
                                             const fox_gpu_tensor *const *ws, const float *x,
                                             size_t x_stride, size_t M, float *const *outs,
                                             const size_t *out_strides, unsigned flags)
{
    if (!x || !outs || !out_strides) return fox_fail(FOX_GPU_ERR_ARG, "gemv_multi: null pointer");
    return fox_gemv_launch(ctx, n, ws, x, x_stride, nullptr, nullptr, M, outs, out_strides,
                           flags, nullptr);
}

extern "C" fox_gpu_status fox_gpu_gemv_i8(fox_gpu_ctx *ctx, const fox_gpu_tensor *w,
                                          const int8_t *q, const float *scale, size_t M,
                                          float *out, size_t out_stride)
{
    if (!q || !scale || !out) return fox_fail(FOX_GPU_ERR_ARG, "gemv_i8: null pointer");
    if (w && !fox_is_block_type(w->type))
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "gemv_i8: %s weights have no int8 path",
                        fox_type_name(w->type));
    const fox_gpu_tensor *ws[1] = {w};
    float *outs[1] = {out};
    size_t strides[1] = {M > 1 ? out_stride : (w ? (size_t)w->ne1 : 0)};
    return fox_gemv_launch(ctx, 1, ws, nullptr, 0, q, scale, M, outs, strides, 0, nullptr);
}

extern "C" fox_gpu_status fox_gpu_block_sums(fox_gpu_ctx *ctx, const fox_gpu_tensor *w,
                                             const int8_t *q, size_t M, int32_t *sums)
{
    if (!q || !sums) return fox_fail(FOX_GPU_ERR_ARG, "block_sums: null pointer");
    if (w && !fox_is_block_type(w->type))
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "block_sums: %s has no integer blocks",
                        fox_type_name(w->type));
    const fox_gpu_tensor *ws[1] = {w};
    return fox_gemv_launch(ctx, 1, ws, nullptr, 0, q, nullptr, M, nullptr, nullptr, 0, sums);
}

// ------------------------------------------------------ prepared activations

struct fox_gpu_act {
    int fmt, type;
    size_t K, M;
    uint8_t *buf;
    Ws w;
};

extern "C" fox_gpu_status fox_gpu_act_prepare(fox_gpu_ctx *ctx, int type, const float *x,
                                              size_t K, size_t M, size_t x_stride,
                                              fox_gpu_act **out)
{
    if (!ctx || !x || !out || K == 0 || M == 0)
        return fox_fail(FOX_GPU_ERR_ARG, "act_prepare: bad argument");
    *out = nullptr;
    const int fmt = fmt_of(type);
    if (fmt < 0)
        return fox_fail(FOX_GPU_ERR_UNSUPPORTED, "act_prepare: %s weights read float "
                        "activations directly", fox_type_name(type));
    if (K % 256) return fox_fail(FOX_GPU_ERR_ARG, "act_prepare: K %% 256 != 0");
    if (M > FOX_GPU_MAX_TOKENS) return fox_fail(FOX_GPU_ERR_ARG, "act_prepare: too many tokens");
    if (M > 1 && x_stride < K) return fox_fail(FOX_GPU_ERR_ARG, "act_prepare: stride < K");
    fox_gpu_act *a = new (std::nothrow) fox_gpu_act();
    if (!a) return fox_fail(FOX_GPU_ERR_NOMEM, "act_prepare: handle");
    a->fmt = fmt;
    a->type = type;
    a->K = K;
    a->M = M;
    hipError_t e = hipMalloc(&a->buf, act_layout(fmt, K, M, nullptr, nullptr));
    if (e != hipSuccess) {
        delete a;
        return fox_hip_fail(e, "act_prepare: buffer");
    }
    act_layout(fmt, K, M, a->buf, &a->w);
    fox_gpu_status st = launch_prep(ctx, fmt, x, M > 1 ? x_stride : K, nullptr, nullptr, K, M,
                                    a->w, a->w.q, a->w.scale);
    if (st) {
        fox_gpu_act_free(ctx, a);
        return st;
    }
    *out = a;
    return FOX_GPU_OK;
}

extern "C" fox_gpu_status fox_gpu_gemv_act(fox_gpu_ctx *ctx, const fox_gpu_tensor *w,
                                           const fox_gpu_act *act, float *out,
                                           size_t out_stride, unsigned flags)
{
    if (!ctx || !w || !act || !out) return fox_fail(FOX_GPU_ERR_ARG, "gemv_act: bad argument");
    if (w->type != act->type || w->ne0 != act->K)
        return fox_fail(FOX_GPU_ERR_ARG, "gemv_act: activations were prepared for %s K=%zu, "
                        "the matrix is %s K=%llu", fox_type_name(act->type), act->K,
                        fox_type_name(w->type), (unsigned long long)w->ne0);
    if (act->M > 1 && out_stride < w->ne1)
        return fox_fail(FOX_GPU_ERR_ARG, "gemv_act: output stride < rows");
    Segs sg;
    memset(&sg, 0, sizeof(sg));
    sg.n = 1;
    sg.w[0] = w->d;
    sg.out[0] = out;
    sg.out_stride[0] = act->M > 1 ? (int)out_stride : (int)w->ne1;
    sg.n_rows[0] = (int)w->ne1;
    sg.tile_start[1] = (int)w->n_tiles;
    return launch_blocks(ctx, act->fmt, sg, (int)w->n_tiles, (int)(act->K / 256), (int)act->M,
                         act->w, flags, nullptr);
}

extern "C" void fox_gpu_act_free(fox_gpu_ctx *ctx, fox_gpu_act *a)
{
    if (!a) return;
    if (ctx) (void)hipSetDevice(ctx->device);
    if (a->buf) (void)hipFree(a->buf);
    delete a;
}
