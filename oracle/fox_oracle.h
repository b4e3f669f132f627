/*
 * fox_oracle.h -- CPU restatement of RustFox's per-token decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the oracle: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only to compute the expected answer.  Nothing in rustfox_amd/ links,
 * loads or calls it; the product path fails loudly when its HIP library is
 * missing instead of falling back to this code.
 *
 * Every function restates the semantics of one reference routine (cited as
 * file:line into the RustFox sources) with plain C11 scalar code, compiled
 * with -ffp-contract=off so that each float operation rounds exactly once,
 * as in the reference built without FMA contraction (FOX_NATIVE=OFF).
 *
 * Parity pinning (see tests/test_oracle.py):
 *   - block sums and decoders: closed forms and known answers of
 *     tests/test_ternary.c and tests/test_kernels.c, a textbook base-3 /
 *     nibble decoder written independently in the test, brute force on
 *     tiny inputs, and bit equality with the reference compiled from its
 *     own sources (oracle/_ref) on seeded data;
 *   - gemv / quantiser: known answers of tests/test_gemv.c and bit
 *     equality with oracle/_ref;
 *   - ops and forward: bit equality with oracle/_ref end to end (logits
 *     of seeded GGUF models, greedy ids).  Where oracle/_ref is absent the
 *     committed fixtures under tests/golden/ take its place.
 */
#ifndef FOX_ORACLE_H
#define FOX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids used on the path (include/fox/fox.h:213-224) */
enum {
    OR_F32 = 0, OR_F16 = 1, OR_Q4_0 = 2, OR_Q8_0 = 8, OR_Q4_K = 12, OR_Q5_K = 13, OR_Q6_K = 14,
    OR_TQ1_0 = 34, OR_TQ2_0 = 35
};

/* status codes, same numbering as fox_status (include/fox/fox.h:17-26) */
enum { OR_OK = 0, OR_ERR_ARG = 1, OR_ERR_NOMEM = 3, OR_ERR_UNSUPPORTED = 5 };

float    or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);

size_t   or_block_elems(int type);
size_t   or_block_bytes(int type);
size_t   or_row_bytes(int type, size_t n_cols);

int  or_quantize_act_i8(const float *x, size_t n, int8_t *q, float *scale);
void or_quantize_act_k(const float *x, size_t n, int8_t *q, float *scales);

int32_t or_tq1_block_sum(const int8_t *x, const uint8_t *blk);
int32_t or_tq2_block_sum(const int8_t *x, const uint8_t *blk);
void    or_q4k_block_sums(const int8_t *x, const uint8_t *blk,
                          int32_t dots[8], int32_t sums[8]);
void    or_q6k_block_sums(const int8_t *x, const uint8_t *blk, int32_t g[4]);

/* per (row, block) integer sums of a whole matrix, the quantities the GPU
 * debug entry point reports: TQ -> 1 per block; Q4_K -> 8 (dots), Q6_K -> 4 */
int or_block_sums(int type, const int8_t *q, const void *w, size_t rows,
                  size_t cols, int32_t *out);

int or_gemv_tq_i8(int type, const int8_t *q, float act_scale, const void *w,
                  size_t rows, size_t cols, float *out);
int or_gemv_qk_i8(int type, const int8_t *q, const float *ascale,
                  const void *w, size_t rows, size_t cols, float *out);
int or_gemv(int type, const float *x, const void *w, size_t rows, size_t cols,
            float *out, int n_threads);
int or_dequant_row(int type, const void *row, size_t n, float *out);

void  or_rmsnorm(float *out, const float *x, const float *w, size_t n, float eps);
void  or_softmax(float *x, size_t n);
void  or_silu_mul(float *gate, const float *up, size_t n);
void  or_add(float *dst, const float *src, size_t n);
void  or_rope(float *vec, size_t n_heads, size_t head_dim,
              const float *cos_row, const float *sin_row);
float or_dot_f32(const float *a, const float *b, size_t n);
void  or_rope_tables(float *cos_t, float *sin_t, size_t n_ctx,
                     size_t head_dim, float freq_base);
uint32_t or_argmax(const float *logits, size_t n);

/* ---- forward pass (src/forward.c) over caller-held tensor bytes ---- */

typedef struct {
    const void *data;
    int         type;
} or_tensor;

typedef struct {
    or_tensor attn_norm, attn_q, attn_k, attn_v, attn_out;
    or_tensor ffn_norm, ffn_gate, ffn_up, ffn_down;
} or_layer;

typedef struct {
    uint32_t n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab;
    float    rms_eps, rope_base;
    or_tensor token_embd, output_norm, output;
    const or_layer *layers;
} or_model;

typedef struct or_context or_context;

int   or_context_create(const or_model *m, uint32_t n_ctx, uint32_t n_batch,
                        int n_threads, or_context **out);
void  or_context_destroy(or_context *c);
void  or_context_reset(or_context *c);
int   or_eval(or_context *c, const uint32_t *tokens, size_t n, float **logits);
uint32_t or_context_pos(const or_context *c);
/* overwrite rows [p0, p0+n) of one layer's K and V cache (kv_dim floats per
 * row) and set the position: the reference has no such entry point, this is
 * how the tests reproduce a pre-filled cache */
int   or_context_set_kv(or_context *c, uint32_t layer, uint32_t p0, uint32_t n,
                        const float *k, const float *v);
int   or_context_set_pos(or_context *c, uint32_t pos);

#ifdef __cplusplus
}
#endif
#endif
