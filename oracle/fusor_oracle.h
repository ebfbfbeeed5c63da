/*
 * fusor_oracle.h — CPU restatement of fusor-ai's quantized matrix-product path.
 *
 * TEST INFRASTRUCTURE ONLY. This is the parity oracle and the CPU baseline, never the product:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only as
 * the checker (or the timed CPU baseline). The product path (fusor-ai_amd/) never links it.
 *
 * Every function restates the x86-64 ("scalar backend") semantics of the Rust reference; the
 * file:line citations are relative to the fusor-ai checkout (crates/kernels/src unless noted).
 * Arithmetic rules it keeps: IEEE f32 division and sqrt, ties-to-even rounding, no fused
 * multiply-add anywhere (built with -ffp-contract=off) except where the reference calls mul_add
 * (exp_fast), saturating float->int casts, float sums in index order from -0.0.
 *
 * What pins each part (tests/test_oracle.py, tests/test_golden.py); the reference is Rust and
 * cannot be built or run here, so nothing is pinned by running it:
 *   layout codec, encode, dequantize_row: the reference's known answers (the ternary byte
 *     0b0001_1000 of tensor.rs:319-330, the subnormal row [127, 64] of matmul.rs:845-856), the
 *     documented position rule, pack/unpack identity, the one-step error bound of
 *     tensor.rs:287-317 and the quantizers' closed forms;
 *   quantize_rows: the closed form (IEEE division, ties-to-even) recomputed in numpy, brute
 *     force on tiny inputs, the invariant sum((u - zp) q) == corr + sum(u q);
 *   matmul: every int32 group accumulator against an int64 brute force; the f32 sums against a
 *     sequential, unfused numpy evaluation and an FMA variant that must differ; the reference
 *     test's own f64 tolerance 1e-4 (1 + |want|) on its own inputs (matmul.rs:809-843);
 *   exp, silu, rms_norm, softmax, rotary angles: closed forms and f64 within stated bounds;
 *   exp_fast, exponentials_apply (tests/test_oracle_attention.py): exp_fast within its stated
 *     6e-5 (ops.rs:137-139) and unlike an unfused evaluation; equal scores summing to their
 *     count exactly; the maximum's exponential 1; the sum against math.fsum of the values;
 *   attend: an independent f64 attention within the Q7b32 stack tolerance over grouped heads,
 *     images, padded sizes and fused operands, and invariance to a shift of every key (the
 *     keys' mean). Its f32 order (the mean, the exponentials' sum) follows the cited code and is
 *     parity unpinned at the bit level: the reference holds no attention fixture;
 *   rng: SplitMix64's published first output and xoshiro256**'s definition;
 *   qwen2 layer and step: an independent f64 evaluation of the same model within the
 *     reference's own tolerance for a Q7b32 stack (3e-2 relative L2, blocks/tests/stacks.rs:49-55).
 *     Their f32 operation order (attention sums, norms, softmax) follows the cited reference
 *     code but is parity unpinned at the bit level: no fixture or known answer of the
 *     reference fixes those bits.
 */
#ifndef FUSOR_ORACLE_H
#define FUSOR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Data types (tensor.rs:19-24). OR_Q8B32 is this build's extension: signed int8 levels in
 * [-127, 127] (zero point 0) in the same quad and scale layout as Q7b32. */
enum {
    OR_F32 = 0,
    OR_Q7B32 = 1,
    OR_Q4B32 = 2,
    OR_T2B128 = 3,
    OR_Q8B32 = 4,
};

/* quant.rs:17-25 */
#define OR_BLOCK 32
#define OR_TERNARY_GROUP 128
#define OR_QUAD 4
#define OR_CHUNK_INPUTS 4
#define OR_WORD 16
#define OR_CHUNKS 8

int or_group(int dtype);
int or_zero_point(int dtype);
int or_codes_per_byte(int dtype);
size_t or_padded_values(size_t rows, size_t cols);
size_t or_quant_len(int dtype, size_t rows, size_t cols);
size_t or_byte_len(int dtype, size_t rows, size_t cols);

/* Quad-layout codec (quant.rs:89-118). */
void or_code_position(int dtype, int lane, int input, size_t *byte, unsigned *shift);
void or_pack_lane(int dtype, int lane, const uint8_t *codes, uint8_t *quad);
void or_unpack_lane(int dtype, const uint8_t *quad, int lane, uint8_t *codes);

/* One group of weights to codes; returns its scale (quant.rs:72-79,143-177). */
float or_quantize_group(int dtype, const float *values, uint8_t *codes);
/* Tensor::encode of a [rows, cols] matrix (tensor.rs:97-143): 0 on success, -1 when cols is
 * not whole groups. `bytes` holds or_byte_len bytes and must be zeroed by the caller. */
int or_encode(int dtype, size_t rows, size_t cols, const float *values, uint8_t *bytes);
/* Matrix::dequantize_row (tensor.rs:247-271). */
void or_dequantize_row(int dtype, size_t rows, size_t cols, const uint8_t *bytes, size_t row,
                       float *out);

/* quantize_rows (matmul.rs:233-257) over `count` values, whole groups of the weights' format. */
void or_quantize_rows(const float *x, size_t count, int dtype, int8_t *quants, float *scales,
                      int32_t *corrections);

/*
 * matmul (matmul.rs:265-317,409-763) of `rows` activation rows (already quantized for `dtype`)
 * against a [n_rows, cols] quantized table, for output columns [col_begin, col_end) in whole
 * quads. out[r * ld_out + (c - col_begin)] = the quad lane's f32 sum, plus bias[c] when `bias`
 * is not NULL (linear.rs:63-68). When `dots` is not NULL it also receives every group's int32
 * accumulator: dots[(r * (col_end - col_begin) + (c - col_begin)) * groups + g].
 * Returns -1 on a shape error.
 */
int or_matmul(int dtype, size_t n_rows, size_t cols, const uint8_t *bytes, const int8_t *quants,
              const float *scales, const int32_t *corrections, size_t rows, size_t col_begin,
              size_t col_end, const float *bias, float *out, size_t ld_out, int32_t *dots);

/* or_matmul with the reference's NEON backend arithmetic when `fused` is set: each group's total
 * scaled with one fused multiply-add, s = fmaf((float)D, cs * row_scale, s) (arch/neon.rs:140-154),
 * in the same group order. */
int or_matmul_fused(int dtype, size_t n_rows, size_t cols, const uint8_t *bytes, const int8_t *quants,
                    const float *scales, const int32_t *corrections, size_t rows, size_t col_begin,
                    size_t col_end, const float *bias, float *out, size_t ld_out, int32_t *dots, int fused);

/* or_matmul over `threads` threads: columns split by 16 (linear.rs:113-119), or by rows when
 * rows >= outputs (conv.rs:584-589). Used for the CPU baseline only. */
int or_matmul_threaded(int dtype, size_t n_rows, size_t cols, const uint8_t *bytes,
                       const int8_t *quants, const float *scales, const int32_t *corrections,
                       size_t rows, const float *bias, float *out, int threads);

/* f32 operations (ops.rs). */
float or_exp(float x);                                   /* ops.rs:121-131 */
float or_silu(float x);                                  /* ops.rs:272-274 */
float or_exp_fast(float x);                              /* ops.rs:137-153 */
/* Exponentials::apply (ops.rs:168-191), scalar backend: scores replaced by their exponentials
 * less the maximum (fast: exp_fast, else exp); returns their sum in the backend's order. */
float or_exponentials_apply(float *scores, size_t n, int fast);
float or_dot_f32(const float *a, const float *b, size_t n); /* scalar.rs:340-342 */
void or_rms_norm(const float *x, const float *weight, size_t dim, float eps, float *out);
void or_rope_inv_freq(float base, size_t head_dim, float *inv_freq);     /* ops.rs:70-74 */
void or_rope_angles(const float *inv_freq, size_t half, size_t position, float *cos_out,
                    float *sin_out);                                     /* rotary.rs angles */
void or_rope_half(float *head, size_t dim, const float *cos_v, const float *sin_v);
void or_softmax(float *scores, size_t n);                                /* ops.rs:301-306 */
void or_weigh(float *scores, size_t n, const float *values, size_t stride, size_t dim,
              float *out);                                                 /* ops.rs:329-342 */

/* Seeded generator (rng.rs:10-52): SplitMix64-seeded xoshiro256**, Box-Muller normals. */
typedef struct {
    uint64_t s[4];
} or_rng;
void or_rng_new(or_rng *rng, uint64_t seed);
uint64_t or_rng_next_u64(or_rng *rng);
double or_rng_uniform(or_rng *rng);
void or_rng_fill_normal(or_rng *rng, float *out, size_t n);

/* The Qwen2 decoder step of blocks::transformer/lm with rows = 1 (layer.rs:161-344,
 * transformer.rs:185-219, lm.rs:147-179). Weights are reference Table bytes. */
typedef struct {
    size_t hidden, layers, heads, kv_heads, head_dim, ffn, vocab, capacity;
    float rope_base, eps;
    int dtype;
} or_qwen2_shape;

typedef struct {
    const float *norm1, *norm2;
    const uint8_t *qkv, *o, *gate, *up, *down;
    const float *qkv_bias; /* NULL for none */
} or_qwen2_layer;

/* One layer over hidden[hidden] at `position`, keeping K and V rows in the caches
 * ([layers][kv_heads][capacity][head_dim] f32 each). */
int or_qwen2_layer_forward(const or_qwen2_shape *shape, const or_qwen2_layer *layer,
                           size_t layer_index, float *kcache, float *vcache, size_t position,
                           const float *cos_v, const float *sin_v, float *hidden, int threads);
/* Embedding of `token` (the tied table's row), every layer, the final norm, the logits over the
 * vocabulary and the greedy token. logits may be NULL (then next_token is not set). */
int or_qwen2_step(const or_qwen2_shape *shape, const or_qwen2_layer *layers,
                  const float *final_norm, const uint8_t *table, float *kcache, float *vcache,
                  int token, size_t position, float *hidden_out, float *logits, int *next_token,
                  int threads);
int or_greedy(const float *logits, size_t n); /* lm.rs:169-179 */
/* Lm::embed (lm.rs:97-108): the table's rows of `ids`, count x hidden, into `out`. */
void or_qwen2_embed(const or_qwen2_shape *shape, const uint8_t *table, const int *ids, size_t count, float *out);
/* Reader::read (lm.rs:205-228) with sequential positions: `count` rows of embeddings (count x
 * hidden) from position `first`, `chunk` rows per call of the stack, each call running every layer
 * over its rows (transformer.rs:294-341, Mask::Causal); then for the last row the final norm, the
 * logits and the greedy token (Prediction::predict, lm.rs:147-166). hidden_out (the last row's
 * residual stream), logits and next_token may be NULL. Returns -1 when the cache does not hold
 * every key the rows see (transformer.rs:329-341). */
int or_qwen2_read(const or_qwen2_shape *shape, const or_qwen2_layer *layers, const float *final_norm,
                  const uint8_t *table, float *kcache, float *vcache, const float *embeddings, size_t count,
                  size_t first, size_t chunk, float *hidden_out, float *logits, int *next_token, int threads);

/* One int8 attention call (blocks/src/attention.rs:35-47): head h of row r of an operand is the
 * head_dim values at r * stride + offset + h * head_dim; `images` images of `queries` query rows
 * over `keys` key and value rows; query heads share key heads in consecutive runs. */
typedef struct {
    size_t heads, kv_heads, head_dim, images, queries, keys;
    const float *query;
    size_t query_stride, query_offset;
    const float *key;
    size_t key_stride, key_offset;
    const float *value;
    size_t value_stride, value_offset;
    int fast; /* Exponentials::Fast, else Exact */
} or_attention;
/* attention::attend (attention.rs:81-214) into out [images * queries][heads * head_dim]. */
int or_attend(const or_attention *call, float *out);

#ifdef __cplusplus
}
#endif

#endif
