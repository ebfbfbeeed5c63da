/*
 * fusor_gpu.h — the C ABI of the MI355X (gfx950) quantized matrix-product path.
 *
 * These entry points are what fusor-ai's `kernels` crate (crates/kernels/src) would bind through
 * a thin `-sys` crate so that its Rust API stays unchanged: each declaration names the reference
 * interface it replaces (file:line, relative to the fusor-ai checkout). Plain pointers and sizes
 * only. Pointers documented as "device" are HIP device addresses; `stream` is a hipStream_t
 * (NULL is the null stream). Every call returns a status code (FG_OK on success); the message of
 * the last failure on the calling thread is fg_last_error(). No call retains a caller pointer
 * after it returns, except the table and model handles, which own their device memory.
 *
 * Calls are thread-safe, except fg_matmul_noalloc: the reference calls the product from every
 * thread of a team (linear.rs:113-143), and concurrent fg_matmul calls on disjoint outputs are
 * independent. fg_matmul_noalloc shares one scratch array per device among all its calls, so its
 * calls that overlap on a device race and must be serialized by the caller. One model handle
 * (fg_qwen2) or upload (fg_upload) is used by one thread at a time.
 */
#ifndef FUSOR_GPU_H
#define FUSOR_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. The reference panics on shape and format misuse (matmul.rs:271-274,301-304,
 * 531-541; linear.rs:58-61) and returns Error::Format on construction (tensor.rs:97-104,
 * 163-171,200-211); a binding maps FG_ERR_SHAPE / FG_ERR_FORMAT to those. */
#define FG_OK 0
#define FG_ERR_SHAPE 1     /* shapes or ranges that do not fit */
#define FG_ERR_FORMAT 2    /* a data type this call does not take */
#define FG_ERR_HIP 3       /* the HIP runtime failed */
#define FG_ERR_NOMEM 4     /* device memory ran out */
#define FG_ERR_ARG 5       /* a null or otherwise invalid argument */

/* Data types: DType (tensor.rs:19-24). FG_Q8B32 is this library's extension: signed int8 levels
 * in [-127, 127] (zero point 0, one byte per code) in Q7b32's quad and scale layout. */
#define FG_F32 0
#define FG_Q7B32 1
#define FG_Q4B32 2
#define FG_T2B128 3
#define FG_Q8B32 4

/* Flags of fg_matmul. */
#define FG_ACCUMULATE 1 /* out += result: project_residual_input (linear.rs:134-143) */
/* Scale each group's total with one fused multiply-add, s = fma((float)D, fl(ws * as), s), the
 * reference's NEON backend (arch/neon.rs:140-154, vfmaq_f32), instead of the scalar backend's
 * separately rounded s + (float)D * (ws * as) (arch/scalar.rs:80-89). Groups stay in order, so the
 * f32 results are the NEON backend's bits. Rows 1..4 then take the matrix cores too. */
#define FG_FUSED_SCALE 2
/* One row only: sum each output's group terms fl(fl((float)D) * fl(ws * as)) in parallel, a team of
 * lanes over strided terms then a lane reduction, instead of in group order. This is the order
 * fg_qwen2 uses when it is not exact (an inspection of that reduction, not a reference backend):
 * the terms are the scalar backend's, only their additions are reordered, so each output is
 * within (G - 1) * 2^-24 * sum_g |term_g| of the scalar backend's (G groups). Not with
 * FG_FUSED_SCALE, not for T2b128. */
#define FG_PARALLEL_SUM 4

/* The last failure's message on this thread ("" when none). */
const char *fg_last_error(void);

/* Library version, for a binding's build check. */
int fg_version(void);

/* ----------------------------------------------------------------------------- tables */

/* A quantized [rows, cols] weight matrix resident on the device: the device mirror of a Table
 * (tensor.rs:195-232), created once per Table and freed on drop. */
typedef struct fg_table fg_table;

/* Table::new + upload (tensor.rs:200-211). `bytes` (host) are the Tensor's bytes in the
 * reference layout: quad-major codes, then f32 scales (tensor.rs:1-9). `len` must equal the
 * dtype's byte length for the shape (tensor.rs:39-51). */
int fg_table_create(const void *bytes, size_t len, int dtype, size_t rows, size_t cols, void *stream,
                    fg_table **out);
/* The same from device bytes in the reference layout. */
int fg_table_create_device(const void *bytes, size_t len, int dtype, size_t rows, size_t cols,
                           void *stream, fg_table **out);
int fg_table_free(fg_table *table);
/* Matrix{rows, cols} and the DType of a table (tensor.rs:67-71). */
int fg_table_shape(const fg_table *table, int *dtype, size_t *rows, size_t *cols);
/* The table's bytes back in the reference layout (device `bytes`, fg_table_byte_len long). */
size_t fg_table_byte_len(int dtype, size_t rows, size_t cols);
int fg_table_read(const fg_table *table, void *bytes, void *stream);

/* A table streamed onto the device as a bundle store receives its bytes, instead of from one whole
 * byte array: the device side of Store::write's copy into a zeroed tensor (bundle/src/store.rs:90-126),
 * Store::end_part's size check (store.rs:129-146) and Table::load (bundle/src/load.rs:72-84). A Store
 * routes each piece of a part to its tensor (store.rs:105-124); for a quantized table the binding
 * passes the piece here instead of into Tensor::bytes_mut. One upload is used by one thread at a
 * time. */
typedef struct fg_upload fg_upload;
/* Store::new's zeroed tensor (store.rs:49-61) for a quantized [rows, cols] table: its device storage
 * and two pinned staging buffers. Every copy of the upload runs on `stream`. */
int fg_upload_begin(int dtype, size_t rows, size_t cols, void *stream, fg_upload **out);
/* The next `len` host bytes of the table's reference bytes (tensor.rs:1-9), at byte `offset` of the
 * table: writes arrive in order, so `offset` is the count of bytes written so far (FG_ERR_SHAPE
 * otherwise); past the table's byte length, FG_ERR_FORMAT "table upload: write past its end"
 * (store.rs:95-97). Pieces of any size, zero included. */
int fg_upload_write(fg_upload *upload, size_t offset, const void *bytes, size_t len);
/* Every byte written (else FG_ERR_FORMAT "table upload: N of M bytes", store.rs:130-137, and the
 * upload stays open): waits for the last copies and hands over the table, which fg_table_free
 * frees. The upload is consumed on success. */
int fg_upload_end(fg_upload *upload, fg_table **out);
/* Store::restart_part (store.rs:148-158): forgets what was written, so the table is written again
 * from byte 0. */
int fg_upload_restart(fg_upload *upload);
/* Drops an upload that did not end, with its device storage. */
int fg_upload_free(fg_upload *upload);

/* Tensor::encode of a quantized [rows, cols] matrix (tensor.rs:97-143, quant.rs:143-177):
 * device f32 `values` (row-major) to device `bytes` (fg_table_byte_len long) in the reference
 * layout. */
int fg_encode(int dtype, size_t rows, size_t cols, const float *values, void *bytes, void *stream);

/* Matrix::dequantize_row (tensor.rs:247-271): row `row` as f32 into device `out` (cols long). */
int fg_dequantize_row(const fg_table *table, size_t row, float *out, void *stream);

/* ---------------------------------------------------------- run-time Q7b32 matrices */

/* QuantizedMatrix (matmul.rs:35-102): a Q7b32 matrix quantized at run time, row by row (an
 * attention's keys and values), created with room for `capacity` rows of up to `cols` values
 * (it grows past them). The handle is a table: fg_matmul, fg_dequantize_row, fg_table_read and fg_table_free take it, and
 * its Matrix is the rows appended so far. Created empty, `cols` wide (reset(cols), matmul.rs:47-53). */
int fg_qmatrix_create(size_t capacity, size_t cols, fg_table **out);
/* QuantizedMatrix::reset (matmul.rs:47-53): no rows, `cols` (whole blocks, at most the width it
 * was created with) values per row. */
int fg_qmatrix_reset(fg_table *matrix, size_t cols);
/* QuantizedMatrix::extend (matmul.rs:66-72): `rows` more rows, zero codes and scales until set.
 * Past the capacity the storage grows (doubling) and moves: the call then waits for `stream`,
 * and work on other streams that reads the matrix must be ordered before it. */
int fg_qmatrix_extend(fg_table *matrix, size_t rows, void *stream);
/* QuantizedMatrix::push / set_block for whole rows (matmul.rs:56-64,77-90): rows
 * [row, row + count), already appended, from device f32 `values` [count][cols]. */
int fg_qmatrix_set_rows(fg_table *matrix, size_t row, size_t count, const float *values, void *stream);
/* QuantizedMatrix::set_block (matmul.rs:77-90): block `block` of row `row` from 32 device f32. */
int fg_qmatrix_set_block(fg_table *matrix, size_t row, size_t block, const float *values, void *stream);

/* ------------------------------------------------------------------- int8 attention */

/* Exponentials (ops.rs:163-166): `exp` (within 2 ulp) or `exp_fast` (within 6e-5, fused). */
#define FG_EXP_EXACT 0
#define FG_EXP_FAST 1

/* attention::Call (blocks/src/attention.rs:35-47) with its three Operands (:24-30): head h of
 * row r of an operand is the head_dim device f32 values at r * stride + offset + h * head_dim.
 * `images` images of `queries` query rows over `keys` key and value rows; `heads` query heads
 * share `kv_heads` key heads in consecutive runs. */
typedef struct fg_attention {
    size_t heads, kv_heads, head_dim, images, queries, keys;
    const float *query;
    size_t query_stride, query_offset;
    const float *key;
    size_t key_stride, key_offset;
    const float *value;
    size_t value_stride, value_offset;
    int exponentials; /* FG_EXP_EXACT or FG_EXP_FAST */
} fg_attention;

/* attention::attend (blocks/src/attention.rs:81-214) for the whole call, into device `out`
 * [images * queries][heads * head_dim]: keys and values quantized at run time (Q7b32 rows),
 * both products on the quantized kernels, the reference's f32 order around them. head_dim whole
 * quads, at most 1024; at most 16384 keys. The work is ordered on `stream` (its scratch comes
 * from and returns to a stream-ordered pool): `out` is ready once the stream's work is. */
int fg_attend(const fg_attention *call, float *out, void *stream);

/* ------------------------------------------------------------------------ activations */

/* quantize_rows (matmul.rs:233-257): `count` device f32 values, whole groups of the weight
 * format `dtype`, to int8 levels, one scale and one correction (-zero_point * sum) per group. */
int fg_quantize_rows(const float *x, size_t count, int dtype, int8_t *quants, float *scales,
                     int32_t *corrections, void *stream);

/* A matmul input (matmul.rs:107-119): f32 rows to quantize inside the product, or rows already
 * quantized by fg_quantize_rows for the table's format (all device pointers). Exactly one of
 * `x` and `quants` is set; `scales` and `corrections` go with `quants`. */
typedef struct {
    const float *x;
    const int8_t *quants;
    const float *scales;
    const int32_t *corrections;
} fg_input;

/* ---------------------------------------------------------------------------- products */

/* matmul + Linear::project_quads (matmul.rs:265-317, linear.rs:52-71): for every input row r
 * and output column c in [col_begin, col_end) (whole quads, within the table's padded rows),
 * out[r * ld_out + (c - col_begin)] = row r · W[c] (+ bias[c] when `bias` is set), written, or
 * added with FG_ACCUMULATE. f32 results are bit-identical to the reference's scalar backend, or
 * with FG_FUSED_SCALE to its NEON backend. Products that quantize f32 rows on the matrix cores take
 * scratch from a stream-ordered pool; under HIP graph capture they take it once, outside the
 * stream's work, owned by the graph (no memory node; two instances of one graph must not run at
 * once), and it is freed after the graph is destroyed. */
int fg_matmul(const fg_table *table, const fg_input *input, size_t rows, size_t col_begin,
              size_t col_end, const float *bias, float *out, size_t ld_out, int flags, void *stream);

/* fg_matmul that allocates nothing. No counterpart in the reference (whose CPU product needs no
 * scratch): it is for callers that cannot allocate device memory, such as code under HIP graph
 * capture or a serving loop that forbids hipMalloc. Products that quantize f32 rows on the matrix
 * cores (5 or more rows, or T2b128) need scratch for the levels, scales and corrections; here it is
 * a fixed array of 32 MiB per device, held by the library from its load until the process ends.
 * A product needs rows * cols bytes of levels plus at most 8 * (rows + 127) * groups bytes of scales
 * and corrections (row-major scales and corrections, 8 * rows * groups, or the block-major scales of
 * the staged kernel, 4 * groups * rows rounded up to 128 rows), each part rounded up to 256 bytes;
 * larger products return FG_ERR_SHAPE and belong to fg_matmul. Nothing in the array needs to start at zero: every
 * call writes what it reads. All calls on one device share the array, so calls that overlap on a
 * device (other threads or streams) race: serialize them. FG_PARALLEL_SUM is not taken. */
int fg_matmul_noalloc(const fg_table *table, const fg_input *input, size_t rows, size_t col_begin,
                      size_t col_end, const float *bias, float *out, size_t ld_out, int flags, void *stream);

/* The int32 group accumulators of the same product (the dots of matmul.rs:671-709, correction
 * included): dots[(r * (col_end - col_begin) + (c - col_begin)) * groups + g]. An inspection
 * entry point for parity checks. */
int fg_matmul_dots(const fg_table *table, const fg_input *input, size_t rows, size_t col_begin,
                   size_t col_end, int32_t *dots, void *stream);

/* ------------------------------------------------------------- the Qwen2 decoder step */

/* Transformer::forward with rows = 1 and Prediction::predict (blocks/src/transformer.rs:294-341,
 * layer.rs:161-344, lm.rs:147-179) for the Qwen2 architecture: RMSNorm, fused QKV with bias,
 * rotary embeddings by halves, grouped-query causal attention over an f32 KV cache, a SiLU-gated
 * feed-forward, a tied embedding/head table. Every projection runs through fg_matmul's kernels. */
typedef struct {
    size_t hidden, layers, heads, kv_heads, head_dim, ffn, vocab, capacity;
    float rope_base, eps;
    int dtype; /* the weight format of every table */
    int exact; /* 1: reductions in the reference's order (bit-identical); 0: parallel trees */
} fg_qwen2_shape;

typedef struct {
    const float *norm1, *norm2; /* device [hidden] */
    const float *qkv_bias;      /* device [(heads + 2 kv_heads) head_dim] or NULL */
    const fg_table *qkv, *o, *gate, *up, *down;
} fg_qwen2_layer;

typedef struct fg_qwen2 fg_qwen2;

/* The model over caller-owned tables, norms and caches (device [layers][kv_heads][capacity]
 * [head_dim] f32 each). The handle owns its activation buffers only. */
int fg_qwen2_create(const fg_qwen2_shape *shape, const fg_qwen2_layer *layers, const float *final_norm,
                    const fg_table *table, float *kcache, float *vcache, fg_qwen2 **out);
/* One token at `position`: embedding, every layer, final norm, logits and the greedy token.
 * Outputs (device, any may be NULL): hidden [hidden], logits [vocab], next_token [1]. */
int fg_qwen2_step(fg_qwen2 *model, int token, size_t position, float *hidden, float *logits,
                  int32_t *next_token, void *stream);
/* One layer over a device hidden row (the residual stream, in and out), for layer-level checks. */
int fg_qwen2_layer_forward(fg_qwen2 *model, size_t layer, size_t position, float *hidden, void *stream);
/* An inspection of one layer's attention (layer.rs:175-209, transformer.rs:185-219) over a device
 * hidden row, as the step runs it: the normed row projected to the query, key and value heads, the
 * position's key and value kept in the caches, the query heads rotated, then attention over keys
 * 0..position. Writes the rotated query heads to `query` and the attention's output row (f32, before
 * the output projection quantizes it) to `row`, both device [heads * head_dim]. `hidden` is not
 * changed. */
int fg_qwen2_attention(fg_qwen2 *model, size_t layer, size_t position, const float *hidden, float *query,
                       float *row, void *stream);

/* What one layer forms on the way (layer.rs:161-344), each written by the launch that forms it:
 * device outputs, any may be NULL. */
typedef struct {
    float *query;         /* [heads * head_dim]: the rotated query heads (layer.rs:175-209) */
    float *attention;     /* [heads * head_dim]: the attention row before the output projection
                             quantizes it (transformer.rs:185-219) */
    float *attended;      /* [hidden]: the residual row after the output projection (layer.rs:239-245) */
    float *inner;         /* [ffn]: silu(gate) * up (layer.rs:298-344) */
    int8_t *levels;       /* [ffn]: that row quantized for the down projection (quantize_rows) */
    float *scales;        /* [ffn / 32] */
    int32_t *corrections; /* [ffn / 32] */
    float *out;           /* [hidden]: the layer's output row (layer.rs:269-291) */
} fg_qwen2_probe;

/* One layer over a device hidden row as the step runs it, with its intermediate rows written to
 * `probe` (an inspection for layer-level parity checks): the position's key and value are kept in
 * the caches, `hidden` is not changed. */
int fg_qwen2_layer_probe(fg_qwen2 *model, size_t layer, size_t position, const float *hidden,
                         const fg_qwen2_probe *probe, void *stream);
/* Lm::embed (blocks/src/lm.rs:97-108): the tied table's rows of the device token ids `ids`
 * (count of them) into device `out` [count][hidden]. */
int fg_qwen2_embed(fg_qwen2 *model, const int32_t *ids, size_t count, float *out, void *stream);
/* Reader::read (blocks/src/lm.rs:205-228) with sequential positions: `count` device rows of
 * `embeddings` [count][hidden] read from position `first` (the cache already holds the positions
 * before it), `chunk` rows per call of the stack (Transformer::forward with rows > 1,
 * transformer.rs:294-341, Mask::Causal): per layer every row is normed and quantized, its
 * products run on the matrix cores over all the chunk's rows, each row attends to the keys up to its
 * own position, and the keys and values of every row are kept. Then the last row's prediction
 * (Prediction::predict, lm.rs:147-166). Outputs (device, any may be NULL): hidden [hidden] (the last
 * row's residual stream), logits [vocab], next_token [1]. first + count must not pass the cache's
 * capacity (transformer.rs:329-341). The model's order applies: exact, the reference's reductions,
 * bit-identical to one decode step per row; else the parallel ones. The first read allocates the
 * rows' buffers (for min(chunk, count, 4096) rows; a larger chunk later grows them). */
int fg_qwen2_read(fg_qwen2 *model, const float *embeddings, size_t count, size_t first, size_t chunk, float *hidden,
                  float *logits, int32_t *next_token, void *stream);
int fg_qwen2_free(fg_qwen2 *model);

#ifdef __cplusplus
}
#endif

#endif
