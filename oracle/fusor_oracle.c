/*
 * fusor_oracle.c — CPU restatement of fusor-ai's quantized matrix-product path (scalar x86-64
 * semantics). TEST INFRASTRUCTURE ONLY: the parity oracle and the CPU baseline, never the
 * product. Citations are relative to the fusor-ai checkout, crates/kernels/src unless noted.
 *
 * Built with -O3 -ffp-contract=off -fno-fast-math: Rust never contracts a + b*c, so neither may
 * this file.
 *
 * What pins it (tests/test_oracle.py, tests/test_oracle_attention.py): the reference tests' known
 * answers and f64 tolerance for the product, closed forms and brute force for the formats and
 * quantizers, and absorption cases for the order of every f32 sum in the decode glue (RMSNorm,
 * softmax, weighted values, the exponentials' offset sums). Parity unpinned: the bits of the exp
 * and exp_fast polynomials, SiLU and the rotary angles, which are checked only against their
 * stated error bounds.
 */
#include "fusor_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- formats (quant.rs:32-87) */

int or_group(int dtype) { return dtype == OR_T2B128 ? OR_TERNARY_GROUP : OR_BLOCK; }

int or_zero_point(int dtype)
{
    switch (dtype) {
    case OR_Q7B32: return 64;
    case OR_Q4B32: return 8;
    case OR_T2B128: return 1;
    default: return 0; /* OR_Q8B32: signed levels */
    }
}

int or_codes_per_byte(int dtype)
{
    switch (dtype) {
    case OR_Q4B32: return 2;
    case OR_T2B128: return 4;
    default: return 1;
    }
}

/* tensor.rs:55-57 */
size_t or_padded_values(size_t rows, size_t cols) { return (rows + OR_QUAD - 1) / OR_QUAD * OR_QUAD * cols; }

size_t or_quant_len(int dtype, size_t rows, size_t cols)
{
    return or_padded_values(rows, cols) / (size_t)or_codes_per_byte(dtype);
}

/* tensor.rs:39-51 */
size_t or_byte_len(int dtype, size_t rows, size_t cols)
{
    if (dtype == OR_F32) return rows * cols * sizeof(float);
    size_t padded = or_padded_values(rows, cols);
    return padded / (size_t)or_codes_per_byte(dtype) + padded / (size_t)or_group(dtype) * sizeof(float);
}

/* A stored code's signed level: u - zero_point (quant.rs:80-85); Q8b32 stores the level itself
 * as a two's-complement byte. */
static int level_of(int dtype, uint8_t code)
{
    if (dtype == OR_Q8B32) return (int)(int8_t)code;
    return (int)code - or_zero_point(dtype);
}

/* -------------------------------------------------------------- quad layout (quant.rs:89-118) */

void or_code_position(int dtype, int lane, int input, size_t *byte, unsigned *shift)
{
    int cpb = or_codes_per_byte(dtype);
    int chunk = input / OR_CHUNK_INPUTS, offset = input % OR_CHUNK_INPUTS;
    int words = OR_BLOCK / OR_CHUNK_INPUTS / cpb;
    int bits = 8 / cpb;
    *byte = (size_t)(chunk % words * OR_WORD + lane * OR_CHUNK_INPUTS + offset);
    *shift = (unsigned)(bits * (chunk / words));
}

void or_pack_lane(int dtype, int lane, const uint8_t *codes, uint8_t *quad)
{
    for (int chunk = 0; chunk < OR_BLOCK / OR_CHUNK_INPUTS; chunk++) {
        size_t first;
        unsigned shift;
        or_code_position(dtype, lane, chunk * OR_CHUNK_INPUTS, &first, &shift);
        for (int i = 0; i < OR_CHUNK_INPUTS; i++)
            quad[first + (size_t)i] |= (uint8_t)(codes[chunk * OR_CHUNK_INPUTS + i] << shift);
    }
}

void or_unpack_lane(int dtype, const uint8_t *quad, int lane, uint8_t *codes)
{
    uint8_t mask = (uint8_t)(0xffu >> (8 - 8 / or_codes_per_byte(dtype)));
    for (int input = 0; input < OR_BLOCK; input++) {
        size_t byte;
        unsigned shift;
        or_code_position(dtype, lane, input, &byte, &shift);
        codes[input] = (uint8_t)((quad[byte] >> shift) & mask);
    }
}

/* ------------------------------------------------------ weight quantizers (quant.rs:119-177) */

/* Rust's saturating `f32 as i8` / `as i32` / `as u8` (NaN to 0). */
static int8_t sat_i8(float v)
{
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}

static int32_t sat_i32(float v)
{
    if (v != v) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}

static uint8_t sat_u8(float v)
{
    if (v != v) return 0;
    if (v >= 255.0f) return 255;
    if (v <= 0.0f) return 0;
    return (uint8_t)v;
}

/* f32::clamp: NaN stays NaN. */
static float clampf(float v, float lo, float hi)
{
    if (v < lo) v = lo;
    if (v > hi) v = hi;
    return v;
}

/* f32::max ignores a NaN operand, as fmaxf does. quant.rs:120-122 */
static float absmax(const float *v, size_t n)
{
    float m = 0.0f;
    for (size_t i = 0; i < n; i++) m = fmaxf(m, fabsf(v[i]));
    return m;
}

/* quant.rs:126-128 */
static float group_scale(float extreme, float level) { return extreme == 0.0f ? 1.0f : extreme / level; }

float or_quantize_group(int dtype, const float *x, uint8_t *codes)
{
    switch (dtype) {
    case OR_Q7B32: { /* quant.rs:131-149 */
        float scale = group_scale(absmax(x, OR_BLOCK), 63.0f);
        for (int i = 0; i < OR_BLOCK; i++) {
            int level = sat_i8(rintf(x[i] / scale));
            if (level < -63) level = -63;
            if (level > 63) level = 63;
            codes[i] = (uint8_t)(level + 64);
        }
        return scale;
    }
    case OR_Q4B32: { /* quant.rs:151-166: the first value of largest magnitude */
        float extreme = 0.0f;
        for (int i = 0; i < OR_BLOCK; i++)
            if (fabsf(x[i]) > fabsf(extreme)) extreme = x[i];
        float scale = group_scale(extreme, -8.0f);
        for (int i = 0; i < OR_BLOCK; i++) codes[i] = sat_u8(clampf(rintf(x[i] / scale) + 8.0f, 0.0f, 15.0f));
        return scale;
    }
    case OR_T2B128: { /* quant.rs:168-177 */
        float scale = group_scale(absmax(x, OR_TERNARY_GROUP), 1.0f);
        for (int i = 0; i < OR_TERNARY_GROUP; i++)
            codes[i] = (uint8_t)(sat_i32(clampf(rintf(x[i] / scale), -1.0f, 1.0f)) + 1);
        return scale;
    }
    case OR_Q8B32: { /* extension: Q7b32's rule at 127 levels, signed codes */
        float scale = group_scale(absmax(x, OR_BLOCK), 127.0f);
        for (int i = 0; i < OR_BLOCK; i++) {
            int level = sat_i8(rintf(x[i] / scale));
            if (level < -127) level = -127;
            codes[i] = (uint8_t)(int8_t)level;
        }
        return scale;
    }
    default: return 0.0f;
    }
}

/* tensor.rs:97-143 */
int or_encode(int dtype, size_t rows, size_t cols, const float *values, uint8_t *bytes)
{
    int group = or_group(dtype);
    if (dtype == OR_F32 || cols % (size_t)group != 0) return -1;
    size_t quant_len = or_quant_len(dtype, rows, cols);
    uint8_t *quants = bytes;
    float *scales = (float *)(void *)(bytes + quant_len);
    size_t blocks = cols / OR_BLOCK, groups = cols / (size_t)group;
    size_t quad_bytes = (size_t)(OR_QUAD * OR_BLOCK / or_codes_per_byte(dtype));
    uint8_t *codes = (uint8_t *)calloc(cols, 1);
    if (!codes) return -1;
    for (size_t row = 0; row < rows; row++) {
        size_t quad = row / OR_QUAD, lane = row % OR_QUAD;
        const float *rv = values + row * cols;
        for (size_t index = 0; index < groups; index++) {
            float scale = or_quantize_group(dtype, rv + index * (size_t)group, codes + index * (size_t)group);
            memcpy(&scales[(quad * groups + index) * OR_QUAD + lane], &scale, sizeof scale);
        }
        for (size_t block = 0; block < blocks; block++) {
            size_t at = (quad * blocks + block) * quad_bytes;
            or_pack_lane(dtype, (int)lane, codes + block * OR_BLOCK, quants + at);
        }
    }
    free(codes);
    return 0;
}

/* tensor.rs:247-271 and quant.rs:81-85 */
void or_dequantize_row(int dtype, size_t rows, size_t cols, const uint8_t *bytes, size_t row, float *out)
{
    size_t quant_len = or_quant_len(dtype, rows, cols);
    const float *scales = (const float *)(const void *)(bytes + quant_len);
    size_t quad = row / OR_QUAD, lane = row % OR_QUAD;
    size_t blocks = cols / OR_BLOCK, groups = cols / (size_t)or_group(dtype);
    size_t quad_bytes = (size_t)(OR_QUAD * OR_BLOCK / or_codes_per_byte(dtype));
    size_t blocks_per_group = (size_t)or_group(dtype) / OR_BLOCK;
    uint8_t codes[OR_BLOCK];
    for (size_t block = 0; block < blocks; block++) {
        or_unpack_lane(dtype, bytes + (quad * blocks + block) * quad_bytes, (int)lane, codes);
        float scale = scales[(quad * groups + block / blocks_per_group) * OR_QUAD + lane];
        for (int i = 0; i < OR_BLOCK; i++) out[block * OR_BLOCK + (size_t)i] = scale * (float)level_of(dtype, codes[i]);
    }
}

/* -------------------------------------------------- activation quantization (matmul.rs:233) */

void or_quantize_rows(const float *x, size_t count, int dtype, int8_t *quants, float *scales,
                      int32_t *corrections)
{
    size_t group = (size_t)or_group(dtype);
    int zp = or_zero_point(dtype);
    for (size_t g = 0; g < count / group; g++) {
        const float *values = x + g * group;
        /* per 32-block absmax (scalar.rs:48-50), then max over the group's blocks */
        float largest = 0.0f;
        for (size_t b = 0; b < group / OR_BLOCK; b++) largest = fmaxf(largest, absmax(values + b * OR_BLOCK, OR_BLOCK));
        float scale = group_scale(largest, 127.0f); /* arch/mod.rs:223-228 */
        int32_t sum = 0;
        for (size_t i = 0; i < group; i++) { /* scalar.rs:57-66 */
            int8_t level = sat_i8(clampf(rintf(values[i] / scale), -127.0f, 127.0f));
            sum += level;
            quants[g * group + i] = level;
        }
        scales[g] = scale;
        corrections[g] = -zp * sum;
    }
}

/* ------------------------------------------------------- the product (matmul.rs:409-763) */

/* Backend::TILE of the scalar backend (scalar.rs:16) and QUADS per pass (matmul.rs:510). */
#define TILE 4
#define QUADS 4
#define ROWS_PER_CALL 64

typedef struct {
    int dtype;
    size_t cols, blocks, groups, blocks_per_group, quad_bytes, words;
    const uint8_t *quants;
    const float *scales;
    const int8_t *x;
    const float *x_scales;
    const int32_t *x_corrections;
    int fused; /* the NEON backend's Backend::scale: one fused multiply-add (arch/neon.rs:140-154) */
} product;

/* Format::chunk (matmul.rs:443-469): code `i` of a word's chunk `part`. */
static inline int32_t chunk_code(const product *p, const uint8_t *word, int part, int i)
{
    uint8_t byte = word[i];
    switch (p->dtype) {
    case OR_Q4B32: return (byte >> (4 * part)) & 0x0f; /* scalar.rs:24-26 */
    case OR_T2B128: return (byte >> (2 * part)) & 0x3; /* scalar.rs:28-30 */
    case OR_Q8B32: return (int8_t)byte;
    default: return byte;
    }
}

/* quad_pass (matmul.rs:628-717) for `rows` activation rows from `first_row` against `pass`
 * quads from `first_quad`; store(row, first column, sums) through `out`. */
static void quad_pass(const product *p, size_t first_row, int rows, size_t first_quad, int pass,
                      float *out, size_t ld_out, size_t col_begin, const float *bias, int32_t *dots_out,
                      size_t out_cols)
{
    float sums[TILE][QUADS][OR_QUAD];
    for (int r = 0; r < rows; r++)
        for (int q = 0; q < pass; q++)
            for (int l = 0; l < OR_QUAD; l++) sums[r][q][l] = 0.0f;
    int parts = OR_CHUNKS / (int)p->words;
    for (size_t group = 0; group < p->groups; group++) {
        int32_t dots[TILE][QUADS][OR_QUAD];
        for (int r = 0; r < rows; r++) { /* Backend::seed */
            int32_t c = p->x_corrections[(first_row + (size_t)r) * p->groups + group];
            for (int q = 0; q < pass; q++)
                for (int l = 0; l < OR_QUAD; l++) dots[r][q][l] = c;
        }
        for (size_t block = group * p->blocks_per_group; block < (group + 1) * p->blocks_per_group; block++) {
            /* accumulate (matmul.rs:741-763) */
            for (size_t word = 0; word < p->words; word++) {
                for (int part = 0; part < parts; part++) {
                    size_t chunk = (size_t)part * p->words + word;
                    for (int r = 0; r < rows; r++) {
                        const int8_t *a = p->x + (first_row + (size_t)r) * p->cols + block * OR_BLOCK + chunk * OR_CHUNK_INPUTS;
                        for (int q = 0; q < pass; q++) {
                            const uint8_t *w = p->quants + ((first_quad + (size_t)q) * p->blocks + block) * p->quad_bytes + word * OR_WORD;
                            for (int l = 0; l < OR_QUAD; l++) { /* Backend::dot (scalar.rs:72-79) */
                                int32_t s = 0;
                                for (int i = 0; i < OR_CHUNK_INPUTS; i++)
                                    s += (int32_t)a[i] * chunk_code(p, w, part, l * OR_CHUNK_INPUTS + i);
                                dots[r][q][l] += s;
                            }
                        }
                    }
                }
            }
        }
        for (int r = 0; r < rows; r++) {
            float row_scale = p->x_scales[(first_row + (size_t)r) * p->groups + group];
            for (int q = 0; q < pass; q++) {
                const float *cs = p->scales + ((first_quad + (size_t)q) * p->groups + group) * OR_QUAD;
                for (int l = 0; l < OR_QUAD; l++) { /* Backend::scale (scalar.rs:81-90) */
                    float product = cs[l] * row_scale;
                    if (p->fused) { /* vfmaq_f32(sums, vcvtq_f32_s32(dots), column_scales * row_scale) */
                        sums[r][q][l] = fmaf((float)dots[r][q][l], product, sums[r][q][l]);
                    } else {
                        float term = (float)dots[r][q][l] * product;
                        sums[r][q][l] = sums[r][q][l] + term;
                    }
                }
                if (dots_out) {
                    for (int l = 0; l < OR_QUAD; l++) {
                        size_t col = (first_quad + (size_t)q) * OR_QUAD + (size_t)l - col_begin;
                        dots_out[((first_row + (size_t)r) * out_cols + col) * p->groups + group] = dots[r][q][l];
                    }
                }
            }
        }
    }
    for (int r = 0; r < rows; r++)
        for (int q = 0; q < pass; q++)
            for (int l = 0; l < OR_QUAD; l++) {
                size_t col = (first_quad + (size_t)q) * OR_QUAD + (size_t)l;
                float v = sums[r][q][l];
                if (bias) v = v + bias[col]; /* linear.rs:63-68 */
                out[(first_row + (size_t)r) * ld_out + (col - col_begin)] = v;
            }
}

int or_matmul(int dtype, size_t n_rows, size_t cols, const uint8_t *bytes, const int8_t *quants,
              const float *scales, const int32_t *corrections, size_t rows, size_t col_begin,
              size_t col_end, const float *bias, float *out, size_t ld_out, int32_t *dots)
{
    return or_matmul_fused(dtype, n_rows, cols, bytes, quants, scales, corrections, rows, col_begin, col_end, bias,
                           out, ld_out, dots, 0);
}

int or_matmul_fused(int dtype, size_t n_rows, size_t cols, const uint8_t *bytes, const int8_t *quants,
                    const float *scales, const int32_t *corrections, size_t rows, size_t col_begin,
                    size_t col_end, const float *bias, float *out, size_t ld_out, int32_t *dots, int fused)
{
    if (dtype == OR_F32 || cols % (size_t)or_group(dtype) != 0) return -1;
    if (col_begin % OR_QUAD || col_end % OR_QUAD || col_end < col_begin) return -1;
    size_t padded_rows = (n_rows + OR_QUAD - 1) / OR_QUAD * OR_QUAD;
    if (col_end > padded_rows) return -1;
    product p;
    p.dtype = dtype;
    p.cols = cols;
    p.blocks = cols / OR_BLOCK;
    p.groups = cols / (size_t)or_group(dtype);
    p.blocks_per_group = (size_t)or_group(dtype) / OR_BLOCK;
    p.quad_bytes = (size_t)(OR_QUAD * OR_BLOCK / or_codes_per_byte(dtype));
    p.words = p.quad_bytes / OR_WORD;
    p.quants = bytes;
    p.scales = (const float *)(const void *)(bytes + or_quant_len(dtype, n_rows, cols));
    p.x = quants;
    p.x_scales = scales;
    p.x_corrections = corrections;
    p.fused = fused;
    size_t first = col_begin / OR_QUAD, end = col_end / OR_QUAD;
    size_t out_cols = col_end - col_begin;
    /* quant_matmul: ROWS_PER_CALL rows per call of quant_tiles, TILE rows per tile (matmul.rs:409-577) */
    for (size_t call = 0; call < rows; call += ROWS_PER_CALL) {
        size_t call_end = call + ROWS_PER_CALL < rows ? call + ROWS_PER_CALL : rows;
        for (size_t start = call; start < call_end; start += TILE) {
            int tile = (int)(call_end - start < TILE ? call_end - start : TILE);
            /* quant_tile (matmul.rs:605-623): QUADS per pass, one when a tile is a single row */
            size_t full = tile == 1 ? first : first + (end - first) / QUADS * QUADS;
            for (size_t quad = first; quad < full; quad += QUADS)
                quad_pass(&p, start, tile, quad, QUADS, out, ld_out, col_begin, bias, dots, out_cols);
            for (size_t quad = full; quad < end; quad++)
                quad_pass(&p, start, tile, quad, 1, out, ld_out, col_begin, bias, dots, out_cols);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ thread team */

typedef struct {
    int dtype;
    size_t n_rows, cols;
    const uint8_t *bytes;
    const int8_t *quants;
    const float *scales;
    const int32_t *corrections;
    size_t rows;
    const float *bias;
    float *out;
    int index, count, by_rows;
    size_t outputs;
} split_job;

/* Ctx::split (team/src/team.rs:88-93) */
static void split(size_t total, size_t align, int index, int count, size_t *start, size_t *end)
{
    size_t units = total / align;
    *start = units * (size_t)index / (size_t)count * align;
    *end = units * (size_t)(index + 1) / (size_t)count * align;
}

static void *split_worker(void *arg)
{
    split_job *j = (split_job *)arg;
    size_t groups = j->cols / (size_t)or_group(j->dtype);
    if (j->by_rows) {
        size_t r0, r1;
        split(j->rows, 1, j->index, j->count, &r0, &r1);
        size_t padded = (j->outputs + 3) / 4 * 4;
        float *tmp = (float *)malloc((r1 - r0 + 1) * padded * sizeof(float));
        if (r1 > r0) {
            or_matmul(j->dtype, j->n_rows, j->cols, j->bytes, j->quants + r0 * j->cols, j->scales + r0 * groups,
                      j->corrections + r0 * groups, r1 - r0, 0, padded, j->bias, tmp, padded, NULL);
            for (size_t r = r0; r < r1; r++) memcpy(j->out + r * j->outputs, tmp + (r - r0) * padded, j->outputs * sizeof(float));
        }
        free(tmp);
    } else {
        size_t c0, c1;
        split(j->outputs, 16, j->index, j->count, &c0, &c1); /* COLUMN_ALIGN (linear.rs:13) */
        if (j->index == j->count - 1) c1 = j->outputs;
        size_t q0 = c0 / 4 * 4, q1 = (c1 + 3) / 4 * 4;
        if (q1 > q0) {
            float *tmp = (float *)malloc(j->rows * (q1 - q0) * sizeof(float));
            or_matmul(j->dtype, j->n_rows, j->cols, j->bytes, j->quants, j->scales, j->corrections, j->rows, q0, q1,
                      j->bias, tmp, q1 - q0, NULL);
            for (size_t r = 0; r < j->rows; r++)
                for (size_t c = c0; c < c1; c++) j->out[r * j->outputs + c] = tmp[r * (q1 - q0) + (c - q0)];
            free(tmp);
        }
    }
    return NULL;
}

int or_matmul_threaded(int dtype, size_t n_rows, size_t cols, const uint8_t *bytes,
                       const int8_t *quants, const float *scales, const int32_t *corrections,
                       size_t rows, const float *bias, float *out, int threads)
{
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    split_job jobs[256];
    pthread_t tids[256];
    int by_rows = rows >= n_rows || n_rows % 16 != 0; /* conv.rs:584-589 */
    for (int t = 0; t < threads; t++) {
        split_job j = {dtype, n_rows, cols, bytes, quants, scales, corrections, rows, bias, out, t, threads, by_rows, n_rows};
        jobs[t] = j;
    }
    for (int t = 1; t < threads; t++) pthread_create(&tids[t], NULL, split_worker, &jobs[t]);
    split_worker(&jobs[0]);
    for (int t = 1; t < threads; t++) pthread_join(tids[t], NULL);
    return 0;
}

/* --------------------------------------------------------------------- f32 ops (ops.rs) */

/* ops.rs:97-131: Cephes expf coefficients, clamp, range reduction in two parts, Horner order,
 * no fused multiply-add. */
float or_exp(float x)
{
    static const float poly_c[6] = {1.9875691e-4f, 1.3981999e-3f, 8.333452e-3f, 4.1665796e-2f, 0.16666666f, 0.5f};
    const float ln2_high = 0.6933594f, ln2_low = -2.1219444e-4f, log2_e = 1.44269504088896340736f;
    x = clampf(x, -87.0f, 88.0f);
    float exponent = rintf(x * log2_e);
    float remainder = x - exponent * ln2_high - exponent * ln2_low;
    float poly = poly_c[0];
    for (int i = 1; i < 6; i++) poly = poly * remainder + poly_c[i];
    poly = poly * remainder * remainder + remainder + 1.0f;
    uint32_t bits = (uint32_t)((sat_i32(exponent) + 127) << 23);
    float two_n;
    memcpy(&two_n, &bits, sizeof two_n);
    return poly * two_n;
}

float or_silu(float x) { return x / (1.0f + or_exp(-x)); }

/* ops.rs:137-153: x clamped below at EXP_MIN, n = round(x·log2 e) (ties to even), r = fma(-n,
 * ln 2, x), the degree-4 Taylor polynomial in fused multiply-adds (Rust's mul_add, the scalar
 * backend's arithmetic), times 2^n. */
float or_exp_fast(float x)
{
    static const float taylor[5] = {1.0f / 24.0f, 1.0f / 6.0f, 0.5f, 1.0f, 1.0f};
    const float log2_e = 1.44269504088896340736f, ln_2 = 0.693147180559945309417f;
    x = fmaxf(x, -87.0f);
    float exponent = rintf(x * log2_e);
    float remainder = fmaf(-exponent, ln_2, x);
    float poly = taylor[0];
    for (int i = 1; i < 5; i++) poly = fmaf(poly, remainder, taylor[i]);
    uint32_t bits = (uint32_t)((sat_i32(exponent) + 127) << 23);
    float two_n;
    memcpy(&two_n, &bits, sizeof two_n);
    return poly * two_n;
}

/* Exponentials::apply (ops.rs:168-191) on the scalar backend: the maximum as a fold from -inf
 * (scalar.rs:52-55); the sweep over whole runs of EXP_RUN = 8 values (arch/mod.rs:46), each
 * value's exponential added to the sum of its offset in the run (scalar.rs:117-126); the rest
 * one by one; then the rest's values and the eight offset sums added in that order. */
float or_exponentials_apply(float *scores, size_t n, int fast)
{
    float max = -INFINITY;
    for (size_t i = 0; i < n; i++) max = fmaxf(max, scores[i]);
    float sums[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    const size_t whole = n / 8 * 8;
    for (size_t i = 0; i < whole; i++) {
        const float v = fast ? or_exp_fast(scores[i] - max) : or_exp(scores[i] - max);
        scores[i] = v;
        sums[i % 8] = sums[i % 8] + v;
    }
    for (size_t i = whole; i < n; i++) scores[i] = fast ? or_exp_fast(scores[i] - max) : or_exp(scores[i] - max);
    float total = -0.0f;
    for (size_t i = whole; i < n; i++) total = total + scores[i];
    for (int k = 0; k < 8; k++) total = total + sums[k];
    return total;
}

/* scalar.rs:340-342: a float sum in index order from -0.0 */
float or_dot_f32(const float *a, const float *b, size_t n)
{
    float s = -0.0f;
    for (size_t i = 0; i < n; i++) s = s + a[i] * b[i];
    return s;
}

/* ops.rs:7-16 */
void or_rms_norm(const float *x, const float *weight, size_t dim, float eps, float *out)
{
    float mean = or_dot_f32(x, x, dim) / (float)dim;
    float inverse = 1.0f / sqrtf(mean + eps);
    for (size_t i = 0; i < dim; i++) out[i] = x[i] * inverse * weight[i];
}

/* ops.rs:70-74 */
void or_rope_inv_freq(float base, size_t head_dim, float *inv_freq)
{
    for (size_t i = 0; i < head_dim / 2; i++) inv_freq[i] = 1.0f / powf(base, (float)(2 * i) / (float)head_dim);
}

/* blocks/src/rotary.rs angles: angle = position * frequency in f32, then cos and sin */
void or_rope_angles(const float *inv_freq, size_t half, size_t position, float *cos_out, float *sin_out)
{
    for (size_t i = 0; i < half; i++) {
        float angle = (float)position * inv_freq[i];
        cos_out[i] = cosf(angle);
        sin_out[i] = sinf(angle);
    }
}

/* ops.rs:77-85 */
void or_rope_half(float *head, size_t dim, const float *c, const float *s)
{
    size_t half = dim / 2;
    for (size_t i = 0; i < half; i++) {
        float x = head[i], y = head[i + half];
        head[i] = x * c[i] - y * s[i];
        head[i + half] = y * c[i] + x * s[i];
    }
}

/* ops.rs:301-306: maximum, the exact exponentials, their sum in index order, the division */
void or_softmax(float *scores, size_t n)
{
    float max = -INFINITY;
    for (size_t i = 0; i < n; i++) max = fmaxf(max, scores[i]);
    for (size_t i = 0; i < n; i++) scores[i] = or_exp(scores[i] - max);
    float total = -0.0f;
    for (size_t i = 0; i < n; i++) total = total + scores[i];
    for (size_t i = 0; i < n; i++) scores[i] = scores[i] / total;
}

/* ops::weigh (ops.rs:329-342) on the scalar backend: `scores` replaced by their softmax, then
 * out = the sum from +0 of w_j·value_j, one key at a time in key order (the default
 * axpy_f32_many, arch/mod.rs:141-147, over blocks of DOTS keys, then the rest one by one: the
 * same order); value j at values + j·stride. */
void or_weigh(float *scores, size_t n, const float *values, size_t stride, size_t dim, float *out)
{
    or_softmax(scores, n);
    for (size_t i = 0; i < dim; i++) out[i] = 0.0f;
    for (size_t j = 0; j < n; j++) {
        const float *v = values + j * stride;
        for (size_t i = 0; i < dim; i++) out[i] = out[i] + scores[j] * v[i];
    }
}

/* ------------------------------------------------- int8 attention (blocks/src/attention.rs) */

static size_t pad32(size_t n) { return (n + 31) / 32 * 32; }

/* attention::attend (attention.rs:81-95) over every (image, head, block of queries); each unit
 * (attention.rs:157-214) is independent, so the units' order does not change a bit. Per (image,
 * key head) (Scratch::quantize, attention.rs:100-137): the keys' mean over the keys in order,
 * divided by their count; each key less the mean, zero-padded to whole blocks, pushed as a
 * Q7b32 row; the values transposed, one Q7b32 row per channel over the keys padded with zeros.
 * Per unit: the queries zero-padded and quantized; scores = the keys' product over the keys
 * rounded up to a quad, each times 1/sqrt(head_dim), zeros past them; Exponentials::apply over
 * the first `keys`; the scores' rows quantized (their whole padded width); the values' product
 * over the channels, each divided by its row's sum. Returns -1 on a shape error. */
int or_attend(const or_attention *c, float *out)
{
    const size_t hd = c->head_dim, keys = c->keys, queries = c->queries;
    if (!hd || !keys || !queries || !c->heads || !c->kv_heads || c->heads % c->kv_heads || hd % 4) return -1;
    const size_t pd = pad32(hd), pk = pad32(keys), keys4 = (keys + 3) / 4 * 4;
    const size_t stride = c->heads * hd, group = c->heads / c->kv_heads;
    const float scale = 1.0f / sqrtf((float)hd);
    float *mean = malloc(hd * sizeof(float));
    float *krows = malloc(keys * pd * sizeof(float)), *vrows = malloc(hd * pk * sizeof(float));
    uint8_t *kbytes = malloc(or_byte_len(OR_Q7B32, keys, pd)), *vbytes = malloc(or_byte_len(OR_Q7B32, hd, pk));
    float *qrows = malloc(32 * pd * sizeof(float)), *scores = malloc(32 * pk * sizeof(float));
    float *prod = malloc(32 * (keys4 > hd ? keys4 : hd) * sizeof(float)), sums[32];
    const size_t wide = pd > pk ? pd : pk;
    int8_t *q = malloc(32 * wide);
    float *qs = malloc(32 * (wide / 32) * sizeof(float));
    int32_t *qc = malloc(32 * (wide / 32) * sizeof(int32_t));
    int rc = 0;
    for (size_t image = 0; image < c->images && !rc; image++) {
        for (size_t kh = 0; kh < c->kv_heads && !rc; kh++) {
            const size_t first = image * keys;
            for (size_t d = 0; d < hd; d++) mean[d] = 0.0f;
            for (size_t k = 0; k < keys; k++) {
                const float *row = c->key + (first + k) * c->key_stride + c->key_offset + kh * hd;
                for (size_t d = 0; d < hd; d++) mean[d] = mean[d] + row[d];
            }
            for (size_t d = 0; d < hd; d++) mean[d] = mean[d] / (float)keys;
            for (size_t k = 0; k < keys; k++) {
                const float *row = c->key + (first + k) * c->key_stride + c->key_offset + kh * hd;
                for (size_t d = 0; d < pd; d++) krows[k * pd + d] = d < hd ? row[d] - mean[d] : 0.0f;
            }
            for (size_t d = 0; d < hd; d++)
                for (size_t k = 0; k < pk; k++)
                    vrows[d * pk + k] = k < keys ? c->value[(first + k) * c->value_stride + c->value_offset + kh * hd + d] : 0.0f;
            /* encoding packs codes into zeroed quads; padding rows keep zero codes and scales */
            memset(kbytes, 0, or_byte_len(OR_Q7B32, keys, pd));
            memset(vbytes, 0, or_byte_len(OR_Q7B32, hd, pk));
            if (or_encode(OR_Q7B32, keys, pd, krows, kbytes) || or_encode(OR_Q7B32, hd, pk, vrows, vbytes)) {
                rc = -1;
                break;
            }
            for (size_t h = kh * group; h < (kh + 1) * group && !rc; h++) {
                for (size_t q0 = 0; q0 < queries; q0 += 32) {
                    const size_t nq = queries - q0 < 32 ? queries - q0 : 32, qfirst = image * queries + q0;
                    for (size_t r = 0; r < nq; r++) {
                        const float *row = c->query + (qfirst + r) * c->query_stride + c->query_offset + h * hd;
                        for (size_t d = 0; d < pd; d++) qrows[r * pd + d] = d < hd ? row[d] : 0.0f;
                    }
                    or_quantize_rows(qrows, nq * pd, OR_Q7B32, q, qs, qc);
                    if (or_matmul(OR_Q7B32, keys, pd, kbytes, q, qs, qc, nq, 0, keys4, NULL, prod, keys4, NULL)) {
                        rc = -1;
                        break;
                    }
                    for (size_t r = 0; r < nq; r++) {
                        for (size_t k = 0; k < pk; k++) scores[r * pk + k] = k < keys4 ? prod[r * keys4 + k] * scale : 0.0f;
                        sums[r] = or_exponentials_apply(scores + r * pk, keys, c->fast);
                    }
                    or_quantize_rows(scores, nq * pk, OR_Q7B32, q, qs, qc);
                    if (or_matmul(OR_Q7B32, hd, pk, vbytes, q, qs, qc, nq, 0, hd, NULL, prod, hd, NULL)) {
                        rc = -1;
                        break;
                    }
                    for (size_t r = 0; r < nq; r++)
                        for (size_t d = 0; d < hd; d++) out[(qfirst + r) * stride + h * hd + d] = prod[r * hd + d] / sums[r];
                }
            }
        }
    }
    free(mean); free(krows); free(vrows); free(kbytes); free(vbytes); free(qrows); free(scores); free(prod);
    free(q); free(qs); free(qc);
    return rc;
}

/* ---------------------------------------------------------------------- rng (rng.rs) */

void or_rng_new(or_rng *rng, uint64_t seed)
{
    uint64_t mixed = seed;
    for (int i = 0; i < 4; i++) {
        mixed += 0x9E3779B97F4A7C15ull;
        uint64_t v = mixed;
        v = (v ^ (v >> 30)) * 0xBF58476D1CE4E5B9ull;
        v = (v ^ (v >> 27)) * 0x94D049BB133111EBull;
        rng->s[i] = v ^ (v >> 31);
    }
}

static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

uint64_t or_rng_next_u64(or_rng *rng)
{
    uint64_t *s = rng->s;
    uint64_t result = rotl(s[1] * 5, 7) * 9;
    uint64_t shifted = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= shifted;
    s[3] = rotl(s[3], 45);
    return result;
}

double or_rng_uniform(or_rng *rng) { return (double)((or_rng_next_u64(rng) >> 11) + 1) / (double)(1ull << 53); }

void or_rng_fill_normal(or_rng *rng, float *out, size_t n)
{
    for (size_t i = 0; i < n; i += 2) {
        double radius = sqrt(-2.0 * log(or_rng_uniform(rng)));
        double angle = 6.283185307179586476925286766559 * or_rng_uniform(rng);
        out[i] = (float)(radius * cos(angle));
        if (i + 1 < n) out[i + 1] = (float)(radius * sin(angle));
    }
}

/* -------------------------------------------------------------------- the Qwen2 step */

/* One projection of a single quantized row: Linear::project over every output
 * (linear.rs:52-97), through the team's column split when threads > 1. */
static void project_row(const or_qwen2_shape *sh, const uint8_t *table, size_t outputs, size_t inputs,
                        const float *x, const float *bias, float *out, int threads)
{
    size_t groups = inputs / (size_t)or_group(sh->dtype);
    int8_t *q = (int8_t *)malloc(inputs);
    float *s = (float *)malloc(groups * sizeof(float));
    int32_t *c = (int32_t *)malloc(groups * sizeof(int32_t));
    or_quantize_rows(x, inputs, sh->dtype, q, s, c);
    if (threads > 1) {
        or_matmul_threaded(sh->dtype, outputs, inputs, table, q, s, c, 1, bias, out, threads);
    } else {
        size_t padded = (outputs + 3) / 4 * 4;
        float *tmp = (float *)malloc(padded * sizeof(float));
        or_matmul(sh->dtype, outputs, inputs, table, q, s, c, 1, 0, padded, bias, tmp, padded, NULL);
        memcpy(out, tmp, outputs * sizeof(float));
        free(tmp);
    }
    free(q);
    free(s);
    free(c);
}

static size_t cache_offset(const or_qwen2_shape *sh, size_t layer, size_t kv_head, size_t position)
{
    return ((layer * sh->kv_heads + kv_head) * sh->capacity + position % sh->capacity) * sh->head_dim;
}

int or_qwen2_layer_forward(const or_qwen2_shape *sh, const or_qwen2_layer *ly, size_t li, float *kcache,
                           float *vcache, size_t position, const float *cos_v, const float *sin_v,
                           float *hidden, int threads)
{
    size_t H = sh->hidden, D = sh->head_dim;
    size_t qkv_width = (sh->heads + 2 * sh->kv_heads) * D, width = sh->heads * D;
    float *normed = (float *)malloc(H * sizeof(float));
    float *qkv = (float *)malloc(qkv_width * sizeof(float));
    float *attn = (float *)malloc(width * sizeof(float));
    float *y = (float *)malloc((H > sh->ffn ? H : sh->ffn) * sizeof(float));
    float *gate = (float *)malloc(sh->ffn * sizeof(float));
    float *up = (float *)malloc(sh->ffn * sizeof(float));
    float *scores = (float *)malloc((position + 1) * sizeof(float));

    /* prepare(norm1, qkv) then attention_input (layer.rs:161-209) */
    or_rms_norm(hidden, ly->norm1, H, sh->eps, normed);
    project_row(sh, ly->qkv, qkv_width, H, normed, ly->qkv_bias, qkv, threads);
    size_t rotated = sh->heads + sh->kv_heads;
    for (size_t unit = 0; unit < sh->heads + 2 * sh->kv_heads; unit++) {
        float *head = qkv + unit * D;
        if (unit < rotated) or_rope_half(head, D, cos_v, sin_v);
        if (unit >= sh->heads) { /* KvCache::keep (transformer.rs:166-180) */
            float *target = unit < rotated ? kcache : vcache;
            memcpy(target + cache_offset(sh, li, (unit - sh->heads) % sh->kv_heads, position), head, D * sizeof(float));
        }
    }
    /* KvCache::attend under Mask::Causal (transformer.rs:185-219) and ops::attend (ops.rs:310-342) */
    float scale = 1.0f / sqrtf((float)D);
    for (size_t h = 0; h < sh->heads; h++) {
        size_t kv = h / (sh->heads / sh->kv_heads);
        const float *query = qkv + h * D;
        for (size_t j = 0; j <= position; j++)
            scores[j] = or_dot_f32(query, kcache + cache_offset(sh, li, kv, j), D) * scale;
        /* keys 0..position are whole rows from the head's first (position < capacity) */
        or_weigh(scores, position + 1, vcache + cache_offset(sh, li, kv, 0), D, D, attn + h * D);
    }
    /* attended_residual: hidden += o(attention) (layer.rs:239-245, linear.rs:134-143) */
    project_row(sh, ly->o, H, width, attn, NULL, y, threads);
    for (size_t i = 0; i < H; i++) hidden[i] = hidden[i] + y[i];
    /* feed_forward_residual with the gated SiLU inner (layer.rs:249-344) */
    or_rms_norm(hidden, ly->norm2, H, sh->eps, normed);
    project_row(sh, ly->gate, sh->ffn, H, normed, NULL, gate, threads);
    project_row(sh, ly->up, sh->ffn, H, normed, NULL, up, threads);
    for (size_t i = 0; i < sh->ffn; i++) gate[i] = or_silu(gate[i]) * up[i];
    project_row(sh, ly->down, H, sh->ffn, gate, NULL, y, threads);
    for (size_t i = 0; i < H; i++) hidden[i] = hidden[i] + y[i];

    free(normed);
    free(qkv);
    free(attn);
    free(y);
    free(gate);
    free(up);
    free(scores);
    return 0;
}

/* lm.rs:169-179: the first of equals */
int or_greedy(const float *logits, size_t n)
{
    size_t best = 0;
    for (size_t t = 0; t < n; t++)
        if (logits[t] > logits[best]) best = t;
    return (int)best;
}

int or_qwen2_step(const or_qwen2_shape *sh, const or_qwen2_layer *layers, const float *final_norm,
                  const uint8_t *table, float *kcache, float *vcache, int token, size_t position,
                  float *hidden_out, float *logits, int *next_token, int threads)
{
    size_t H = sh->hidden, half = sh->head_dim / 2;
    if (position >= sh->capacity) return -1; /* transformer.rs:329-341 */
    float *hidden = (float *)malloc(H * sizeof(float));
    float *inv = (float *)malloc(half * sizeof(float));
    float *cos_v = (float *)malloc(half * sizeof(float));
    float *sin_v = (float *)malloc(half * sizeof(float));
    or_dequantize_row(sh->dtype, sh->vocab, H, table, (size_t)token, hidden); /* lm.rs:99-107 */
    or_rope_inv_freq(sh->rope_base, sh->head_dim, inv);
    or_rope_angles(inv, half, position, cos_v, sin_v); /* Stack::turn (layer.rs:140-154) */
    for (size_t l = 0; l < sh->layers; l++)
        or_qwen2_layer_forward(sh, &layers[l], l, kcache, vcache, position, cos_v, sin_v, hidden, threads);
    if (hidden_out) memcpy(hidden_out, hidden, H * sizeof(float));
    if (logits) { /* Prediction::predict (lm.rs:147-166) */
        float *normed = (float *)malloc(H * sizeof(float));
        or_rms_norm(hidden, final_norm, H, sh->eps, normed);
        project_row(sh, table, sh->vocab, H, normed, NULL, logits, threads);
        if (next_token) *next_token = or_greedy(logits, sh->vocab);
        free(normed);
    }
    free(hidden);
    free(inv);
    free(cos_v);
    free(sin_v);
    return 0;
}

/* lm.rs:97-108 */
void or_qwen2_embed(const or_qwen2_shape *sh, const uint8_t *table, const int *ids, size_t count, float *out)
{
    for (size_t r = 0; r < count; r++) or_dequantize_row(sh->dtype, sh->vocab, sh->hidden, table, (size_t)ids[r], out + r * sh->hidden);
}

/* Reader::read (lm.rs:205-228): chunks of rows through the stack, each layer over every row of the
 * chunk before the next layer (Stack::forward_layers). Within a layer the reference projects every
 * row, keeps their keys and values, then attends each row over the keys up to its own position
 * (Mask::Causal, transformer.rs:185-219): row r reads only rows 0..r of the chunk, all kept by then,
 * so taking the rows one after another through or_qwen2_layer_forward is that arithmetic. */
int or_qwen2_read(const or_qwen2_shape *sh, const or_qwen2_layer *layers, const float *final_norm,
                  const uint8_t *table, float *kcache, float *vcache, const float *embeddings, size_t count,
                  size_t first, size_t chunk, float *hidden_out, float *logits, int *next_token, int threads)
{
    size_t H = sh->hidden, half = sh->head_dim / 2;
    if (count == 0 || chunk == 0) return -1;
    if (first + count > sh->capacity) return -1; /* transformer.rs:329-341 */
    float *rows = (float *)malloc(chunk * H * sizeof(float));
    float *inv = (float *)malloc(half * sizeof(float));
    float *cos_v = (float *)malloc(chunk * half * sizeof(float));
    float *sin_v = (float *)malloc(chunk * half * sizeof(float));
    or_rope_inv_freq(sh->rope_base, sh->head_dim, inv);
    for (size_t start = 0; start < count; start += chunk) {
        size_t n = count - start < chunk ? count - start : chunk;
        memcpy(rows, embeddings + start * H, n * H * sizeof(float));
        for (size_t r = 0; r < n; r++) or_rope_angles(inv, half, first + start + r, cos_v + r * half, sin_v + r * half);
        for (size_t l = 0; l < sh->layers; l++)
            for (size_t r = 0; r < n; r++)
                or_qwen2_layer_forward(sh, &layers[l], l, kcache, vcache, first + start + r, cos_v + r * half,
                                       sin_v + r * half, rows + r * H, threads);
        if (start + n == count) {
            const float *last = rows + (n - 1) * H;
            if (hidden_out) memcpy(hidden_out, last, H * sizeof(float));
            if (logits) { /* Prediction::predict (lm.rs:147-166) of the last row */
                float *normed = (float *)malloc(H * sizeof(float));
                or_rms_norm(last, final_norm, H, sh->eps, normed);
                project_row(sh, table, sh->vocab, H, normed, NULL, logits, threads);
                if (next_token) *next_token = or_greedy(logits, sh->vocab);
                free(normed);
            }
        }
    }
    free(rows);
    free(inv);
    free(cos_v);
    free(sin_v);
    return 0;
}
