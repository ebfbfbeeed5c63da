// The projection kernel's parameter block, modes and LDS layout, shared by the generic product
// and the decoder.
#pragma once

#include "common.h"

namespace fg {

// Input of a projection: rows already quantized, f32 rows quantized in-kernel, one f32 row
// RMS-normalized then quantized in-kernel (rms_norm, ops.rs:7-16), or the attention's output row
// merged from per-chunk softmax states, then quantized.
constexpr int IN_PREQ = 0, IN_F32 = 1, IN_NORM = 2, IN_ATTN = 3, IN_EMBED = 4;
// Chunks of keys per query head in the fast attention; the output projection merges them.
constexpr int kMaxChunks = 8;
constexpr int kTileKeys = 64;  // keys per tile of the fast attention
// Output: store (bias / residual / greedy candidates), the int32 group accumulators, the QKV
// epilogue, the gated feed-forward epilogue, and the query heads attended over chunks of the
// cached keys (with the new key and value rows) in one launch.
constexpr int OUT_STORE = 0, OUT_DOTS = 1, OUT_QKV = 2, OUT_SWIGLU = 3, OUT_QATTN = 4;

struct ProjParams {
    const int8_t *codes, *codes2;      // device table(s); codes2 is the SwiGLU up table
    const float *wscales, *wscales2;
    int B, G, K, n_rows;
    // Workgroup w owns quads base + j·qstride, j < qpw, base = quad_begin + (w / qstride)·qstride·qpw
    // + w % qstride: consecutive quads when qstride is 1; the two halves of a rotary pair (quads
    // D/8 apart) when the QKV epilogue asks for qstride = D/8, qpw = 2.
    int quad_begin, quad_end, qpw, qstride;
    int qshift;  // log2 qstride (set by the launcher)
    // Set by the launcher (proj_derive): reciprocals for exact small quotients (divq), log2 D
    float rcp_B, rcp_chunks, rcp_group;
    int dshift;
    // input
    const float *x;
    const int8_t *q;
    const float *as;
    const int32_t *corr;
    int zp;
    const float *norm_w;
    // IN_EMBED: RMSNorm of a table row (Buffers::embed_row, lm.rs:99-107), dequantized in the
    // prologue from the row's quad (its codes and scales) and lane; workgroup 0 also stores the
    // row to x_out
    const int8_t *e_codes;
    const float *e_scales;
    int e_lane;
    float *x_out;
    float eps;
    // IN_ATTN: per (head, chunk) records of D + 4 floats (max, total, -, -, sums), merged with the
    // new key's own state (rotated query in qkv_out, key and value at the position in the caches)
    const float *part;
    int chunks;
    float *merged_out;  // when set, workgroup 0 also writes the merged f32 row (an inspection)
    // store
    const float *bias;
    float *out;
    long ld_out;
    int col_begin, accumulate;
    int32_t *dots;
    int dots_cols;
    float *pval;  // greedy candidates per workgroup, or null
    int32_t *pidx;
    // QKV epilogue
    float *qkv_out;
    const float *rope;  // cos[half] then sin[half] of the position
    int heads, kv_heads, D;
    float *kcache, *vcache;
    size_t layer_base;
    int capacity, position;
    // SwiGLU epilogue: silu(gate)·up, f32 (when set)
    float *act_out;
    // OUT_SWIGLU with 8 quads per workgroup (32 outputs, one group of 32): the row also quantized
    // per group (quantize_rows' levels, scales and corrections), when q_out is set
    int8_t *q_out;
    float *s_out;
    int32_t *c_out;
    // OUT_QATTN: workgroup w < heads·chunks projects query head w / chunks (its D rows) and attends
    // over keys [c·per_chunk, min((c + 1)·per_chunk, position)) of chunk c = w % chunks, writing the
    // chunk's record to `states`; the rest project the key and value rows in rotary pairs
    int per_chunk;
    float *states;
    // ... in the exact order, the chunk's scores instead: [heads][capacity]
    float *scores;
};

// a / b for 0 <= a < 2^22 and b >= 1 from rcp = fl(1/b): (a + 1/2)/b is at least 1/(2b) from
// an integer, and the two roundings move it by less than that, so the floor is the quotient.
__device__ __forceinline__ int divq(int a, float rcp) { return int((float(a) + 0.5f) * rcp); }

// The launcher's derived fields of a parameter block.
inline void proj_derive(ProjParams &p)
{
    p.rcp_B = 1.0f / float(p.B > 0 ? p.B : 1);
    p.rcp_chunks = 1.0f / float(p.chunks > 0 ? p.chunks : 1);
    p.rcp_group = 1.0f / float(p.kv_heads > 0 && p.heads >= p.kv_heads ? p.heads / p.kv_heads : 1);
    p.dshift = p.D > 0 ? __builtin_ctz(unsigned(p.D)) : 0;
}

// Byte offsets of the LDS regions (every region 16-byte aligned).
struct ProjLayout {
    int off_s, off_c, off_red, off_y, off_terms, off_n, off_att, total;
};

__host__ __device__ inline int align16(int b) { return (b + 15) & ~15; }

__host__ __device__ inline ProjLayout proj_layout(int R, int K, int G, int NW, int in, int out)
{
    const int NT = out == OUT_SWIGLU ? 2 : 1;
    const int ny = out == OUT_SWIGLU ? 2 : 1;
    ProjLayout l;
    l.off_s = align16(R * K);
    l.off_c = l.off_s + align16(R * G * 4);
    l.off_red = l.off_c + align16(R * G * 4);
    l.off_y = l.off_red + 16 * 4;
    l.off_terms = l.off_y + align16(ny * R * NW * 4);
    l.off_n = l.off_terms + (out == OUT_DOTS ? 0 : align16(NT * R * NW * ((G + 3) & ~3) * 4 + 4));  // + a spare slot
    l.off_att = l.off_n + (in == IN_NORM || in == IN_EMBED ? align16(K * 4) : 0);  // the exact RMSNorm's row
    // OUT_QATTN: the rotated query [NW = D], the waves' maxima and totals [8] and weighted sums [4][D]
    l.total = l.off_att + (out == OUT_QATTN ? align16((NW + 8 + 4 * NW) * 4) : 0);
    return l;
}

// ops::exp (ops.rs:97-131): clamp, n = round(x·log2 e), r = x − n·ln2_hi − n·ln2_lo, Cephes
// polynomial in Horner order, times 2^n through the exponent bits. No fused multiply-add.
__device__ __forceinline__ float ref_exp(float x)
{
    x = x < -87.0f ? -87.0f : (x > 88.0f ? 88.0f : x);
    const float exponent = __builtin_rintf(x * 1.44269504088896340736f);
    const float remainder = x - exponent * 0.6933594f - exponent * -2.1219444e-4f;
    float poly = 1.9875691e-4f;
    poly = poly * remainder + 1.3981999e-3f;
    poly = poly * remainder + 8.333452e-3f;
    poly = poly * remainder + 4.1665796e-2f;
    poly = poly * remainder + 0.16666666f;
    poly = poly * remainder + 0.5f;
    poly = poly * remainder * remainder + remainder + 1.0f;
    const int bits = (int(exponent) + 127) << 23;
    return poly * __int_as_float(bits);
}

// ops::silu (ops.rs:272-274)
__device__ __forceinline__ float ref_silu(float x) { return x / (1.0f + ref_exp(-x)); }

size_t proj_smem(const ProjParams &p, int rows, int in, int out);
int launch_proj(const ProjParams &p, int dtype, int in, int out, bool exact, hipStream_t s);
int launch_norm_quantize(const ProjParams &p, bool exact, hipStream_t s);
// The same for `rows` rows: x [rows][K] to q_out [rows][K], s_out and c_out [rows][G].
int launch_norm_quantize_rows(const ProjParams &p, int rows, bool exact, hipStream_t s);

}  // namespace fg
