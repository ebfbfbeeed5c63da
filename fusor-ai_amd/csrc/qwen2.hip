// The Qwen2 decoder step on the device: Transformer::forward with one row and
// Prediction::predict (blocks/src/transformer.rs:185-341, layer.rs:161-344,
// layer/input.rs:22-66, lm.rs:97-179), every projection through the projection kernel.
//
// Five launches per layer, each projection with its neighbours fused in:
//   1. RMSNorm + quantize -> QKV product + bias -> RoPE on query/key heads, keys and values kept
//   2. attention of every query head over the cache (scores, softmax, weighted values), output
//      quantized for the output projection
//   3. output projection added to the residual row
//   4. RMSNorm + quantize -> gate and up products -> silu(gate)·up quantized for down
//   5. down projection added to the residual row
// then RMSNorm + quantize -> head product (logits) with per-workgroup greedy candidates, and the
// greedy token. Elementwise arithmetic is the reference's operation for operation (no fused
// multiply-add; ops::exp's polynomial). Reductions whose order changes f32 bits (RMSNorm's sum of
// squares, the softmax total, the attention's weighted sum) run in the reference's index order when
// the model is exact, or as parallel trees otherwise.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "common.h"
#include "proj.h"

namespace fg {
namespace {

constexpr int kAttnThreads = 256;
constexpr int kAttnRegs = 32;  // float4 per thread for one staged chunk of keys or values

struct AttnParams {
    const float *qkv;  // rotated query heads first
    const float *kcache, *vcache;
    size_t layer_base;
    int heads, kv_heads, D, capacity, keys, chunk;
    int zp;
    int8_t *q;
    float *scales;
    int32_t *corr;
};

__device__ float attn_block_max(float v, float *red)
{
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__device__ float attn_block_sum(float v, float *red)
{
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[4 + (threadIdx.x >> 6)] = v;
    __syncthreads();
    return ((red[4] + red[5]) + red[6]) + red[7];
}

// Rows [j0, j0 + n) of one head of the cache (positions mod capacity) into registers, float4 by
// float4; then into LDS rows of D + 1 floats (conflict-free column reads).
__device__ __forceinline__ void fetch_rows(const float *base, int capacity, int D, int j0, int n, float4 *regs)
{
    const int per_row = D / 4;
#pragma unroll
    for (int r = 0; r < kAttnRegs; r++) {
        const int e = int(threadIdx.x) + r * kAttnThreads;  // float4 index within the chunk
        const int row = e / per_row, c4 = e - row * per_row;
        // branch-free (rows past n re-read row j0), so that every load issues before any wait
        const int rr = row < n ? row : 0;
        regs[r] = *reinterpret_cast<const float4 *>(base + size_t((j0 + rr) % capacity) * D + c4 * 4);
    }
}

__device__ __forceinline__ void stash_rows(const float4 *regs, int D, int n, float *lds)
{
    const int per_row = D / 4, S = D + 1;
#pragma unroll
    for (int r = 0; r < kAttnRegs; r++) {
        const int e = int(threadIdx.x) + r * kAttnThreads;
        const int row = e / per_row, c4 = e - row * per_row;
        if (row < n) {
            float *dst = lds + row * S + c4 * 4;
            dst[0] = regs[r].x;
            dst[1] = regs[r].y;
            dst[2] = regs[r].z;
            dst[3] = regs[r].w;
        }
    }
}

// ops::attend for one query head over positions 0..keys-1 (ops.rs:310-342 under Mask::Causal,
// transformer.rs:185-219): scores = dot_f32(q, k_j)·(1/√D), softmax with ops::exp, the weighted
// sum of values; then the head's output quantized for the output projection.
template <bool EXACT>
__global__ __launch_bounds__(kAttnThreads) void attention_kernel(AttnParams a)
{
    extern __shared__ __align__(16) float ash[];
    const int D = a.D, S = D + 1, keys = a.keys, CH = a.chunk;
    float *rows = ash;                 // [CH][D + 1]
    float *score = rows + CH * S;      // [keys]
    float *query = score + keys;       // [D]
    float *parts = query + D;          // [4][D]
    float *out = parts + 4 * D;        // [D]
    float *red = out + D;              // [16]
    const int head = blockIdx.x;
    const int kv = head / (a.heads / a.kv_heads);
    const float *kbase = a.kcache + a.layer_base + size_t(kv) * a.capacity * D;
    const float *vbase = a.vcache + a.layer_base + size_t(kv) * a.capacity * D;
    float4 regs[kAttnRegs];

    fetch_rows(kbase, a.capacity, D, 0, min(CH, keys), regs);
    for (int i = threadIdx.x; i < D; i += kAttnThreads) query[i] = a.qkv[head * D + i];
    const float scale = 1.0f / sqrtf(float(D));
    float local_max = -INFINITY;
    for (int j0 = 0; j0 < keys; j0 += CH) {
        const int n = min(CH, keys - j0);
        __syncthreads();
        stash_rows(regs, D, n, rows);
        __syncthreads();
        if (j0 + CH < keys) fetch_rows(kbase, a.capacity, D, j0 + CH, min(CH, keys - j0 - CH), regs);
        for (int j = threadIdx.x; j < n; j += kAttnThreads) {
            const float *k = rows + j * S;
            float s = -0.0f;  // dot_f32 in index order
            for (int d = 0; d < D; d += 16) {
                float qv[16], kv[16];
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    qv[e] = query[d + e];
                    kv[e] = k[d + e];
                }
#pragma unroll
                for (int e = 0; e < 16; e++) s = s + qv[e] * kv[e];
            }
            s = s * scale;
            score[j0 + j] = s;
            local_max = fmaxf(local_max, s);
        }
    }
    // the first chunk of values is on its way while the softmax runs
    fetch_rows(vbase, a.capacity, D, 0, min(CH, keys), regs);
    const float peak = attn_block_max(local_max, red);
    for (int j = threadIdx.x; j < keys; j += kAttnThreads) score[j] = ref_exp(score[j] - peak);
    __syncthreads();
    float total;
    if (EXACT) {
        if (threadIdx.x == 0) {
            float t = -0.0f;
            int j = 0;
            for (; j + 16 <= keys; j += 16) {
                float v[16];
#pragma unroll
                for (int e = 0; e < 16; e++) v[e] = score[j + e];
#pragma unroll
                for (int e = 0; e < 16; e++) t = t + v[e];
            }
            for (; j < keys; j++) t = t + score[j];
            red[8] = t;
        }
        __syncthreads();
        total = red[8];
    } else {
        float p = 0.0f;
        for (int j = threadIdx.x; j < keys; j += kAttnThreads) p = p + score[j];
        total = attn_block_sum(p, red);
    }
    for (int j = threadIdx.x; j < keys; j += kAttnThreads) score[j] = score[j] / total;
    // weigh (ops.rs:329-342): out[i] = Σ_j w_j·v_j[i], from +0; exact: index order per output
    const int slices = EXACT ? 1 : min(4, kAttnThreads / D);
    const int slice = int(threadIdx.x) / D, i = int(threadIdx.x) - slice * D;
    float o = 0.0f;
    for (int j0 = 0; j0 < keys; j0 += CH) {
        const int n = min(CH, keys - j0);
        __syncthreads();
        stash_rows(regs, D, n, rows);
        __syncthreads();
        if (j0 + CH < keys) fetch_rows(vbase, a.capacity, D, j0 + CH, min(CH, keys - j0 - CH), regs);
        if (slice < slices) {
            int j = slice;
            for (; j + 16 * slices <= n; j += 16 * slices) {
                float w[16], v[16];
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    w[e] = score[j0 + j + e * slices];
                    v[e] = rows[(j + e * slices) * S + i];
                }
#pragma unroll
                for (int e = 0; e < 16; e++) o = o + w[e] * v[e];
            }
            for (; j < n; j += slices) o = o + score[j0 + j] * rows[j * S + i];
        }
    }
    if (slice < slices) parts[slice * D + i] = o;
    __syncthreads();
    for (int k = threadIdx.x; k < D; k += kAttnThreads) {
        float v = parts[k];
        for (int s2 = 1; s2 < slices; s2++) v = v + parts[s2 * D + k];
        out[k] = v;
    }
    __syncthreads();
    // quantize the head's D outputs (D / 32 groups), 8 lanes per group
    const int groups = D / 32;
    const int sub = threadIdx.x & 7, g = threadIdx.x >> 3;
    const bool active = g < groups;
    float x0 = 0, x1 = 0, x2 = 0, x3 = 0;
    if (active) {
        x0 = out[g * 32 + sub * 4];
        x1 = out[g * 32 + sub * 4 + 1];
        x2 = out[g * 32 + sub * 4 + 2];
        x3 = out[g * 32 + sub * 4 + 3];
    }
    float amax = fmaxf(fmaxf(fabsf(x0), fabsf(x1)), fmaxf(fabsf(x2), fabsf(x3)));
    amax = fmaxf(0.0f, amax);
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
    const float d = group_scale(amax, 127.0f);
    const int l0 = quantize_level(x0, d), l1 = quantize_level(x1, d), l2 = quantize_level(x2, d), l3 = quantize_level(x3, d);
    int sum = l0 + l1 + l2 + l3;
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    sum += __shfl_xor(sum, 4, 64);
    if (active) {
        const int G = head * groups + g;
        reinterpret_cast<int *>(a.q)[G * 8 + sub] = pack4(l0, l1, l2, l3);
        if (sub == 0) {
            a.scales[G] = d;
            a.corr[G] = -a.zp * sum;
        }
    }
}

// Prediction::greedy (lm.rs:169-179) over the head's per-workgroup candidates: the first index of
// the largest logit; NaNs never win, and a NaN first logit keeps index 0.
__global__ __launch_bounds__(1024) void greedy_kernel(const float *__restrict__ pval, const int32_t *__restrict__ pidx, int n,
                                                      const float *__restrict__ logits, int32_t *out)
{
    __shared__ float bv[16];
    __shared__ int bi[16];
    float best = 0.0f;
    int idx = -1;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int ci = pidx[i];
        const float cv = pval[i];
        if (ci >= 0 && (idx < 0 || cv > best || (cv == best && ci < idx))) {
            best = cv;
            idx = ci;
        }
    }
    for (int m = 32; m >= 1; m >>= 1) {
        const float ob = __shfl_xor(best, m, 64);
        const int oi = __shfl_xor(idx, m, 64);
        if (oi >= 0 && (idx < 0 || ob > best || (ob == best && oi < idx))) {
            best = ob;
            idx = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        bv[threadIdx.x >> 6] = best;
        bi[threadIdx.x >> 6] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < int(blockDim.x >> 6); w++) {
            if (bi[w] >= 0 && (idx < 0 || bv[w] > best || (bv[w] == best && bi[w] < idx))) {
                best = bv[w];
                idx = bi[w];
            }
        }
        const float first = logits[0];
        *out = (first != first || idx < 0) ? 0 : idx;
    }
}

}  // namespace
}  // namespace fg

using namespace fg;

struct fg_qwen2 {
    fg_qwen2_shape shape;
    std::vector<fg_qwen2_layer> layers;
    const float *final_norm;
    const fg_table *table;
    float *kcache, *vcache;
    // activations
    float *hidden, *qkv, *logits, *rope;  // rope: [capacity][cos | sin]
    int8_t *xq;
    float *xs;
    int32_t *xc;
    float *pval;
    int32_t *pidx;
    int head_groups;  // workgroups of the head product (greedy candidates)
    int attn_chunk;
    size_t attn_smem;
    int zp;
};

namespace {

ProjParams table_params(const fg_table *t)
{
    ProjParams p{};
    p.codes = t->codes;
    p.wscales = t->scales;
    p.B = int(t->blocks);
    p.G = int(t->groups);
    p.K = int(t->cols);
    p.n_rows = int(t->rows);
    p.quad_begin = 0;
    p.quad_end = int(t->quads);
    return p;
}

// 1. RMSNorm -> QKV + bias -> RoPE, keys and values kept.
int qkv_launch(fg_qwen2 *m, const fg_qwen2_layer &ly, size_t li, size_t position, hipStream_t st)
{
    const fg_qwen2_shape &sh = m->shape;
    ProjParams p = table_params(ly.qkv);
    p.qpw = int(sh.head_dim / 4);  // one head per workgroup
    p.x = m->hidden;
    p.norm_w = ly.norm1;
    p.eps = sh.eps;
    p.zp = m->zp;
    p.bias = ly.qkv_bias;
    p.qkv_out = m->qkv;
    p.rope = m->rope + position * sh.head_dim;
    p.heads = int(sh.heads);
    p.kv_heads = int(sh.kv_heads);
    p.D = int(sh.head_dim);
    p.kcache = m->kcache;
    p.vcache = m->vcache;
    p.layer_base = li * sh.kv_heads * sh.capacity * sh.head_dim;
    p.capacity = int(sh.capacity);
    p.position = int(position);
    return launch_proj(p, sh.dtype, IN_NORM, OUT_QKV, sh.exact != 0, st);
}

// 3. and 5. a projection of the prepared input added to the residual row.
int residual_launch(fg_qwen2 *m, const fg_table *t, hipStream_t st)
{
    ProjParams p = table_params(t);
    p.qpw = 1;
    p.q = m->xq;
    p.as = m->xs;
    p.corr = m->xc;
    p.zp = m->zp;
    p.out = m->hidden;
    p.ld_out = long(t->quads * 4);
    p.accumulate = 1;
    return launch_proj(p, m->shape.dtype, IN_PREQ, OUT_STORE, false, st);
}

// 4. RMSNorm -> gate and up -> silu(gate)·up quantized for down.
int swiglu_launch(fg_qwen2 *m, const fg_qwen2_layer &ly, hipStream_t st)
{
    const fg_qwen2_shape &sh = m->shape;
    ProjParams p = table_params(ly.gate);
    p.codes2 = ly.up->codes;
    p.wscales2 = ly.up->scales;
    p.qpw = 8;  // 32 outputs: one group of the down projection's input
    p.x = m->hidden;
    p.norm_w = ly.norm2;
    p.eps = sh.eps;
    p.zp = m->zp;
    p.q_out = m->xq;
    p.s_out = m->xs;
    p.c_out = m->xc;
    p.zp_out = m->zp;
    return launch_proj(p, sh.dtype, IN_NORM, OUT_SWIGLU, sh.exact != 0, st);
}

int attention_launch(fg_qwen2 *m, size_t li, size_t position, hipStream_t st)
{
    const fg_qwen2_shape &sh = m->shape;
    AttnParams a{};
    a.qkv = m->qkv;
    a.kcache = m->kcache;
    a.vcache = m->vcache;
    a.layer_base = li * sh.kv_heads * sh.capacity * sh.head_dim;
    a.heads = int(sh.heads);
    a.kv_heads = int(sh.kv_heads);
    a.D = int(sh.head_dim);
    a.capacity = int(sh.capacity);
    a.keys = int(position) + 1;
    a.chunk = m->attn_chunk;
    a.zp = m->zp;
    a.q = m->xq;
    a.scales = m->xs;
    a.corr = m->xc;
    if (sh.exact) attention_kernel<true><<<unsigned(sh.heads), kAttnThreads, m->attn_smem, st>>>(a);
    else attention_kernel<false><<<unsigned(sh.heads), kAttnThreads, m->attn_smem, st>>>(a);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

int run_layer(fg_qwen2 *m, size_t li, size_t position, hipStream_t st)
{
    const fg_qwen2_layer &ly = m->layers[li];
    int rc;
    if ((rc = qkv_launch(m, ly, li, position, st))) return rc;
    if ((rc = attention_launch(m, li, position, st))) return rc;
    if ((rc = residual_launch(m, ly.o, st))) return rc;
    if ((rc = swiglu_launch(m, ly, st))) return rc;
    return residual_launch(m, ly.down, st);
}

int head_launch(fg_qwen2 *m, hipStream_t st)
{
    const fg_qwen2_shape &sh = m->shape;
    ProjParams p = table_params(m->table);
    p.qpw = 64;
    p.x = m->hidden;
    p.norm_w = m->final_norm;
    p.eps = sh.eps;
    p.zp = m->zp;
    p.out = m->logits;
    p.ld_out = long(m->table->quads * 4);
    p.pval = m->pval;
    p.pidx = m->pidx;
    return launch_proj(p, sh.dtype, IN_NORM, OUT_STORE, sh.exact != 0, st);
}

bool table_is(const fg_table *t, int dtype, size_t rows, size_t cols)
{
    return t && t->dtype == dtype && t->rows == rows && t->cols == cols;
}

}  // namespace

extern "C" int fg_qwen2_create(const fg_qwen2_shape *shape, const fg_qwen2_layer *layers, const float *final_norm,
                               const fg_table *table, float *kcache, float *vcache, fg_qwen2 **out)
{
    if (!shape || !layers || !final_norm || !table || !kcache || !vcache || !out)
        return set_error(FG_ERR_ARG, "fg_qwen2_create: a null argument");
    const fg_qwen2_shape sh = *shape;
    if (sh.dtype != FG_Q7B32 && sh.dtype != FG_Q8B32 && sh.dtype != FG_Q4B32)
        return set_error(FG_ERR_FORMAT, "fg_qwen2_create: weights must be Q7b32, Q8b32 or Q4b32");
    if (sh.kv_heads == 0 || sh.heads % sh.kv_heads != 0)
        return set_error(FG_ERR_SHAPE, "fg_qwen2_create: heads must be a multiple of kv_heads");
    if (sh.head_dim != 32 && sh.head_dim != 64 && sh.head_dim != 128)
        return set_error(FG_ERR_SHAPE, "fg_qwen2_create: head_dim must be 32, 64 or 128");
    if (sh.hidden % 32 || sh.ffn % 32 || sh.hidden > 16384 || sh.capacity == 0 || sh.capacity > 8192)
        return set_error(FG_ERR_SHAPE, "fg_qwen2_create: hidden and ffn must be whole groups (hidden <= 16384, capacity <= 8192)");
    const size_t qkv_w = (sh.heads + 2 * sh.kv_heads) * sh.head_dim, width = sh.heads * sh.head_dim;
    for (size_t l = 0; l < sh.layers; l++) {
        const fg_qwen2_layer &ly = layers[l];
        if (!ly.norm1 || !ly.norm2 || !table_is(ly.qkv, sh.dtype, qkv_w, sh.hidden) || !table_is(ly.o, sh.dtype, sh.hidden, width) ||
            !table_is(ly.gate, sh.dtype, sh.ffn, sh.hidden) || !table_is(ly.up, sh.dtype, sh.ffn, sh.hidden) ||
            !table_is(ly.down, sh.dtype, sh.hidden, sh.ffn))
            return set_error(FG_ERR_SHAPE, "fg_qwen2_create: layer " + std::to_string(l) + " tables do not fit the shape");
    }
    if (!table_is(table, sh.dtype, sh.vocab, sh.hidden)) return set_error(FG_ERR_SHAPE, "fg_qwen2_create: the table is not [vocab, hidden]");
    fg_qwen2 *m = new fg_qwen2();
    m->shape = sh;
    m->layers.assign(layers, layers + sh.layers);
    m->final_norm = final_norm;
    m->table = table;
    m->kcache = kcache;
    m->vcache = vcache;
    m->zp = zero_point_of(sh.dtype);
    m->head_groups = int((table->quads + 63) / 64);
    // attention: chunks of keys staged in LDS, kAttnRegs float4 per thread
    const int D = int(sh.head_dim);
    m->attn_chunk = kAttnRegs * kAttnThreads * 4 / D;
    const size_t keys = sh.capacity;
    m->attn_smem = (size_t(m->attn_chunk) * (D + 1) + keys + D + 4 * D + D + 16) * 4;
    if (m->attn_smem > 160 * 1024) {
        delete m;
        return set_error(FG_ERR_SHAPE, "fg_qwen2_create: the attention does not fit in LDS");
    }
    const size_t widest = std::max(sh.hidden, std::max(width, sh.ffn));
    const size_t padded_vocab = table->quads * 4;
    struct Alloc {
        void **ptr;
        size_t bytes;
    } allocs[] = {
        {reinterpret_cast<void **>(&m->hidden), sh.hidden * 4},
        {reinterpret_cast<void **>(&m->qkv), (qkv_w + 3) / 4 * 4 * 4},
        {reinterpret_cast<void **>(&m->logits), padded_vocab * 4},
        {reinterpret_cast<void **>(&m->rope), sh.capacity * sh.head_dim * 4},
        {reinterpret_cast<void **>(&m->xq), widest},
        {reinterpret_cast<void **>(&m->xs), widest / 32 * 4},
        {reinterpret_cast<void **>(&m->xc), widest / 32 * 4},
        {reinterpret_cast<void **>(&m->pval), size_t(m->head_groups) * 4},
        {reinterpret_cast<void **>(&m->pidx), size_t(m->head_groups) * 4},
    };
    for (auto &a : allocs) {
        hipError_t e = hipMalloc(a.ptr, a.bytes);
        if (e != hipSuccess) {
            int rc = check_hip(e, "fg_qwen2_create: hipMalloc");
            fg_qwen2_free(m);
            return rc;
        }
    }
    hipError_t e = hipSuccess;
    if (m->attn_smem > 64 * 1024) {
        e = hipFuncSetAttribute(reinterpret_cast<const void *>(attention_kernel<true>), hipFuncAttributeMaxDynamicSharedMemorySize,
                                160 * 1024);
        if (e == hipSuccess)
            e = hipFuncSetAttribute(reinterpret_cast<const void *>(attention_kernel<false>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    }
    // Rotary angles per position (blocks/src/rotary.rs angles; ops.rs:70-74), on the host in f32
    // with the C library's powf/cosf/sinf, as the reference computes them.
    const size_t half = sh.head_dim / 2;
    std::vector<float> inv(half), rope(sh.capacity * sh.head_dim);
    for (size_t i = 0; i < half; i++) inv[i] = 1.0f / powf(sh.rope_base, float(2 * i) / float(sh.head_dim));
    for (size_t p = 0; p < sh.capacity; p++)
        for (size_t i = 0; i < half; i++) {
            const float angle = float(p) * inv[i];
            rope[p * sh.head_dim + i] = cosf(angle);
            rope[p * sh.head_dim + half + i] = sinf(angle);
        }
    if (e == hipSuccess) e = hipMemcpy(m->rope, rope.data(), rope.size() * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        int rc = check_hip(e, "fg_qwen2_create");
        fg_qwen2_free(m);
        return rc;
    }
    *out = m;
    return FG_OK;
}

extern "C" int fg_qwen2_layer_forward(fg_qwen2 *m, size_t layer, size_t position, float *hidden, void *stream)
{
    if (!m || !hidden) return set_error(FG_ERR_ARG, "fg_qwen2_layer_forward: a null argument");
    if (layer >= m->shape.layers || position >= m->shape.capacity)
        return set_error(FG_ERR_SHAPE, "fg_qwen2_layer_forward: layer or position out of range");
    hipStream_t st = as_stream(stream);
    FG_HIP(hipMemcpyAsync(m->hidden, hidden, m->shape.hidden * 4, hipMemcpyDeviceToDevice, st));
    int rc = run_layer(m, layer, position, st);
    if (rc) return rc;
    FG_HIP(hipMemcpyAsync(hidden, m->hidden, m->shape.hidden * 4, hipMemcpyDeviceToDevice, st));
    return FG_OK;
}

extern "C" int fg_qwen2_step(fg_qwen2 *m, int token, size_t position, float *hidden, float *logits, int32_t *next_token,
                             void *stream)
{
    if (!m) return set_error(FG_ERR_ARG, "fg_qwen2_step: a null model");
    const fg_qwen2_shape &sh = m->shape;
    // transformer.rs:329-341: the cache holds every key the span sees
    if (position >= sh.capacity) return set_error(FG_ERR_SHAPE, "fg_qwen2_step: the cache holds every key the span sees");
    if (token < 0 || size_t(token) >= sh.vocab) return set_error(FG_ERR_SHAPE, "fg_qwen2_step: token out of the vocabulary");
    hipStream_t st = as_stream(stream);
    int rc = launch_dequantize_row(m->table, size_t(token), m->hidden, st);  // lm.rs:99-107
    if (rc) return rc;
    for (size_t l = 0; l < sh.layers; l++)
        if ((rc = run_layer(m, l, position, st))) return rc;
    if (hidden) FG_HIP(hipMemcpyAsync(hidden, m->hidden, sh.hidden * 4, hipMemcpyDeviceToDevice, st));
    if (logits || next_token) {
        if ((rc = head_launch(m, st))) return rc;
        if (logits) FG_HIP(hipMemcpyAsync(logits, m->logits, sh.vocab * 4, hipMemcpyDeviceToDevice, st));
        if (next_token) {
            greedy_kernel<<<1, 1024, 0, st>>>(m->pval, m->pidx, m->head_groups, m->logits, next_token);
            FG_HIP(hipGetLastError());
        }
    }
    return FG_OK;
}

extern "C" int fg_qwen2_free(fg_qwen2 *m)
{
    if (!m) return FG_OK;
    void *ptrs[] = {m->hidden, m->qkv, m->logits, m->rope, m->xq, m->xs, m->xc, m->pval, m->pidx};
    for (void *p : ptrs)
        if (p) (void)hipFree(p);
    delete m;
    return FG_OK;
}
