// The Qwen2 decoder step on the device: Transformer::forward with one row and
// Prediction::predict (blocks/src/transformer.rs:185-341, layer.rs:161-344,
// layer/input.rs:22-66, lm.rs:97-179), every projection through the product kernels.
//
// Between projections the activations stay on the device: each producer writes the next
// projection's input already quantized (levels, scales, corrections), as `prepare` does
// (layer/input.rs:22-66). Elementwise arithmetic is the reference's, operation for operation
// (no fused multiply-add; the exponential is ops::exp's polynomial). Reductions whose order
// changes f32 bits (RMSNorm's sum of squares, the softmax total, the attention's weighted sum)
// run in the reference's index order when the model is exact, or as parallel trees otherwise.
#include <cmath>
#include <cstring>
#include <vector>

#include "common.h"

namespace fg {
namespace {

constexpr int kNormThreads = 256;

// ops::exp (ops.rs:97-131): clamp, n = round(x·log2 e), r = x − n·ln2_hi − n·ln2_lo, Cephes
// polynomial in Horner order, times 2^n through the exponent bits.
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

// Quantize `n` (a multiple of 32) LDS values into q/scales/corrections at group `g0`, 8 lanes
// per group of 32 (quantize_rows, matmul.rs:233-257). All threads of the block take part.
__device__ void quantize_lds(const float *v, int n, int g0, int zp, int8_t *q, float *scales, int32_t *corr)
{
    const int sub = threadIdx.x & 7;
    const int groups = n / 32;
    const int rounds = (groups + int(blockDim.x) / 8 - 1) / (int(blockDim.x) / 8);
    for (int round = 0; round < rounds; round++) {
        const int g = round * (int(blockDim.x) / 8) + int(threadIdx.x >> 3);
        const bool active = g < groups;
        float x0 = 0, x1 = 0, x2 = 0, x3 = 0;
        if (active) {
            x0 = v[g * 32 + sub * 4];
            x1 = v[g * 32 + sub * 4 + 1];
            x2 = v[g * 32 + sub * 4 + 2];
            x3 = v[g * 32 + sub * 4 + 3];
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
            reinterpret_cast<int *>(q)[(g0 + g) * 8 + sub] = pack4(l0, l1, l2, l3);
            if (sub == 0) {
                scales[g0 + g] = d;
                corr[g0 + g] = -zp * sum;
            }
        }
    }
}

// A float sum over the block; the result is in every thread.
__device__ float block_sum(float v, float *red)
{
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    const int wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
    for (int w = 0; w < waves; w++) t = t + red[w];
    return t;
}

__device__ float block_max(float v, float *red)
{
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    const int wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float t = red[0];
    for (int w = 1; w < waves; w++) t = fmaxf(t, red[w]);
    return t;
}

// rms_norm (ops.rs:7-16) then quantize_rows: the projection's prepared input.
template <bool EXACT>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_quant_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                                    int H, float eps, int zp, int8_t *q, float *scales,
                                                                    int32_t *corr, float *normed_out)
{
    extern __shared__ float sh[];
    float *v = sh;            // [H]
    float *red = sh + H;      // [waves + 1]
    for (int i = threadIdx.x; i < H; i += blockDim.x) v[i] = x[i];
    __syncthreads();
    float total;
    if (EXACT) {
        // dot_f32(row, row): products summed in index order from -0.0 (arch/scalar.rs:340-342)
        if (threadIdx.x == 0) {
            float s = -0.0f;
            for (int i = 0; i < H; i++) s = s + v[i] * v[i];
            red[0] = s;
        }
        __syncthreads();
        total = red[0];
        __syncthreads();
    } else {
        float part = 0.0f;
        for (int i = threadIdx.x; i < H; i += blockDim.x) part = part + v[i] * v[i];
        total = block_sum(part, red);
    }
    const float mean = total / float(H);
    const float inverse = 1.0f / sqrtf(mean + eps);
    __syncthreads();
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        const float n = v[i] * inverse * w[i];
        v[i] = n;
        if (normed_out) normed_out[i] = n;
    }
    __syncthreads();
    quantize_lds(v, H, 0, zp, q, scales, corr);
}

// rope_half on the query and key heads (ops.rs:77-85), then KvCache::keep of the key and
// value heads (transformer.rs:166-180). One thread per (unit, i < head_dim / 2).
__global__ void rope_keep_kernel(float *__restrict__ qkv, const float *__restrict__ cos_t, const float *__restrict__ sin_t,
                                 int heads, int kv_heads, int D, float *__restrict__ kcache, float *__restrict__ vcache,
                                 size_t layer_base, int capacity, int position)
{
    const int half = D / 2;
    const int id = int(blockIdx.x) * int(blockDim.x) + int(threadIdx.x);
    const int units = heads + 2 * kv_heads;
    if (id >= units * half) return;
    const int unit = id / half, i = id % half;
    float *head = qkv + unit * D;
    float x = head[i], y = head[i + half];
    if (unit < heads + kv_heads) {
        const float c = cos_t[i], s = sin_t[i];
        const float nx = x * c - y * s;
        const float ny = y * c + x * s;
        x = nx;
        y = ny;
        head[i] = x;
        head[i + half] = y;
    }
    if (unit >= heads) {
        const bool key = unit < heads + kv_heads;
        const int kv = (unit - heads) % kv_heads;
        float *cache = key ? kcache : vcache;
        const size_t at = layer_base + (size_t(kv) * capacity + size_t(position % capacity)) * D;
        cache[at + i] = x;
        cache[at + i + half] = y;
    }
}

// ops::attend for one query head over positions 0..=position (ops.rs:310-342, under
// Mask::Causal, transformer.rs:185-219), then the head's output quantized for the output
// projection (two groups of 32 per 64-wide head).
template <bool EXACT>
__global__ __launch_bounds__(256) void attention_kernel(const float *__restrict__ qkv, const float *__restrict__ kcache,
                                                        const float *__restrict__ vcache, size_t layer_base, int heads,
                                                        int kv_heads, int D, int capacity, int keys, int zp, int8_t *q,
                                                        float *scales, int32_t *corr, float *attn_out)
{
    extern __shared__ float sh[];
    float *query = sh;                 // [D]
    float *out = sh + D;               // [D]
    float *part = out + D;             // [4][D]
    float *red = part + 4 * D;         // [8]
    float *score = red + 8;            // [keys]
    const int head = blockIdx.x;
    const int kv = head / (heads / kv_heads);
    const float *kbase = kcache + layer_base + size_t(kv) * capacity * D;
    const float *vbase = vcache + layer_base + size_t(kv) * capacity * D;
    for (int i = threadIdx.x; i < D; i += blockDim.x) query[i] = qkv[head * D + i];
    __syncthreads();
    const float scale = 1.0f / sqrtf(float(D));
    float local_max = -INFINITY;
    for (int j = threadIdx.x; j < keys; j += blockDim.x) {
        const float *k = kbase + size_t(j % capacity) * D;
        float s = -0.0f;  // dot_f32 in index order
        for (int d = 0; d < D; d++) s = s + query[d] * k[d];
        s = s * scale;
        score[j] = s;
        local_max = fmaxf(local_max, s);
    }
    const float peak = block_max(local_max, red);
    for (int j = threadIdx.x; j < keys; j += blockDim.x) score[j] = ref_exp(score[j] - peak);
    __syncthreads();
    float total;
    if (EXACT) {
        if (threadIdx.x == 0) {
            float t = -0.0f;
            for (int j = 0; j < keys; j++) t = t + score[j];
            red[0] = t;
        }
        __syncthreads();
        total = red[0];
    } else {
        float p = 0.0f;
        for (int j = threadIdx.x; j < keys; j += blockDim.x) p = p + score[j];
        total = block_sum(p, red);
    }
    __syncthreads();
    for (int j = threadIdx.x; j < keys; j += blockDim.x) score[j] = score[j] / total;
    __syncthreads();
    if (EXACT) {
        // weigh: out[i] = Σ_j w_j·v_j[i] in index order from +0 (ops.rs:329-342)
        for (int i = threadIdx.x; i < D; i += blockDim.x) {
            float o = 0.0f;
            for (int j = 0; j < keys; j++) o = o + score[j] * vbase[size_t(j % capacity) * D + i];
            out[i] = o;
        }
    } else {
        // up to four slices of the keys per output, then the slices added in order
        const int slices = min(4, max(1, int(blockDim.x) / D));
        for (int t = threadIdx.x; t < slices * D; t += blockDim.x) {
            const int slice = t / D, i = t % D;
            float o = 0.0f;
            for (int j = slice; j < keys; j += slices) o = o + score[j] * vbase[size_t(j % capacity) * D + i];
            part[slice * D + i] = o;
        }
        __syncthreads();
        for (int i2 = threadIdx.x; i2 < D; i2 += blockDim.x) {
            float o = part[i2];
            for (int s2 = 1; s2 < slices; s2++) o = o + part[s2 * D + i2];
            out[i2] = o;
        }
    }
    __syncthreads();
    if (attn_out)
        for (int i = threadIdx.x; i < D; i += blockDim.x) attn_out[head * D + i] = out[i];
    quantize_lds(out, D, head * D / 32, zp, q, scales, corr);
}

// The gated feed-forward's inner values (layer.rs:321-341): silu(gate) · up, quantized for down.
__global__ __launch_bounds__(256) void silu_mul_quant_kernel(const float *__restrict__ gate, const float *__restrict__ up,
                                                             int n, int zp, int8_t *q, float *scales, int32_t *corr)
{
    __shared__ float v[256 * 4];
    const int base = int(blockIdx.x) * 1024;
    for (int i = threadIdx.x; i < 1024; i += blockDim.x) {
        const int k = base + i;
        v[i] = k < n ? ref_silu(gate[k]) * up[k] : 0.0f;
    }
    __syncthreads();
    const int len = min(1024, n - base);
    quantize_lds(v, len, base / 32, zp, q, scales, corr);
}

// Prediction::greedy (lm.rs:169-179): the first index of the largest logit; NaNs never win,
// and a NaN first logit keeps index 0.
__global__ __launch_bounds__(1024) void argmax_kernel(const float *__restrict__ logits, int n, int32_t *out)
{
    __shared__ float bv[16];
    __shared__ int bi[16];
    float best = -INFINITY;
    int idx = -1;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float x = logits[i];
        if (x == x && (idx < 0 || x > best)) {
            best = x;
            idx = i;
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
    float *hidden, *qkv, *gate, *up, *logits, *rope;  // rope: [capacity][cos | sin]
    int8_t *xq;
    float *xs;
    int32_t *xc;
    int32_t *token;
    int zp;
};

namespace {

int product(const fg_table *t, const int8_t *q, const float *s, const int32_t *c, const float *bias, float *out,
            int accumulate, hipStream_t st)
{
    ProductArgs a{};
    a.t = t;
    a.q = q;
    a.as = s;
    a.corr = c;
    a.rows = 1;
    a.quad_begin = 0;
    a.quad_end = (t->rows + 3) / 4;
    a.bias = bias;
    a.out = out;
    a.ld_out = a.quad_end * 4;
    a.accumulate = accumulate;
    return launch_matvec(a, st);
}

int norm_quant(fg_qwen2 *m, const float *w, hipStream_t st)
{
    const int H = int(m->shape.hidden);
    const size_t smem = size_t(H + 8) * 4;
    if (m->shape.exact)
        rmsnorm_quant_kernel<true><<<1, kNormThreads, smem, st>>>(m->hidden, w, H, m->shape.eps, m->zp, m->xq, m->xs, m->xc, nullptr);
    else
        rmsnorm_quant_kernel<false><<<1, kNormThreads, smem, st>>>(m->hidden, w, H, m->shape.eps, m->zp, m->xq, m->xs, m->xc, nullptr);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

int run_layer(fg_qwen2 *m, size_t li, size_t position, hipStream_t st)
{
    const fg_qwen2_shape &sh = m->shape;
    const fg_qwen2_layer &ly = m->layers[li];
    const int H = int(sh.hidden), D = int(sh.head_dim);
    const int heads = int(sh.heads), kvh = int(sh.kv_heads), cap = int(sh.capacity);
    const size_t layer_base = li * sh.kv_heads * sh.capacity * sh.head_dim;
    int rc;
    if ((rc = norm_quant(m, ly.norm1, st))) return rc;
    if ((rc = product(ly.qkv, m->xq, m->xs, m->xc, ly.qkv_bias, m->qkv, 0, st))) return rc;
    const int rope_threads = (heads + 2 * kvh) * D / 2;
    const float *cos_t = m->rope + position * size_t(D);
    rope_keep_kernel<<<(rope_threads + 255) / 256, 256, 0, st>>>(m->qkv, cos_t, cos_t + D / 2, heads, kvh, D, m->kcache,
                                                                m->vcache, layer_base, cap, int(position));
    FG_HIP(hipGetLastError());
    const int keys = int(position) + 1;
    const size_t smem = size_t(6 * D + 8 + keys) * 4;
    if (sh.exact)
        attention_kernel<true><<<heads, 256, smem, st>>>(m->qkv, m->kcache, m->vcache, layer_base, heads, kvh, D, cap, keys,
                                                         m->zp, m->xq, m->xs, m->xc, nullptr);
    else
        attention_kernel<false><<<heads, 256, smem, st>>>(m->qkv, m->kcache, m->vcache, layer_base, heads, kvh, D, cap, keys,
                                                          m->zp, m->xq, m->xs, m->xc, nullptr);
    FG_HIP(hipGetLastError());
    if ((rc = product(ly.o, m->xq, m->xs, m->xc, nullptr, m->hidden, 1, st))) return rc;
    if ((rc = norm_quant(m, ly.norm2, st))) return rc;
    if ((rc = product(ly.gate, m->xq, m->xs, m->xc, nullptr, m->gate, 0, st))) return rc;
    if ((rc = product(ly.up, m->xq, m->xs, m->xc, nullptr, m->up, 0, st))) return rc;
    const int F = int(sh.ffn);
    silu_mul_quant_kernel<<<(F + 1023) / 1024, 256, 0, st>>>(m->gate, m->up, F, m->zp, m->xq, m->xs, m->xc);
    FG_HIP(hipGetLastError());
    if ((rc = product(ly.down, m->xq, m->xs, m->xc, nullptr, m->hidden, 1, st))) return rc;
    (void)H;
    return FG_OK;
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
    if (sh.head_dim % 64 != 0 && sh.head_dim != 32)
        return set_error(FG_ERR_SHAPE, "fg_qwen2_create: head_dim must be 32 or a multiple of 64");
    if (sh.hidden % 32 || sh.ffn % 32 || sh.hidden > 8192 || sh.capacity == 0 || sh.capacity > 8192)
        return set_error(FG_ERR_SHAPE, "fg_qwen2_create: hidden and ffn must be whole blocks (hidden, capacity <= 8192)");
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
    const size_t widest = std::max(sh.hidden, std::max(width, sh.ffn));
    const size_t padded_vocab = (sh.vocab + 3) / 4 * 4;
    struct Alloc {
        void **ptr;
        size_t bytes;
    } allocs[] = {
        {reinterpret_cast<void **>(&m->hidden), sh.hidden * 4},
        {reinterpret_cast<void **>(&m->qkv), (qkv_w + 3) / 4 * 4 * 4},
        {reinterpret_cast<void **>(&m->gate), (sh.ffn + 3) / 4 * 4 * 4},
        {reinterpret_cast<void **>(&m->up), (sh.ffn + 3) / 4 * 4 * 4},
        {reinterpret_cast<void **>(&m->logits), padded_vocab * 4},
        {reinterpret_cast<void **>(&m->rope), sh.capacity * sh.head_dim * 4},
        {reinterpret_cast<void **>(&m->xq), widest},
        {reinterpret_cast<void **>(&m->xs), widest / 32 * 4},
        {reinterpret_cast<void **>(&m->xc), widest / 32 * 4},
        {reinterpret_cast<void **>(&m->token), 4},
    };
    for (auto &a : allocs) {
        hipError_t e = hipMalloc(a.ptr, a.bytes);
        if (e != hipSuccess) {
            int rc = check_hip(e, "fg_qwen2_create: hipMalloc");
            fg_qwen2_free(m);
            return rc;
        }
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
    hipError_t e = hipMemcpy(m->rope, rope.data(), rope.size() * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        int rc = check_hip(e, "fg_qwen2_create: rotary table");
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
        if ((rc = norm_quant(m, m->final_norm, st))) return rc;
        // into the padded internal row: the product writes whole quads
        if ((rc = product(m->table, m->xq, m->xs, m->xc, nullptr, m->logits, 0, st))) return rc;
        if (logits) FG_HIP(hipMemcpyAsync(logits, m->logits, sh.vocab * 4, hipMemcpyDeviceToDevice, st));
        if (next_token) {
            argmax_kernel<<<1, 1024, 0, st>>>(m->logits, int(sh.vocab), next_token);
            FG_HIP(hipGetLastError());
        }
    }
    return FG_OK;
}

extern "C" int fg_qwen2_free(fg_qwen2 *m)
{
    if (!m) return FG_OK;
    void *ptrs[] = {m->hidden, m->qkv, m->gate, m->up, m->logits, m->rope, m->xq, m->xs, m->xc, m->token};
    for (void *p : ptrs)
        if (p) (void)hipFree(p);
    delete m;
    return FG_OK;
}
