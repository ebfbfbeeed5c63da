// Int8 attention over run-time quantized keys and values.
//
// Reference: attention::attend (blocks/src/attention.rs:81-214). Per (image, key head),
// Scratch::quantize (:100-137): the keys' mean over the keys in order, each key less the mean
// pushed as a Q7b32 row padded to whole blocks, and the values transposed, one Q7b32 row per
// channel over the keys (zeros past them). Per (image, head) and its queries, Scratch::unit
// (:157-214): scores = the product of the quantized queries with the keys over the keys rounded
// up to a quad, each times 1/sqrt(head_dim), zeros past them; Exponentials::apply (ops.rs:168-191)
// over the first `keys`; the scores' rows quantized over their whole padded width and multiplied
// with the values; each output divided by its row's sum. The reference runs its units 32 queries
// at a time; every query row is independent (its own quantization groups and sums), so a head's
// queries run as one product here, with the same bits.
//
// Both products are the path's own quantized product (launch_product): bit-exact int32 group
// accumulators and the reference's f32 group order. The f32 steps around them follow the
// reference's order: the mean is a sequential sum per channel, the exponentials' sum is the
// scalar backend's (eight offset sums over whole runs of eight, then the rest and those sums).
#include "common.h"
#include "proj.h"

#include <cmath>

namespace fg {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxRowBytes = 64 * 1024;  // one padded score row in LDS: at most 16384 keys

size_t pad32(size_t n) { return (n + 31) / 32 * 32; }

// exp_fast (ops.rs:137-153): clamped below at EXP_MIN, n = round(x · log2 e) ties to even,
// r = fma(−n, ln 2, x), the degree-4 Taylor polynomial in fused multiply-adds, times 2^n.
__device__ __forceinline__ float ref_exp_fast(float x)
{
    x = fmaxf(x, -87.0f);
    const float n = rintf(x * 1.44269504088896340736f);
    const float r = __builtin_fmaf(-n, 0.693147180559945309417f, x);
    float poly = 1.0f / 24.0f;
    poly = __builtin_fmaf(poly, r, 1.0f / 6.0f);
    poly = __builtin_fmaf(poly, r, 0.5f);
    poly = __builtin_fmaf(poly, r, 1.0f);
    poly = __builtin_fmaf(poly, r, 1.0f);
    return poly * __int_as_float((int(n) + 127) << 23);
}

// mean[(image · kv_heads + kh) · hd + d] = (Σ over the image's keys in order of key[d]) / keys,
// one thread per (image, key head, channel), every key head of the call in one launch; each
// thread issues 32 keys' loads before it adds them, in order
__global__ void key_mean_kernel(const float *__restrict__ key, size_t stride, size_t offset, int images, int kv_heads,
                                int keys, int hd, float *__restrict__ mean)
{
    const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= size_t(images) * kv_heads * hd) return;
    const int d = int(i % hd);
    const size_t ih = i / hd;
    const int kh = int(ih % kv_heads);
    const size_t image = ih / kv_heads;
    const float *base = key + image * size_t(keys) * stride + offset + size_t(kh) * hd + d;
    float s = 0.0f;
    for (int k0 = 0; k0 < keys; k0 += 32) {
        float v[32];
#pragma unroll
        for (int u = 0; u < 32; u++) v[u] = base[size_t(min(k0 + u, keys - 1)) * stride];
#pragma unroll
        for (int u = 0; u < 32; u++)
            if (k0 + u < keys) s = s + v[u];
    }
    mean[i] = s / float(keys);
}

// rows[k][d] = key[k][d] − mean[d] for d < hd, zeros to the padded width pd
__global__ void key_rows_kernel(const float *__restrict__ key, size_t stride, size_t base, int keys, int hd, int pd,
                                const float *__restrict__ mean, float *__restrict__ rows)
{
    const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= size_t(keys) * pd) return;
    const int k = int(i / pd), d = int(i % pd);
    rows[i] = d < hd ? key[base + size_t(k) * stride + d] - mean[d] : 0.0f;
}

// rows[d][k] = value[k][d] for k < keys, zeros to the padded width pk (Scratch::transpose)
__global__ void value_rows_kernel(const float *__restrict__ value, size_t stride, size_t base, int keys, int hd, int pk,
                                  float *__restrict__ rows)
{
    const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= size_t(hd) * pk) return;
    const int d = int(i / pk), k = int(i % pk);
    rows[i] = k < keys ? value[base + size_t(k) * stride + d] : 0.0f;
}

// rows[r][d] = query[r][d] for d < hd, zeros to pd
__global__ void query_rows_kernel(const float *__restrict__ query, size_t stride, size_t base, int queries, int hd,
                                  int pd, float *__restrict__ rows)
{
    const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= size_t(queries) * pd) return;
    const int r = int(i / pd), d = int(i % pd);
    rows[i] = d < hd ? query[base + size_t(r) * stride + d] : 0.0f;
}

// One workgroup of four waves per query row: the row's scores (product · scale below keys4,
// zeros to pk) staged in LDS, their maximum over the first `keys`, the exponentials there (all
// 256 threads), and their sum in the scalar backend's order (scalar.rs:117-126, ops.rs:170-175):
// lane o < 8 of the first wave sums offset o over the whole runs of eight in order, lane 0 adds
// the rest in order, then the eight offset sums in order.
template <bool FAST>
__global__ __launch_bounds__(256) void exponentials_kernel(const float *__restrict__ prod, int keys4, float scale,
                                                           int keys, int pk, float *__restrict__ scores,
                                                           float *__restrict__ sums)
{
    extern __shared__ float row[];  // [pk], then the four waves' maxima
    float *wmax = row + pk;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t r = blockIdx.x;
    float m = -INFINITY;
    for (int i = tid; i < pk; i += 256) {
        const float v = i < keys4 ? prod[r * keys4 + i] * scale : 0.0f;
        row[i] = v;
        if (i < keys) m = fmaxf(m, v);
    }
    for (int s = 32; s >= 1; s >>= 1) m = fmaxf(m, __shfl_xor(m, s, 64));
    if (lane == 0) wmax[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    for (int i = tid; i < keys; i += 256) row[i] = FAST ? ref_exp_fast(row[i] - m) : ref_exp(row[i] - m);
    __syncthreads();
    if (wave == 0) {
        const int whole = keys / 8 * 8;
        float part = 0.0f;
        if (lane < 8) {
            // sixteen reads out before their sixteen additions, in run order
            int i = lane;
            for (; i + 8 * 15 < whole; i += 8 * 16) {
                float v[16];
#pragma unroll
                for (int u = 0; u < 16; u++) v[u] = row[i + 8 * u];
#pragma unroll
                for (int u = 0; u < 16; u++) part = part + v[u];
            }
            for (; i < whole; i += 8) part = part + row[i];
        }
        float total = -0.0f;
        if (lane == 0) {
            for (int i = whole; i < keys; i++) total = total + row[i];
        }
#pragma unroll
        for (int o = 0; o < 8; o++) {
            const float po = __shfl(part, o, 64);
            if (lane == 0) total = total + po;
        }
        if (lane == 0) sums[r] = total;
    }
    for (int i = tid; i < pk; i += 256) scores[r * pk + i] = row[i];
}

// out[(first + r) · stride + d] = prod[r][d] / sums[r]
__global__ void divide_kernel(const float *__restrict__ prod, const float *__restrict__ sums, int queries, int hd,
                              float *__restrict__ out, size_t stride, size_t base)
{
    const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= size_t(queries) * hd) return;
    const int r = int(i / hd), d = int(i % hd);
    out[base + size_t(r) * stride + d] = prod[i] / sums[r];
}

unsigned blocks_for(size_t n) { return unsigned((n + kThreads - 1) / kThreads); }

// A query row per workgroup; a row of 16384 keys takes 64 KiB and 16 bytes of LDS, past the
// default limit, which is then raised for the kernel on the current device.
template <bool FAST>
int launch_exponentials(const float *prod, int keys4, float scale, int keys, int pk, float *scores, float *sums,
                        unsigned queries, hipStream_t st)
{
    const size_t smem = size_t(pk) * 4 + 16;
    if (smem > 64 * 1024)
        FG_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(exponentials_kernel<FAST>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
    exponentials_kernel<FAST><<<queries, 256, smem, st>>>(prod, keys4, scale, keys, pk, scores, sums);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

struct Scratch {
    float *mean = nullptr, *krows = nullptr, *vrows = nullptr, *qrows = nullptr, *prod = nullptr, *scores = nullptr,
          *sums = nullptr;
    fg_table *keys = nullptr, *values = nullptr;
};

int run(const fg_attention *c, float *out, hipStream_t st, Scratch &w)
{
    const int hd = int(c->head_dim), keys = int(c->keys), queries = int(c->queries);
    const int pd = int(pad32(c->head_dim)), pk = int(pad32(c->keys)), keys4 = (keys + 3) / 4 * 4;
    const size_t group = c->heads / c->kv_heads, stride = c->heads * c->head_dim;
    const float scale = 1.0f / sqrtf(float(hd));
    const size_t bytes[] = {c->images * c->kv_heads * size_t(hd) * 4, size_t(keys) * pd * 4,
                            size_t(hd) * pk * 4, size_t(queries) * pd * 4,
                            size_t(queries) * size_t(keys4 > hd ? keys4 : hd) * 4,
                            size_t(queries) * pk * 4, size_t(queries) * 4};
    float **ptrs[] = {&w.mean, &w.krows, &w.vrows, &w.qrows, &w.prod, &w.scores, &w.sums};
    for (int i = 0; i < 7; i++) FG_HIP(hipMallocAsync(reinterpret_cast<void **>(ptrs[i]), bytes[i], st));
    int rc;
    if ((rc = fg_qmatrix_create(size_t(keys), size_t(pd), &w.keys)) || (rc = fg_qmatrix_create(size_t(hd), size_t(pk), &w.values)))
        return rc;
    key_mean_kernel<<<blocks_for(c->images * c->kv_heads * size_t(hd)), kThreads, 0, st>>>(
        c->key, c->key_stride, c->key_offset, int(c->images), int(c->kv_heads), keys, hd, w.mean);
    FG_HIP(hipGetLastError());
    for (size_t image = 0; image < c->images; image++) {
        for (size_t kh = 0; kh < c->kv_heads; kh++) {
            // Scratch::quantize (attention.rs:100-137)
            const size_t kbase = image * c->keys * c->key_stride + c->key_offset + kh * c->head_dim;
            const size_t vbase = image * c->keys * c->value_stride + c->value_offset + kh * c->head_dim;
            key_rows_kernel<<<blocks_for(size_t(keys) * pd), kThreads, 0, st>>>(
                c->key, c->key_stride, kbase, keys, hd, pd, w.mean + (image * c->kv_heads + kh) * size_t(hd), w.krows);
            value_rows_kernel<<<blocks_for(size_t(hd) * pk), kThreads, 0, st>>>(c->value, c->value_stride, vbase, keys, hd,
                                                                                pk, w.vrows);
            FG_HIP(hipGetLastError());
            if ((rc = fg_qmatrix_reset(w.keys, size_t(pd))) || (rc = fg_qmatrix_extend(w.keys, size_t(keys), st)) ||
                (rc = fg_qmatrix_set_rows(w.keys, 0, size_t(keys), w.krows, st)) ||
                (rc = fg_qmatrix_reset(w.values, size_t(pk))) || (rc = fg_qmatrix_extend(w.values, size_t(hd), st)) ||
                (rc = fg_qmatrix_set_rows(w.values, 0, size_t(hd), w.vrows, st)))
                return rc;
            for (size_t h = kh * group; h < (kh + 1) * group; h++) {
                // Scratch::unit (attention.rs:157-214) for every query of the image at once
                const size_t qbase = image * c->queries * c->query_stride + c->query_offset + h * c->head_dim;
                query_rows_kernel<<<blocks_for(size_t(queries) * pd), kThreads, 0, st>>>(c->query, c->query_stride, qbase,
                                                                                         queries, hd, pd, w.qrows);
                FG_HIP(hipGetLastError());
                ProductArgs a{};
                a.t = w.keys;
                a.x = w.qrows;
                a.rows = size_t(queries);
                a.quad_begin = 0;
                a.quad_end = size_t(keys4 / 4);
                a.out = w.prod;
                a.ld_out = size_t(keys4);
                if ((rc = launch_product(a, st))) return rc;
                rc = c->exponentials == FG_EXP_FAST
                         ? launch_exponentials<true>(w.prod, keys4, scale, keys, pk, w.scores, w.sums, unsigned(queries), st)
                         : launch_exponentials<false>(w.prod, keys4, scale, keys, pk, w.scores, w.sums, unsigned(queries), st);
                if (rc) return rc;
                ProductArgs b{};
                b.t = w.values;
                b.x = w.scores;
                b.rows = size_t(queries);
                b.quad_begin = 0;
                b.quad_end = size_t(hd / 4);
                b.out = w.prod;
                b.ld_out = size_t(hd);
                if ((rc = launch_product(b, st))) return rc;
                divide_kernel<<<blocks_for(size_t(queries) * hd), kThreads, 0, st>>>(
                    w.prod, w.sums, queries, hd, out, stride, image * c->queries * stride + h * c->head_dim);
                FG_HIP(hipGetLastError());
            }
        }
    }
    return FG_OK;
}

}  // namespace
}  // namespace fg

using namespace fg;

extern "C" int fg_attend(const fg_attention *c, float *out, void *stream)
{
    if (!c || !out || !c->query || !c->key || !c->value) return set_error(FG_ERR_ARG, "fg_attend: null argument");
    if (!c->heads || !c->kv_heads || !c->head_dim || !c->images || !c->queries || !c->keys || c->heads % c->kv_heads)
        return set_error(FG_ERR_SHAPE, "fg_attend: heads, key heads, head_dim, images, queries and keys must be positive, "
                                       "the heads a multiple of the key heads");
    if (c->head_dim % 4) return set_error(FG_ERR_SHAPE, "fg_attend: head_dim must be whole quads");
    if (c->exponentials != FG_EXP_EXACT && c->exponentials != FG_EXP_FAST)
        return set_error(FG_ERR_ARG, "fg_attend: exponentials must be FG_EXP_EXACT or FG_EXP_FAST");
    if (pad32(c->keys) * 4 > size_t(kMaxRowBytes)) return set_error(FG_ERR_SHAPE, "fg_attend: at most 16384 keys");
    // every head of a row lies within the row's stride
    if (c->query_offset + c->heads * c->head_dim > c->query_stride ||
        c->key_offset + c->kv_heads * c->head_dim > c->key_stride ||
        c->value_offset + c->kv_heads * c->head_dim > c->value_stride)
        return set_error(FG_ERR_SHAPE, "fg_attend: an operand's heads run past its row stride");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    Scratch w;
    int rc = run(c, out, st, w);
    // the scratch is ordered on the stream; the run-time matrices are freed once it has finished
    float *ptrs[] = {w.mean, w.krows, w.vrows, w.qrows, w.prod, w.scores, w.sums};
    for (float *p : ptrs)
        if (p) (void)hipFreeAsync(p, st);
    const hipError_t e = hipStreamSynchronize(st);
    if (rc == FG_OK && e != hipSuccess) rc = check_hip(e, "hipStreamSynchronize");
    if (w.keys) (void)fg_table_free(w.keys);
    if (w.values) (void)fg_table_free(w.values);
    return rc;
}
