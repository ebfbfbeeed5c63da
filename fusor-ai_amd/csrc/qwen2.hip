// The Qwen2 decoder step on the device: Transformer::forward with one row and
// Prediction::predict (blocks/src/transformer.rs:185-341, layer.rs:161-344,
// layer/input.rs:22-66, lm.rs:97-179), every projection through the projection kernel.
//
// Per layer, each projection with its neighbours fused in, four launches:
//   1. RMSNorm + quantize -> QKV product + bias -> RoPE: every query head's rows recomputed by
//      each of its chunk workgroups, which then take their chunk of the cached keys; the key and
//      value rows of the position projected, rotated and kept by the remaining workgroups
//   2. output projection added to the residual row, its input the attention row
//   3. RMSNorm + quantize -> gate and up products -> silu(gate)·up, each workgroup's 32 outputs
//      quantized as one group for down
//   4. down projection added to the residual row
// In parallel order the chunk workgroups attend over their keys (flash decoding) and the output
// projection's prologue merges the chunks with the new key's own state. In the reference's order
// (exact) they write their keys' scores, and one more launch between 1 and 2 takes the attention
// of every query head by head and 32 value dimensions: the new key's score, the softmax and the
// weighted values in key order, quantized for the output projection (head sizes 64 and 128; other
// sizes project QKV by rotary pairs and take the scores by key blocks in a launch of their own).
// Then RMSNorm + quantize (one workgroup) -> head product (logits) with per-workgroup greedy
// candidates, and the greedy token. Elementwise arithmetic is the reference's operation for
// operation (no fused multiply-add; ops::exp's polynomial). Reductions whose order changes f32
// bits (RMSNorm's sum of squares, the softmax total, the attention's weighted sum) run in the
// reference's index order when the model is exact, or as parallel trees otherwise.
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
constexpr int kScoreKeys = 32;   // keys per workgroup of the scores
constexpr int kWeighKeys = 256;  // keys per staged chunk of values
constexpr int kWeighDims = 32;   // value dimensions per workgroup (one quantization group)
constexpr int kHeadQuads = 16;  // quads per workgroup of the logits product

struct AttnParams {
    const float *qkv;  // query heads first (rotated, except for attn_rows_kernel, which rotates them)
    const float *kcache, *vcache;
    size_t layer_base;
    int heads, kv_heads, D, capacity, keys;
    float *scores;  // [heads][capacity]
    int zp;
    int8_t *q;
    float *scales;
    int32_t *corr;
    float *row_out;  // when set, the f32 attention row before its quantization (an inspection)
    // rows of a prefill (grid z): row z's query heads at qkv + z·qkv_stride, its scores [heads][capacity]
    // after z such blocks, its outputs (levels, scales, corrections, row_out) z·row_width values on, and
    // keys + z keys (its own position's included)
    size_t qkv_stride, row_width;
    // a prefill's attention that also rotates its chunk's rows and keeps their keys and values
    // (attn_rows_kernel): the angles [capacity][D], and the caches written
    const float *rope;
    float *kkeep, *vkeep;
};

// Row blockIdx.z of a prefill's attention: its own query, scores, outputs and key count.
__device__ __forceinline__ void attn_row(AttnParams &a)
{
    const size_t z = blockIdx.z;
    if (z == 0) return;
    a.qkv += z * a.qkv_stride;
    a.scores += z * size_t(a.heads) * a.capacity;
    a.keys += int(z);
    a.q += z * a.row_width;
    a.scales += z * a.row_width / 32;
    a.corr += z * a.row_width / 32;
    if (a.row_out) a.row_out += z * a.row_width;
}

// Scores of every query head of one KV head against kScoreKeys keys (ops.rs:310-326):
// dot_f32(q, k_j) in index order, times 1/√D. Grid: (kv_heads, key blocks).
__global__ __launch_bounds__(kAttnThreads) void attn_scores_kernel(AttnParams a)
{
    extern __shared__ __align__(16) float ash[];
    attn_row(a);
    const int D = a.D, S = D + 1;
    const int group = a.heads / a.kv_heads;
    const int kv = blockIdx.x, j0 = int(blockIdx.y) * kScoreKeys;
    if (j0 >= a.keys) return;  // a prefill's earlier rows see fewer keys (uniform per workgroup)
    const int n = min(kScoreKeys, a.keys - j0);
    float *krows = ash;                      // [kScoreKeys][D + 1]
    float *query = krows + kScoreKeys * S;   // [group][D]
    const float *kbase = a.kcache + a.layer_base + size_t(kv) * a.capacity * D;
    // all loads first (branch-free: past-the-end rows re-read row j0)
    const int per_row = D / 4;
    const int nk4 = kScoreKeys * per_row, nq = group * D;
    float4 kr[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int e = int(threadIdx.x) + r * kAttnThreads;
        const int row = e / per_row, c4 = e - row * per_row;
        const int rr = (e < nk4 && row < n) ? row : 0;
        kr[r] = *reinterpret_cast<const float4 *>(kbase + size_t((j0 + rr) % a.capacity) * D + c4 * 4);
    }
    float qv[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int e = int(threadIdx.x) + r * kAttnThreads;
        qv[r] = a.qkv[size_t(kv * group) * D + min(e, nq - 1)];
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int e = int(threadIdx.x) + r * kAttnThreads;
        const int row = e / per_row, c4 = e - row * per_row;
        if (e < nk4) {
            float *dst = krows + row * S + c4 * 4;
            dst[0] = kr[r].x;
            dst[1] = kr[r].y;
            dst[2] = kr[r].z;
            dst[3] = kr[r].w;
        }
        if (e < nq) query[e] = qv[r];
    }
    __syncthreads();
    const float scale = 1.0f / sqrtf(float(D));
    for (int t = threadIdx.x; t < group * kScoreKeys; t += kAttnThreads) {
        const int h = t / kScoreKeys, j = t - h * kScoreKeys;
        if (j >= n) continue;
        const float *k = krows + j * S;
        const float *q = query + h * D;
        float s = -0.0f;  // dot_f32 in index order (arch/scalar.rs:340-342)
        for (int d = 0; d < D; d += 16) {
            float x[16], y[16];
#pragma unroll
            for (int e = 0; e < 16; e++) {
                x[e] = q[d + e];
                y[e] = k[d + e];
            }
#pragma unroll
            for (int e = 0; e < 16; e++) s = s + x[e] * y[e];
        }
        a.scores[size_t(kv * group + h) * a.capacity + j0 + j] = s * scale;
    }
}

__device__ float attn_block_max(float v, float *red)
{
    v = wave_allmax(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__device__ float attn_block_sum(float v, float *red)
{
    v = wave_allsum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[4 + (threadIdx.x >> 6)] = v;
    __syncthreads();
    return ((red[4] + red[5]) + red[6]) + red[7];
}

// kWeighKeys keys x kWeighDims dims of one KV head's values into registers (8 float4 per thread);
// rows past the n keys are not read (a prefill's early rows see few keys).
__device__ __forceinline__ void fetch_values(const float *vbase, int capacity, int D, int d0, int j0, int n, float4 *r)
{
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int e = int(threadIdx.x) + k * kAttnThreads;  // float4 index: row e / 8, column (e % 8) * 4
        const int row = e >> 3, c4 = e & 7;
        r[k] = row < n ? *reinterpret_cast<const float4 *>(vbase + size_t((j0 + row) % capacity) * D + d0 + c4 * 4)
                       : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
}

// Softmax of one head's scores (ops.rs:301-306: maximum, ops::exp, the total, the division) and
// the weighted sum of kWeighDims value dimensions (ops.rs:329-342), then those outputs quantized
// (one group) for the output projection. Grid: (heads, D / kWeighDims).
template <bool EXACT>
__global__ __launch_bounds__(kAttnThreads) void attn_weigh_kernel(AttnParams a)
{
    extern __shared__ __align__(16) float ash[];
    attn_row(a);
    constexpr int S = kWeighDims + 1;
    const int D = a.D, keys = a.keys;
    const int head = blockIdx.x, d0 = int(blockIdx.y) * kWeighDims;
    const int kv = head / (a.heads / a.kv_heads);
    float *vrows = ash;                    // [kWeighKeys][kWeighDims + 1]
    float *w = vrows + kWeighKeys * S;     // [keys]
    float *parts = w + a.capacity;         // [8][kWeighDims]
    float *red = parts + 8 * kWeighDims;   // [16]
    const float *vbase = a.vcache + a.layer_base + size_t(kv) * a.capacity * D;
    const float *sc = a.scores + size_t(head) * a.capacity;
    float4 vr[8];
    fetch_values(vbase, a.capacity, D, d0, 0, min(kWeighKeys, keys), vr);
    float local_max = -INFINITY;
    for (int j = threadIdx.x; j < keys; j += kAttnThreads) {
        const float s = sc[j];
        w[j] = s;
        local_max = fmaxf(local_max, s);
    }
    const float peak = attn_block_max(local_max, red);
    for (int j = threadIdx.x; j < keys; j += kAttnThreads) w[j] = ref_exp(w[j] - peak);
    __syncthreads();
    float total;
    if (EXACT) {
        if (threadIdx.x == 0) {
            float t = -0.0f;  // the exponentials summed in index order
            int j = 0;
            for (; j + 16 <= keys; j += 16) {
                float v[16];
#pragma unroll
                for (int e = 0; e < 16; e++) v[e] = w[j + e];
#pragma unroll
                for (int e = 0; e < 16; e++) t = t + v[e];
            }
            for (; j < keys; j++) t = t + w[j];
            red[8] = t;
        }
        __syncthreads();
        total = red[8];
    } else {
        float p = 0.0f;
        for (int j = threadIdx.x; j < keys; j += kAttnThreads) p = p + w[j];
        total = attn_block_sum(p, red);
    }
    for (int j = threadIdx.x; j < keys; j += kAttnThreads) w[j] = w[j] / total;
    // weigh: out[i] = Σ_j w_j·v_j[i] from +0; exact: index order per output
    const int slices = EXACT ? 1 : 8;
    const int slice = int(threadIdx.x) / kWeighDims, i = int(threadIdx.x) - slice * kWeighDims;
    float o = 0.0f;
    for (int j0 = 0; j0 < keys; j0 += kWeighKeys) {
        const int n = min(kWeighKeys, keys - j0);
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int e = int(threadIdx.x) + k * kAttnThreads;
            const int row = e >> 3, c4 = e & 7;
            if (row < n) {
                float *dst = vrows + row * S + c4 * 4;
                dst[0] = vr[k].x;
                dst[1] = vr[k].y;
                dst[2] = vr[k].z;
                dst[3] = vr[k].w;
            }
        }
        __syncthreads();
        if (j0 + kWeighKeys < keys) fetch_values(vbase, a.capacity, D, d0, j0 + kWeighKeys, min(kWeighKeys, keys - j0 - kWeighKeys), vr);
        if (slice < slices) {
            int j = slice;
            for (; j + 16 * slices <= n; j += 16 * slices) {
                float ww[16], vv[16];
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    ww[e] = w[j0 + j + e * slices];
                    vv[e] = vrows[(j + e * slices) * S + i];
                }
#pragma unroll
                for (int e = 0; e < 16; e++) o = o + ww[e] * vv[e];
            }
            for (; j < n; j += slices) o = o + w[j0 + j] * vrows[j * S + i];
        }
    }
    if (slice < slices) parts[slice * kWeighDims + i] = o;
    __syncthreads();
    // the slices added in order, then the group of kWeighDims outputs quantized (8 lanes)
    const int sub = threadIdx.x & 7;
    if (threadIdx.x < 8) {
        float x[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float v = parts[sub * 4 + e];
            for (int s2 = 1; s2 < slices; s2++) v = v + parts[s2 * kWeighDims + sub * 4 + e];
            x[e] = v;
        }
        if (a.row_out) {
#pragma unroll
            for (int e = 0; e < 4; e++) a.row_out[head * D + d0 + sub * 4 + e] = x[e];
        }
        float amax = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
        amax = max8(fmaxf(0.0f, amax));
        int l0, l1, l2, l3;
        const float d = scale_and_levels(amax, x[0], x[1], x[2], x[3], l0, l1, l2, l3);
        const int sum = sum8(l0 + l1 + l2 + l3);
        const int G = (head * D + d0) / 32;
        reinterpret_cast<int *>(a.q)[G * 8 + sub] = pack4(l0, l1, l2, l3);
        if (sub == 0) {
            a.scales[G] = d;
            a.corr[G] = -a.zp * sum;
        }
    }
}

// s + Σ t[j] for j in 0..n, added in index order by one lane; t 16-byte aligned. Runs of 32 (eight
// 128-bit reads) into two register sets in turn, run c + 1's reads (clamped, never past the last
// run) issued before run c is added: 32 dependent additions outlast an LDS read, so the chain
// neither waits for LDS nor shares its issue slots with more than a read per four terms.
__device__ __forceinline__ float chain_sum(float s, int n, const float *t)
{
    constexpr int V = 8;  // 128-bit reads per run
    const v4f *t4 = reinterpret_cast<const v4f *>(t);
    const int runs = n / (4 * V);
    v4f A[V], B[V];
    auto load = [&](v4f *r, int c) {
#pragma unroll
        for (int e = 0; e < V; e++) r[e] = t4[c * V + e];
    };
    auto add = [&](const v4f *r) {
#pragma unroll
        for (int e = 0; e < V; e++) {
            s = s + r[e].x;
            s = s + r[e].y;
            s = s + r[e].z;
            s = s + r[e].w;
        }
    };
    if (runs > 0) {
        load(A, 0);
        for (int c = 0; c < runs; c += 2) {
            load(B, min(c + 1, runs - 1));
            __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of the additions
            add(A);
            load(A, min(c + 2, runs - 1));
            __builtin_amdgcn_sched_barrier(0);
            if (c + 1 < runs) add(B);
        }
    }
    for (int j = runs * 4 * V; j < n; j++) s = s + t[j];
    return s;
}

// A prefill's attention, per (head, block of R = 256 / D rows), straight from the chunk's QKV rows
// (bias added, not yet rotated): each row's query heads rotated by halves at its own position
// (ops.rs:77-85), its scores against the keys up to that position (ops.rs:310-326: dot_f32 in
// index order from -0, times 1/sqrt(D); one thread per row and key), its softmax (ops.rs:301-306:
// maximum, ops::exp, the total, the division; a wave per row, the total in key order by one lane
// when exact, else a wave tree), its weighted values in key order from +0 (ops.rs:329-342, one
// thread per row and value dimension), then its outputs quantized per group of 32 for the output
// projection. The block's rows share one KV head's keys and values, staged once per pass of
// 4096 / D keys for all of them: the cached rows before the chunk as kept, the chunk's own rows
// from its QKV rows, keys rotated as they are staged. The workgroup of each KV head's first query
// head keeps its rows' rotated keys and values in the caches (KvCache::keep, transformer.rs:166-180);
// no workgroup of the launch reads the caches at the chunk's positions.
// LDS: the rows' scores, then weights [R][kstride]; a pass of keys [4096 / D][D + 1] or values
// [4096 / D][D] (then the outputs [R][D]); the query rows [R][D]; the totals [R].
template <bool EXACT>
__global__ __launch_bounds__(kAttnThreads) void attn_rows_kernel(AttnParams a, int n, int kstride)
{
    extern __shared__ __align__(16) float ash[];
    const int D = a.D, R = kAttnThreads / D, KC = 4096 / D, S = D + 1;
    const int head = blockIdx.x, z0 = int(blockIdx.y) * R;
    const int kv = head / (a.heads / a.kv_heads);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float *w = ash;
    float *stage = w + R * kstride;
    float *qrows = stage + KC * S;
    float *tot = qrows + R * D;
    const float *kbase = a.kcache + a.layer_base + size_t(kv) * a.capacity * D;
    const float *vbase = a.vcache + a.layer_base + size_t(kv) * a.capacity * D;
    const int rows = min(R, n - z0);
    const int kblock = a.keys + z0 + rows - 1;  // keys of the block's last row, the most
    // Passes 0 .. P - 1 stage keys, P .. 2P - 1 values, KC rows each: every thread's share of pass
    // p + 1 is loaded into registers while pass p is worked on. A key pass takes matching float4s
    // of a row's two halves (at most two pairs a thread) with their angles; a value pass at most four
    // float4s.
    const int P = (kblock + KC - 1) / KC, D4 = D / 4, D8 = D / 8, half = D / 2;
    const int first = a.keys - 1;
    const bool keeper = head % (a.heads / a.kv_heads) == 0;  // keeps this block's rows in the caches
    const int keep_lo = first + z0, keep_hi = first + z0 + rows;
    float *kkeep = a.kkeep + a.layer_base + size_t(kv) * a.capacity * D;
    float *vkeep = a.vkeep + a.layer_base + size_t(kv) * a.capacity * D;
    auto key_row = [&](int pos) {
        return pos < first ? kbase + size_t(pos % a.capacity) * D : a.qkv + size_t(pos - first) * a.qkv_stride + size_t(a.heads + kv) * D;
    };
    auto value_row = [&](int pos) {
        return pos < first ? vbase + size_t(pos % a.capacity) * D
                           : a.qkv + size_t(pos - first) * a.qkv_stride + size_t(a.heads + a.kv_heads + kv) * D;
    };
    float4 ahead[4], cosv[2], sinv[2];
    auto load_pass = [&](int p) {
        if (p < P) {
            const int c0 = p * KC, nk = min(KC, kblock - c0);
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const int e = tid + k * kAttnThreads, row = e / D8, c = (e - row * D8) * 4;
                if (row >= nk) continue;
                const int pos = c0 + row;
                const float *src = key_row(pos);
                ahead[2 * k] = *reinterpret_cast<const float4 *>(src + c);
                ahead[2 * k + 1] = *reinterpret_cast<const float4 *>(src + half + c);
                if (pos >= first) {
                    cosv[k] = *reinterpret_cast<const float4 *>(a.rope + size_t(pos) * D + c);
                    sinv[k] = *reinterpret_cast<const float4 *>(a.rope + size_t(pos) * D + half + c);
                }
            }
        } else {
            const int c0 = (p - P) * KC, nk = min(KC, kblock - c0);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int e = tid + k * kAttnThreads, row = e / D4;
                if (row < nk) ahead[k] = *reinterpret_cast<const float4 *>(value_row(c0 + row) + (e - row * D4) * 4);
            }
        }
    };
    auto store_pass = [&](int p) {
        if (p < P) {  // keys: rows D + 1 floats apart
            const int c0 = p * KC, nk = min(KC, kblock - c0);
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const int e = tid + k * kAttnThreads, row = e / D8, c = (e - row * D8) * 4;
                if (row >= nk) continue;
                const int pos = c0 + row;
                float4 x = ahead[2 * k], y = ahead[2 * k + 1];
                if (pos >= first) {  // the rotation by halves of rope_keep_rows_kernel
                    const float4 cs = cosv[k], sn = sinv[k];
                    const float4 nx = make_float4(x.x * cs.x - y.x * sn.x, x.y * cs.y - y.y * sn.y, x.z * cs.z - y.z * sn.z,
                                                  x.w * cs.w - y.w * sn.w);
                    const float4 ny = make_float4(y.x * cs.x + x.x * sn.x, y.y * cs.y + x.y * sn.y, y.z * cs.z + x.z * sn.z,
                                                  y.w * cs.w + x.w * sn.w);
                    x = nx;
                    y = ny;
                    if (keeper && pos >= keep_lo && pos < keep_hi) {
                        float *dst = kkeep + size_t(pos % a.capacity) * D;
                        *reinterpret_cast<float4 *>(dst + c) = x;
                        *reinterpret_cast<float4 *>(dst + half + c) = y;
                    }
                }
                float *dst = stage + row * S + c;
                dst[0] = x.x;
                dst[1] = x.y;
                dst[2] = x.z;
                dst[3] = x.w;
                dst[half] = y.x;
                dst[half + 1] = y.y;
                dst[half + 2] = y.z;
                dst[half + 3] = y.w;
            }
        } else {
            const int c0 = (p - P) * KC, nk = min(KC, kblock - c0);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int e = tid + k * kAttnThreads, row = e / D4;
                if (row >= nk) continue;
                reinterpret_cast<float4 *>(stage)[e] = ahead[k];
                const int pos = c0 + row;
                if (keeper && pos >= keep_lo && pos < keep_hi)
                    *reinterpret_cast<float4 *>(vkeep + size_t(pos % a.capacity) * D + (e - row * D4) * 4) = ahead[k];
            }
        }
    };
    load_pass(0);
    // the block's query rows, rotated at their own positions
    for (int e = tid; e < rows * D; e += kAttnThreads) {
        const int r = e / D, d = e - r * D, j = d < half ? d : d - half;
        const float *src = a.qkv + size_t(z0 + r) * a.qkv_stride + size_t(head) * D;
        const float *cs = a.rope + size_t(first + z0 + r) * D;
        const float c = cs[j], sn = cs[half + j], x = src[j], y = src[half + j];
        qrows[e] = d < half ? x * c - y * sn : y * c + x * sn;
    }
    // scores (pairs key-fastest: neighbouring lanes read neighbouring key rows, D + 1 floats
    // apart, and one query row)
    const float scale = 1.0f / sqrtf(float(D));
    for (int p = 0; p < P; p++) {
        const int c0 = p * KC, nk = min(KC, kblock - c0);
        __syncthreads();  // the previous pass's keys are read (the first: the queries are written)
        store_pass(p);
        __syncthreads();
        load_pass(p + 1);
        for (int pr = tid; pr < rows * nk; pr += kAttnThreads) {
            const int r = pr / nk, j = pr - r * nk;
            if (c0 + j >= a.keys + z0 + r) continue;  // past the row's own position
            const float *q = qrows + r * D, *k = stage + j * S;
            float sum = -0.0f;
            for (int d = 0; d < D; d += 16) {
                float x[16], y[16];
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    x[e] = q[d + e];
                    y[e] = k[d + e];
                }
#pragma unroll
                for (int e = 0; e < 16; e++) sum = sum + x[e] * y[e];
            }
            w[r * kstride + c0 + j] = sum * scale;
        }
    }
    __syncthreads();
    for (int r = wave; r < rows; r += kAttnThreads / 64) {
        const int keys = a.keys + z0 + r;
        float *wr = w + r * kstride;
        float m = -INFINITY;
        for (int j = lane; j < keys; j += 64) m = fmaxf(m, wr[j]);
        const float peak = wave_allmax(m);
        float part = 0.0f;
        for (int j = lane; j < keys; j += 64) {
            const float e = ref_exp(wr[j] - peak);
            wr[j] = e;
            part = part + e;
        }
        if (!EXACT) {
            const float t = wave_allsum(part);
            if (lane == 0) tot[r] = t;
        }
    }
    __syncthreads();
    if (EXACT && tid < rows) tot[tid] = chain_sum(-0.0f, a.keys + z0 + tid, w + tid * kstride);
    __syncthreads();
    for (int e = tid; e < rows * kstride; e += kAttnThreads) {
        const int r = e / kstride, j = e - r * kstride;
        if (j < a.keys + z0 + r) w[e] = w[e] / tot[r];
    }
    const int r = tid / D, i = tid - r * D;  // this thread's row and value dimension
    const bool live = r < rows;
    const int keys = a.keys + z0 + r;
    float o = 0.0f;
    for (int p = P; p < 2 * P; p++) {
        const int c0 = (p - P) * KC, nk = min(KC, kblock - c0);
        __syncthreads();  // the weights are final; the previous pass's values are read
        store_pass(p);
        __syncthreads();
        if (p + 1 < 2 * P) load_pass(p + 1);
        if (live) {
            // sixteen weights and values read ahead of their sixteen ordered additions
            const int end = min(nk, keys - c0);
            const float *wr = w + r * kstride + c0;
            int j = 0;
            for (; j + 16 <= end; j += 16) {
                float ww[16], vv[16];
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    ww[e] = wr[j + e];
                    vv[e] = stage[(j + e) * D + i];
                }
#pragma unroll
                for (int e = 0; e < 16; e++) o = o + ww[e] * vv[e];
            }
            for (; j < end; j++) o = o + wr[j] * stage[j * D + i];
        }
    }
    __syncthreads();
    if (live) stage[r * D + i] = o;
    __syncthreads();
    // the block's rows x D / 32 groups (at most 8), eight lanes each
    if (tid < 8 * (rows * D / 32)) {
        const int g = tid >> 3, sub = tid & 7;
        const int r2 = g * 32 / D, c = g * 32 - r2 * D;
        float x[4];
#pragma unroll
        for (int e = 0; e < 4; e++) x[e] = stage[r2 * D + c + sub * 4 + e];
        const size_t at = size_t(z0 + r2) * a.row_width + size_t(head) * D + c;
        if (a.row_out) {
#pragma unroll
            for (int e = 0; e < 4; e++) a.row_out[at + sub * 4 + e] = x[e];
        }
        float amax = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
        amax = max8(fmaxf(0.0f, amax));
        int l0, l1, l2, l3;
        const float d = scale_and_levels(amax, x[0], x[1], x[2], x[3], l0, l1, l2, l3);
        const int sum = sum8(l0 + l1 + l2 + l3);
        const size_t G = at / 32;
        reinterpret_cast<int *>(a.q)[G * 8 + sub] = pack4(l0, l1, l2, l3);
        if (sub == 0) {
            a.scales[G] = d;
            a.corr[G] = -a.zp * sum;
        }
    }
}

// LDS of attn_rows_kernel for a prefill whose last row sees kmax keys (0 when it does not fit 64 KiB
// or the head is wider than a workgroup).
inline size_t attn_rows_smem(int D, int kmax)
{
    const int R = kAttnThreads / D;
    if (R < 1) return 0;
    const size_t bytes = (size_t(R) * ((kmax + 3) / 4 * 4) + size_t(4096 / D) * (D + 1) + size_t(R) * D + 16) * 4;
    return bytes <= 64 * 1024 ? bytes : 0;
}

// The exact-order attention of one query head for kWeighDims value dimensions (the reference's
// arithmetic of attn_weigh_kernel<true>, ops.rs:301-342), over the scores of the cached keys that
// the query launch formed (score_chunk). Grid: (heads, D / kWeighDims), 256 threads.
//   scores: the cached keys' read back; the position's own key (the last) scored here: dot_f32 of
//           the rotated query and the new key in index order from −0, times 1/√D;
//   softmax: the maximum, w_j = ops::exp(s_j − max), their total from −0 in index order (one lane,
//           reads running ahead of the additions: chain_sum), w_j / total;
//   values: per chunk of 192 keys, lane l of waves 1..3 holds piece l % 8 (four dimensions) of
//           rows l / 8 + 8·e of its 64 (neighbouring lanes read neighbouring 16 bytes of a row)
//           and forms their products w_j·v_j[i] into LDS (a padded row per dimension, two
//           buffers); lanes 0..31 of the first wave add their row to their output i in key order
//           from +0 while the other waves form the next chunk's products, so the first wave's
//           additions run back to back. The value rows of the first two chunks are requested
//           with the scores, so their latency hides under the softmax.
// Then the 32 outputs are quantized as one group for the output projection.
constexpr int kExactChunk = 192;  // three waves of 64 rows
constexpr int kProdRow = kExactChunk + 4;  // one dimension's products over a chunk, padded: the
                                          // lanes' 128-bit reads of their rows spread over the banks
// the region after the weights: two buffers of value products
constexpr int kExactRegion = 2 * kWeighDims * kProdRow * 4;

inline size_t exact_attention_smem(size_t capacity) { return size_t((capacity + 15) / 16 * 16 + 16) * 4 + kExactRegion; }

template <int D>
__global__ __launch_bounds__(kAttnThreads) void attn_exact_kernel(AttnParams a)
{
    extern __shared__ __align__(16) float ash[];
    const int keys = a.keys, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int head = blockIdx.x, d0 = int(blockIdx.y) * kWeighDims;
    const int kv = head / (a.heads / a.kv_heads);
    float *w = ash;                                     // [capacity] scores, then weights
    float *red = w + (a.capacity + 15) / 16 * 16;       // [16]
    float *prod = red + 16;                             // [2][kWeighDims][kProdRow] value products
    const float *kbase = a.kcache + a.layer_base + size_t(kv) * a.capacity * D;
    const float *vbase = a.vcache + a.layer_base + size_t(kv) * a.capacity * D + d0;
    const int vpiece = lane & 7, vrow = lane >> 3;  // this lane's piece and row of a value load
    const int pw = wave - 1;                         // the product waves 1..3: 64 rows of a chunk each
    // (clamped re-reads past the last key: in bounds, never stored)
    auto fetch_rows = [&](int c, v4f *v) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int j = min(c * kExactChunk + pw * 64 + 8 * e + vrow, keys - 1);
            v[e] = *reinterpret_cast<const v4f *>(vbase + size_t(j) * D + 4 * vpiece);
        }
    };
    const float scale = 1.0f / sqrtf(float(D));
    float local_max = -INFINITY;
    if (wave == 0) {
        // the position's own key: lanes 4i .. 4i + 3 hold a quarter of the dimensions each, and
        // the quarters' products are added one after another, each lane continuing the sum the
        // previous quarter's lane passes on
        constexpr int DQ = D / 4;
        const int part = lane & 3;
        const float *qh = a.qkv + size_t(head) * D + part * DQ;
        const float *kn = kbase + size_t(keys - 1) * D + part * DQ;
        v4f qk[DQ / 4];
#pragma unroll
        for (int i = 0; i < DQ / 4; i++)
            qk[i] = *reinterpret_cast<const v4f *>(qh + 4 * i) * *reinterpret_cast<const v4f *>(kn + 4 * i);
        float s = -0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            float run = s;
#pragma unroll
            for (int i = 0; i < DQ / 4; i++) {
                run = run + qk[i].x;
                run = run + qk[i].y;
                run = run + qk[i].z;
                run = run + qk[i].w;
            }
            s = quad_broadcast(run, t);
        }
        if (lane == 0) {
            w[keys - 1] = s * scale;
            local_max = s * scale;
        }
    }
    const float *sc = a.scores + size_t(head) * a.capacity;
    for (int j = tid; j < keys - 1; j += kAttnThreads) {
        const float v = sc[j];
        w[j] = v;
        local_max = fmaxf(local_max, v);
    }
    // the value rows of the first two chunks: the softmax hides their latency
    v4f va[8], vb[8];
    if (wave > 0) {
        fetch_rows(0, va);
        if (kExactChunk < keys) fetch_rows(1, vb);
    }
    const float peak = attn_block_max(local_max, red);  // its barriers publish the scores
    for (int j = tid; j < keys; j += kAttnThreads) w[j] = ref_exp(w[j] - peak);
    __syncthreads();
    // the exponentials summed in index order by one lane
    if (tid == 0) red[8] = chain_sum(-0.0f, keys, w);
    __syncthreads();
    const float total = red[8];
    for (int j = tid; j < keys; j += kAttnThreads) w[j] = w[j] / total;
    float o = 0.0f;  // lanes 0..31 of wave 0: output d0 + lane
    // Chunk c's products from the registers `v` into `buf` (every weight read before the first
    // product is written: the compiler cannot tell the two regions apart)
    auto products = [&](int c, const v4f *v, float *buf) {
        const int j0 = c * kExactChunk, n = min(kExactChunk, keys - j0);
        float wj[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int r = pw * 64 + 8 * e + vrow;
            wj[e] = r < n ? w[j0 + r] : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float *col = buf + 4 * vpiece * kProdRow + pw * 64 + 8 * e + vrow;
            col[0] = wj[e] * v[e].x;
            col[kProdRow] = wj[e] * v[e].y;
            col[2 * kProdRow] = wj[e] * v[e].z;
            col[3 * kProdRow] = wj[e] * v[e].w;
        }
    };
    // Step k: after the barrier chunk k's products are whole and chunk k - 1's sums are done, so
    // waves 1..3 form chunk k + 1's products into the other buffer (and request chunk k + 3 into
    // the freed registers) while lanes 0..31 of wave 0 add chunk k's.
    const int chunks = (keys + kExactChunk - 1) / kExactChunk;
    float *const buf0 = prod, *const buf1 = prod + kWeighDims * kProdRow;
    auto step = [&](int k, v4f *vnext, float *bnext, const float *bcur) {
        __syncthreads();
        if (wave > 0 && k + 1 < chunks) {
            products(k + 1, vnext, bnext);
            if (k + 3 < chunks) fetch_rows(k + 3, vnext);
        }
        if (tid < kWeighDims) o = chain_sum(o, min(kExactChunk, keys - k * kExactChunk), bcur + tid * kProdRow);
    };
    __syncthreads();  // the weights
    if (wave > 0) {
        products(0, va, buf0);
        if (2 < chunks) fetch_rows(2, va);
    }
    for (int k = 0; k < chunks; k += 2) {
        step(k, vb, buf1, buf0);
        if (k + 1 < chunks) step(k + 1, va, buf0, buf1);
    }
    // the 32 outputs quantized as one group (eight lanes, four values each)
    __syncthreads();
    if (tid < kWeighDims) prod[tid] = o;
    __syncthreads();
    const int sub = tid & 7;
    if (tid < 8) {
        float x[4];
#pragma unroll
        for (int e = 0; e < 4; e++) x[e] = prod[sub * 4 + e];
        if (a.row_out) {
#pragma unroll
            for (int e = 0; e < 4; e++) a.row_out[head * D + d0 + sub * 4 + e] = x[e];
        }
        float amax = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
        amax = max8(fmaxf(0.0f, amax));
        int l0, l1, l2, l3;
        const float d = scale_and_levels(amax, x[0], x[1], x[2], x[3], l0, l1, l2, l3);
        const int sum = sum8(l0 + l1 + l2 + l3);
        const int G = (head * D + d0) / 32;
        reinterpret_cast<int *>(a.q)[G * 8 + sub] = pack4(l0, l1, l2, l3);
        if (sub == 0) {
            a.scales[G] = d;
            a.corr[G] = -a.zp * sum;
        }
    }
}

// A prefill's rotary embeddings and kept rows: row r's query and key heads rotated by halves at
// position first + r (ops.rs:77-85, the row's own angles), its key and value heads kept at that
// position (KvCache::keep, transformer.rs:166-180). Grid: (rows, heads + 2·kv_heads), D/2 threads.
__global__ void rope_keep_rows_kernel(float *__restrict__ qkv, size_t stride, const float *__restrict__ rope, int heads,
                                      int kv_heads, int D, float *__restrict__ kcache, float *__restrict__ vcache,
                                      size_t layer_base, int capacity, int first)
{
    const int r = int(blockIdx.x), unit = int(blockIdx.y), j = int(threadIdx.x), half = D / 2;
    if (j >= half) return;
    float *head = qkv + size_t(r) * stride + size_t(unit) * D;
    const int position = first + r;
    float x = head[j], y = head[j + half];
    if (unit < heads + kv_heads) {
        const float *cs = rope + size_t(position) * D;  // cos[half] then sin[half]
        const float c = cs[j], sn = cs[half + j];
        const float nx = x * c - y * sn;
        const float ny = y * c + x * sn;
        x = nx;
        y = ny;
        head[j] = x;
        head[j + half] = y;
    }
    if (unit >= heads) {
        const bool key = unit < heads + kv_heads;
        const int kv = (unit - heads) % kv_heads;
        float *cache = key ? kcache : vcache;
        const size_t at = layer_base + (size_t(kv) * capacity + size_t(position % capacity)) * D;
        cache[at + j] = x;
        cache[at + j + half] = y;
    }
}

// silu(gate)·up of a prefill's rows (layer.rs:321-341), quantized per group of 32 for the down
// projection with quantize_rows' arithmetic: 8 lanes per group, four values per lane.
__global__ void swiglu_quantize_kernel(const float *__restrict__ gate, const float *__restrict__ up, size_t groups, int zp,
                                       int8_t *__restrict__ q, float *__restrict__ scales, int32_t *__restrict__ corr)
{
    const size_t t = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t g = t / 8;
    const int sub = int(t % 8);
    const bool active = g < groups;
    const size_t at = active ? g * 8 + sub : 0;
    const float4 a = reinterpret_cast<const float4 *>(gate)[at], b = reinterpret_cast<const float4 *>(up)[at];
    const float4 v = make_float4(ref_silu(a.x) * b.x, ref_silu(a.y) * b.y, ref_silu(a.z) * b.z, ref_silu(a.w) * b.w);
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = max8(fmaxf(0.0f, amax));
    int l0, l1, l2, l3;
    const float d = scale_and_levels(amax, v.x, v.y, v.z, v.w, l0, l1, l2, l3);
    const int sum = sum8(l0 + l1 + l2 + l3);
    if (!active) return;
    reinterpret_cast<int *>(q)[at] = pack4(l0, l1, l2, l3);
    if (sub == 0) {
        scales[g] = d;
        corr[g] = -zp * sum;
    }
}

// Prediction::greedy (lm.rs:169-179) over the head's per-workgroup candidates: the first index of
// the largest logit; NaNs never win, and a NaN first logit keeps index 0.
__global__ __launch_bounds__(1024) void greedy_kernel(const float *__restrict__ pval, const int32_t *__restrict__ pidx, int n,
                                                      const float *__restrict__ logits, int32_t *out)
{
    __shared__ float bv[16];
    __shared__ int bi[16];
    const float first = logits[0];  // read at once, beside the candidates
    float best = 0.0f;
    int idx = -1;
    auto take = [&](float ob, int oi) {
        if (oi >= 0 && (idx < 0 || ob > best || (ob == best && oi < idx))) {
            best = ob;
            idx = oi;
        }
    };
    for (int i = threadIdx.x; i < n; i += blockDim.x) take(pval[i], pidx[i]);
    for (int m = 32; m >= 1; m >>= 1) take(__shfl_xor(best, m, 64), __shfl_xor(idx, m, 64));
    if ((threadIdx.x & 63) == 0) {
        bv[threadIdx.x >> 6] = best;
        bi[threadIdx.x >> 6] = idx;
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        // the waves' candidates, one per lane, reduced across the lanes
        const int waves = int(blockDim.x >> 6);
        best = 0.0f;
        idx = -1;
        if (int(threadIdx.x) < waves) {
            best = bv[threadIdx.x];
            idx = bi[threadIdx.x];
        }
        for (int m = 8; m >= 1; m >>= 1) take(__shfl_xor(best, m, 64), __shfl_xor(idx, m, 64));
        if (threadIdx.x == 0) *out = (first != first || idx < 0) ? 0 : idx;
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
    float *scores;     // [heads][capacity]
    float *part;       // fast attention: [heads][chunks][D + 4]
    int chunks, per_chunk;
    size_t score_smem, weigh_smem, exact_smem;
    int zp;
    // a prefill's rows (fg_qwen2_read), allocated on the first read and grown to its chunk
    struct {
        size_t rows;
        float *x, *qkv, *gate, *up, *scores;  // [rows][hidden], [rows][qkv], [rows][ffn] x2, [rows][heads][capacity]
        int8_t *lev;                          // [rows][widest]: the levels handed to the next product
        float *lsc;                           // [rows][widest / 32]
        int32_t *lco;
    } pre;
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
    p.qpw = 2;  // a rotary pair of quads per workgroup
    p.qstride = int(sh.head_dim / 8);
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

// Whether the attention runs as flash decoding merged by the output projection (parallel order).
bool fast_attention(const fg_qwen2 *m) { return !m->shape.exact && m->shape.heads * m->shape.head_dim <= 1024; }

// Whether, in the exact order, the query launch forms the cached keys' scores and the attention
// launch reads them (head sizes 64 and 128).
bool prescored_attention(const fg_qwen2 *m) { return m->shape.exact && (m->shape.head_dim == 64 || m->shape.head_dim == 128); }

// 1.-2. in parallel order, one launch: every query head's rows (RMSNorm + quantize -> product +
// bias -> RoPE) recomputed by each of its chunk workgroups, which then attend over their chunk of
// the cached keys [0, position); the key and value rows of the position projected, rotated and
// kept by the remaining workgroups. The output projection merges the chunks with the new key.
// In the exact order the same launch with the reference's sums, whose chunk workgroups write
// their keys' scores for the attention launch instead of attending.
int qattn_launch(fg_qwen2 *m, const fg_qwen2_layer &ly, size_t li, size_t position, hipStream_t st, int token = -1)
{
    const fg_qwen2_shape &sh = m->shape;
    // chunks of whole tiles over the cached keys, at most kMaxChunks per head (at least one)
    const int keys = int(position);
    const int per = (keys + kMaxChunks - 1) / kMaxChunks;
    m->per_chunk = std::max(kTileKeys, (per + kTileKeys - 1) / kTileKeys * kTileKeys);
    m->chunks = std::max(1, (keys + m->per_chunk - 1) / m->per_chunk);
    ProjParams p = table_params(ly.qkv);
    p.qpw = int(sh.head_dim / 4);  // a query head's quads
    p.qstride = 1;
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
    p.chunks = m->chunks;
    p.per_chunk = m->per_chunk;
    p.states = m->part;
    p.scores = m->scores;
    if (token >= 0) {
        // the first layer reads the token's table row itself (Buffers::embed_row, lm.rs:99-107)
        // and keeps it in hidden for the residual
        const fg_table *t = m->table;
        const size_t quad = size_t(token) / 4, qbytes = t->dtype == FG_Q4B32 ? 64 : 128;
        p.e_codes = t->codes + quad * t->blocks * qbytes;
        p.e_scales = t->scales + quad * t->groups * 4;
        p.e_lane = token % 4;
        p.x_out = m->hidden;
        return launch_proj(p, sh.dtype, IN_EMBED, OUT_QATTN, false, st);
    }
    return launch_proj(p, sh.dtype, IN_NORM, OUT_QATTN, sh.exact != 0, st);
}

// 3. and 5. a projection added to the residual row: of the attention's output (o: quantized by
// the attention, or merged from its chunks and the new key and quantized in the prologue), or of
// the silu(gate)·up row quantized by the SwiGLU epilogue (down).
int residual_launch(fg_qwen2 *m, const fg_table *t, int in, hipStream_t st, size_t li = 0, size_t position = 0,
                    float *merged_out = nullptr)
{
    const fg_qwen2_shape &sh = m->shape;
    ProjParams p = table_params(t);
    p.qpw = 1;
    if (in == IN_ATTN) {
        p.part = m->part;
        p.chunks = m->chunks;
        p.heads = int(sh.heads);
        p.kv_heads = int(sh.kv_heads);
        p.D = int(sh.head_dim);
        p.qkv_out = m->qkv;
        p.kcache = m->kcache;
        p.vcache = m->vcache;
        p.layer_base = li * sh.kv_heads * sh.capacity * sh.head_dim;
        p.capacity = int(sh.capacity);
        p.position = int(position);
        p.merged_out = merged_out;
    } else {
        p.q = m->xq;
        p.as = m->xs;
        p.corr = m->xc;
    }
    p.zp = m->zp;
    p.out = m->hidden;
    p.ld_out = long(t->quads * 4);
    p.accumulate = 1;
    return launch_proj(p, m->shape.dtype, in, OUT_STORE, m->shape.exact != 0, st);
}

// 4. RMSNorm -> gate and up -> silu(gate)·up (also to act_out, f32, when set).
int swiglu_launch(fg_qwen2 *m, const fg_qwen2_layer &ly, hipStream_t st, float *act_out = nullptr)
{
    const fg_qwen2_shape &sh = m->shape;
    ProjParams p = table_params(ly.gate);
    p.codes2 = ly.up->codes;
    p.wscales2 = ly.up->scales;
    p.qpw = 8;  // 32 outputs per workgroup: one group of the row, quantized in the epilogue
    p.x = m->hidden;
    p.norm_w = ly.norm2;
    p.eps = sh.eps;
    p.zp = m->zp;
    p.q_out = m->xq;
    p.s_out = m->xs;
    p.c_out = m->xc;
    p.act_out = act_out;
    return launch_proj(p, sh.dtype, IN_NORM, OUT_SWIGLU, sh.exact != 0, st);
}

int attention_launch(fg_qwen2 *m, size_t li, size_t position, hipStream_t st, float *row_out = nullptr)
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
    a.scores = m->scores;
    a.zp = m->zp;
    a.q = m->xq;
    a.scales = m->xs;
    a.corr = m->xc;
    a.row_out = row_out;
    const dim3 wgrid(unsigned(sh.heads), unsigned(sh.head_dim / kWeighDims));
    if (prescored_attention(m)) {
        // the cached keys' scores come from the query launch; the softmax and ordered weighted sums.
        // Past the default 64 KiB of LDS the kernel's limit is raised to the CU's 160 KiB on the
        // current device before each launch (a host call with no stream work), as the projection
        // and the batched product do: no per-model value that another model could lower.
        const void *f = sh.head_dim == 64 ? reinterpret_cast<const void *>(attn_exact_kernel<64>)
                                          : reinterpret_cast<const void *>(attn_exact_kernel<128>);
        if (m->exact_smem > 64 * 1024) FG_HIP(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        if (sh.head_dim == 64) attn_exact_kernel<64><<<wgrid, kAttnThreads, m->exact_smem, st>>>(a);
        else attn_exact_kernel<128><<<wgrid, kAttnThreads, m->exact_smem, st>>>(a);
        FG_HIP(hipGetLastError());
        return FG_OK;
    }
    const dim3 sgrid(unsigned(sh.kv_heads), unsigned((a.keys + kScoreKeys - 1) / kScoreKeys));
    attn_scores_kernel<<<sgrid, kAttnThreads, m->score_smem, st>>>(a);
    FG_HIP(hipGetLastError());
    if (sh.exact) attn_weigh_kernel<true><<<wgrid, kAttnThreads, m->weigh_smem, st>>>(a);
    else attn_weigh_kernel<false><<<wgrid, kAttnThreads, m->weigh_smem, st>>>(a);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

// token >= 0: the layer's input is that table row (the first layer of a step in parallel order)
int run_layer(fg_qwen2 *m, size_t li, size_t position, hipStream_t st, int token = -1)
{
    const fg_qwen2_layer &ly = m->layers[li];
    int rc;
    if (fast_attention(m)) {
        if ((rc = qattn_launch(m, ly, li, position, st, token))) return rc;
        if ((rc = residual_launch(m, ly.o, IN_ATTN, st, li, position))) return rc;
    } else {
        if ((rc = prescored_attention(m) ? qattn_launch(m, ly, li, position, st) : qkv_launch(m, ly, li, position, st)))
            return rc;
        if ((rc = attention_launch(m, li, position, st))) return rc;
        if ((rc = residual_launch(m, ly.o, IN_PREQ, st))) return rc;
    }
    if ((rc = swiglu_launch(m, ly, st))) return rc;
    return residual_launch(m, ly.down, IN_PREQ, st);
}

int head_launch(fg_qwen2 *m, hipStream_t st)
{
    const fg_qwen2_shape &sh = m->shape;
    ProjParams p = table_params(m->table);
    p.x = m->hidden;
    p.norm_w = m->final_norm;
    p.eps = sh.eps;
    p.zp = m->zp;
    // the final norm's row formed once (not in each of the product's workgroups)
    p.q_out = m->xq;
    p.s_out = m->xs;
    p.c_out = m->xc;
    int rc = launch_norm_quantize(p, sh.exact != 0, st);
    if (rc) return rc;
    p.q = m->xq;
    p.as = m->xs;
    p.corr = m->xc;
    p.qpw = kHeadQuads;
    p.out = m->logits;
    p.ld_out = long(m->table->quads * 4);
    p.pval = m->pval;
    p.pidx = m->pidx;
    return launch_proj(p, sh.dtype, IN_PREQ, OUT_STORE, sh.exact != 0, st);
}

// ------------------------------------------------------------------ prefill (Reader::read)

void free_prefill(fg_qwen2 *m)
{
    void *ptrs[] = {m->pre.x, m->pre.qkv, m->pre.gate, m->pre.up, m->pre.scores, m->pre.lev, m->pre.lsc, m->pre.lco};
    for (void *p : ptrs)
        if (p) (void)hipFree(p);
    m->pre = {};
}

// Room for `rows` rows of a prefill (grown once past what an earlier read used).
int ensure_prefill(fg_qwen2 *m, size_t rows)
{
    if (m->pre.rows >= rows) return FG_OK;
    free_prefill(m);
    const fg_qwen2_shape &sh = m->shape;
    const size_t qkv_w = (sh.heads + 2 * sh.kv_heads) * sh.head_dim, width = sh.heads * sh.head_dim;
    const size_t widest = std::max(sh.hidden, std::max(width, sh.ffn));
    struct {
        void **ptr;
        size_t bytes;
    } allocs[] = {
        {reinterpret_cast<void **>(&m->pre.x), rows * sh.hidden * 4},
        {reinterpret_cast<void **>(&m->pre.qkv), rows * qkv_w * 4},
        {reinterpret_cast<void **>(&m->pre.gate), rows * sh.ffn * 4},
        {reinterpret_cast<void **>(&m->pre.up), rows * sh.ffn * 4},
        {reinterpret_cast<void **>(&m->pre.scores), rows * sh.heads * sh.capacity * 4},
        {reinterpret_cast<void **>(&m->pre.lev), rows * widest},
        {reinterpret_cast<void **>(&m->pre.lsc), rows * widest / 32 * 4},
        {reinterpret_cast<void **>(&m->pre.lco), rows * widest / 32 * 4},
    };
    for (auto &a : allocs) {
        const hipError_t e = hipMalloc(a.ptr, a.bytes);
        if (e != hipSuccess) {
            free_prefill(m);
            return check_hip(e, "fg_qwen2_read: hipMalloc");
        }
    }
    m->pre.rows = rows;
    return FG_OK;
}

// RMSNorm + quantize of the prefill's n rows (ops.rs:7-16, the model's order) into its levels.
int prefill_norm(fg_qwen2 *m, const float *weight, int n, hipStream_t st)
{
    const fg_qwen2_shape &sh = m->shape;
    ProjParams p{};
    p.K = int(sh.hidden);
    p.G = int(sh.hidden / 32);
    p.B = p.G;
    p.x = m->pre.x;
    p.norm_w = weight;
    p.eps = sh.eps;
    p.zp = m->zp;
    p.q_out = m->pre.lev;
    p.s_out = m->pre.lsc;
    p.c_out = m->pre.lco;
    return launch_norm_quantize_rows(p, n, sh.exact != 0, st);
}

// The product of the prefill's n quantized rows (every output, the reference's group order) into
// out (ld columns per row), written or added.
int prefill_product(fg_qwen2 *m, const fg_table *t, int n, const float *bias, float *out, size_t ld, bool accumulate,
                    hipStream_t st)
{
    ProductArgs a{};
    a.t = t;
    a.q = m->pre.lev;
    a.as = m->pre.lsc;
    a.corr = m->pre.lco;
    a.rows = size_t(n);
    a.quad_begin = 0;
    a.quad_end = t->quads;
    a.bias = bias;
    a.out = out;
    a.ld_out = ld;
    a.accumulate = accumulate ? 1 : 0;
    return launch_product(a, st);
}

// One layer over the prefill's n rows at positions first .. first + n - 1 (layer.rs:161-344 with
// rows > 1): each step over every row, the products on the matrix cores.
int prefill_layer(fg_qwen2 *m, size_t li, size_t first, int n, hipStream_t st)
{
    const fg_qwen2_shape &sh = m->shape;
    const fg_qwen2_layer &ly = m->layers[li];
    const size_t qkv_w = (sh.heads + 2 * sh.kv_heads) * sh.head_dim, width = sh.heads * sh.head_dim;
    const size_t layer_base = li * sh.kv_heads * sh.capacity * sh.head_dim;
    int rc;
    // prepare + QKV (layer/input.rs:22-66), rotary embeddings and the kept keys and values
    if ((rc = prefill_norm(m, ly.norm1, n, st))) return rc;
    if ((rc = prefill_product(m, ly.qkv, n, ly.qkv_bias, m->pre.qkv, qkv_w, false, st))) return rc;
    // rotary embeddings, the kept keys and values, and the attention of every row over the keys up
    // to its own position (Mask::Causal), its output row quantized for the output projection
    AttnParams a{};
    a.qkv = m->pre.qkv;
    a.qkv_stride = qkv_w;
    a.kcache = m->kcache;
    a.vcache = m->vcache;
    a.layer_base = layer_base;
    a.heads = int(sh.heads);
    a.kv_heads = int(sh.kv_heads);
    a.D = int(sh.head_dim);
    a.capacity = int(sh.capacity);
    a.keys = int(first) + 1;
    a.scores = m->pre.scores;
    a.zp = m->zp;
    a.q = m->pre.lev;
    a.scales = m->pre.lsc;
    a.corr = m->pre.lco;
    a.row_width = width;
    const int D = int(sh.head_dim), kmax = int(first) + n;
    if (const size_t rsmem = attn_rows_smem(D, kmax)) {
        // blocks of rows sharing their keys and values (each row over its own keys), the chunk's
        // rows rotated and kept on the way
        a.rope = m->rope;
        a.kkeep = m->kcache;
        a.vkeep = m->vcache;
        const int R = kAttnThreads / D;
        const dim3 rgrid(unsigned(sh.heads), unsigned((n + R - 1) / R));
        if (sh.exact) attn_rows_kernel<true><<<rgrid, kAttnThreads, rsmem, st>>>(a, n, (kmax + 3) / 4 * 4);
        else attn_rows_kernel<false><<<rgrid, kAttnThreads, rsmem, st>>>(a, n, (kmax + 3) / 4 * 4);
    } else {
        rope_keep_rows_kernel<<<dim3(unsigned(n), unsigned(sh.heads + 2 * sh.kv_heads)), unsigned(sh.head_dim / 2), 0, st>>>(
            m->pre.qkv, qkv_w, m->rope, int(sh.heads), int(sh.kv_heads), int(sh.head_dim), m->kcache, m->vcache, layer_base,
            int(sh.capacity), int(first));
        FG_HIP(hipGetLastError());
        const dim3 sgrid(unsigned(sh.kv_heads), unsigned((first + n + kScoreKeys - 1) / kScoreKeys), unsigned(n));
        attn_scores_kernel<<<sgrid, kAttnThreads, m->score_smem, st>>>(a);
        FG_HIP(hipGetLastError());
        const dim3 wgrid(unsigned(sh.heads), unsigned(sh.head_dim / kWeighDims), unsigned(n));
        if (sh.exact) attn_weigh_kernel<true><<<wgrid, kAttnThreads, m->weigh_smem, st>>>(a);
        else attn_weigh_kernel<false><<<wgrid, kAttnThreads, m->weigh_smem, st>>>(a);
    }
    FG_HIP(hipGetLastError());
    // hidden += o(attention) (layer.rs:239-245)
    if ((rc = prefill_product(m, ly.o, n, nullptr, m->pre.x, sh.hidden, true, st))) return rc;
    // hidden += down(silu(gate(x))·up(x)), x the normed rows (layer.rs:249-344)
    if ((rc = prefill_norm(m, ly.norm2, n, st))) return rc;
    {
        // gate and up of the same rows, one launch where the kernel allows it
        ProductArgs g{}, u{};
        g.t = ly.gate;
        u.t = ly.up;
        for (ProductArgs *a : {&g, &u}) {
            a->q = m->pre.lev;
            a->as = m->pre.lsc;
            a->corr = m->pre.lco;
            a->rows = size_t(n);
            a->quad_begin = 0;
            a->quad_end = a->t->quads;
            a->ld_out = sh.ffn;
        }
        g.out = m->pre.gate;
        u.out = m->pre.up;
        if ((rc = launch_product_pair(g, u, st))) return rc;
    }
    const size_t groups = size_t(n) * sh.ffn / 32;
    swiglu_quantize_kernel<<<unsigned((groups * 8 + 255) / 256), 256, 0, st>>>(m->pre.gate, m->pre.up, groups, m->zp, m->pre.lev,
                                                                              m->pre.lsc, m->pre.lco);
    FG_HIP(hipGetLastError());
    return prefill_product(m, ly.down, n, nullptr, m->pre.x, sh.hidden, true, st);
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
    if (sh.hidden % 32 || sh.ffn % 32 || sh.hidden > 4096 || sh.capacity == 0 || sh.capacity > 8192)
        return set_error(FG_ERR_SHAPE, "fg_qwen2_create: hidden and ffn must be whole groups (hidden <= 4096, capacity <= 8192)");
    const size_t qkv_w = (sh.heads + 2 * sh.kv_heads) * sh.head_dim, width = sh.heads * sh.head_dim;
    for (size_t l = 0; l < sh.layers; l++) {
        const fg_qwen2_layer &ly = layers[l];
        if (!ly.norm1 || !ly.norm2 || (reinterpret_cast<uintptr_t>(ly.norm1) & 15) || (reinterpret_cast<uintptr_t>(ly.norm2) & 15))
            return set_error(FG_ERR_ARG, "fg_qwen2_create: norm weights must be 16-byte aligned device arrays");
        if (!table_is(ly.qkv, sh.dtype, qkv_w, sh.hidden) || !table_is(ly.o, sh.dtype, sh.hidden, width) ||
            !table_is(ly.gate, sh.dtype, sh.ffn, sh.hidden) || !table_is(ly.up, sh.dtype, sh.ffn, sh.hidden) ||
            !table_is(ly.down, sh.dtype, sh.hidden, sh.ffn))
            return set_error(FG_ERR_SHAPE, "fg_qwen2_create: layer " + std::to_string(l) + " tables do not fit the shape");
    }
    if (!table_is(table, sh.dtype, sh.vocab, sh.hidden)) return set_error(FG_ERR_SHAPE, "fg_qwen2_create: the table is not [vocab, hidden]");
    if (reinterpret_cast<uintptr_t>(final_norm) & 15) return set_error(FG_ERR_ARG, "fg_qwen2_create: norm weights must be 16-byte aligned device arrays");
    fg_qwen2 *m = new fg_qwen2();
    m->shape = sh;
    m->layers.assign(layers, layers + sh.layers);
    m->final_norm = final_norm;
    m->table = table;
    m->kcache = kcache;
    m->vcache = vcache;
    m->zp = zero_point_of(sh.dtype);
    m->head_groups = int((table->quads + kHeadQuads - 1) / kHeadQuads);
    // attention LDS: a block of keys and the group's queries; a chunk of values and the weights
    const int D = int(sh.head_dim);
    const int group = int(sh.heads / sh.kv_heads);
    m->score_smem = size_t(kScoreKeys * (D + 1) + group * D) * 4;
    m->weigh_smem = size_t(kWeighKeys * (kWeighDims + 1) + sh.capacity + 8 * kWeighDims + 16) * 4;
    m->exact_smem = exact_attention_smem(sh.capacity);
    if (group * D > 4 * kAttnThreads || m->score_smem > 64 * 1024 || m->weigh_smem > 64 * 1024 ||
        m->exact_smem > 160 * 1024) {
        delete m;
        return set_error(FG_ERR_SHAPE, "fg_qwen2_create: the attention does not fit (heads per KV head x head_dim <= 1024, capacity)");
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
        {reinterpret_cast<void **>(&m->scores), sh.heads * sh.capacity * 4},
        {reinterpret_cast<void **>(&m->part), sh.heads * kMaxChunks * (sh.head_dim + 4) * 4},
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

extern "C" int fg_qwen2_attention(fg_qwen2 *m, size_t layer, size_t position, const float *hidden, float *query, float *row,
                                  void *stream)
{
    if (!m || !hidden || !query || !row) return set_error(FG_ERR_ARG, "fg_qwen2_attention: a null argument");
    if (layer >= m->shape.layers || position >= m->shape.capacity)
        return set_error(FG_ERR_SHAPE, "fg_qwen2_attention: layer or position out of range");
    const fg_qwen2_shape &sh = m->shape;
    const fg_qwen2_layer &ly = m->layers[layer];
    hipStream_t st = as_stream(stream);
    FG_HIP(hipMemcpyAsync(m->hidden, hidden, sh.hidden * 4, hipMemcpyDeviceToDevice, st));
    int rc;
    if (fast_attention(m)) {
        // the chunks, then their merge in the output projection's prologue (which also writes the
        // projection to the model's own hidden row, not the caller's)
        if ((rc = qattn_launch(m, ly, layer, position, st))) return rc;
        if ((rc = residual_launch(m, ly.o, IN_ATTN, st, layer, position, row))) return rc;
    } else {
        if ((rc = prescored_attention(m) ? qattn_launch(m, ly, layer, position, st) : qkv_launch(m, ly, layer, position, st)))
            return rc;
        if ((rc = attention_launch(m, layer, position, st, row))) return rc;
    }
    FG_HIP(hipMemcpyAsync(query, m->qkv, sh.heads * sh.head_dim * 4, hipMemcpyDeviceToDevice, st));
    return FG_OK;
}

extern "C" int fg_qwen2_layer_probe(fg_qwen2 *m, size_t layer, size_t position, const float *hidden,
                                    const fg_qwen2_probe *probe, void *stream)
{
    if (!m || !hidden || !probe) return set_error(FG_ERR_ARG, "fg_qwen2_layer_probe: a null argument");
    if (layer >= m->shape.layers || position >= m->shape.capacity)
        return set_error(FG_ERR_SHAPE, "fg_qwen2_layer_probe: layer or position out of range");
    const fg_qwen2_shape &sh = m->shape;
    const fg_qwen2_layer &ly = m->layers[layer];
    const size_t width = sh.heads * sh.head_dim, groups = sh.ffn / 32;
    hipStream_t st = as_stream(stream);
    auto copy = [&](void *to, const void *from, size_t bytes) -> hipError_t {
        return to ? hipMemcpyAsync(to, from, bytes, hipMemcpyDeviceToDevice, st) : hipSuccess;
    };
    FG_HIP(hipMemcpyAsync(m->hidden, hidden, sh.hidden * 4, hipMemcpyDeviceToDevice, st));
    int rc;
    // attention and the output projection, as run_layer runs them (the attention row captured by
    // the launch that forms it)
    if (fast_attention(m)) {
        if ((rc = qattn_launch(m, ly, layer, position, st))) return rc;
        if ((rc = residual_launch(m, ly.o, IN_ATTN, st, layer, position, probe->attention))) return rc;
    } else {
        if ((rc = prescored_attention(m) ? qattn_launch(m, ly, layer, position, st) : qkv_launch(m, ly, layer, position, st)))
            return rc;
        if ((rc = attention_launch(m, layer, position, st, probe->attention))) return rc;
        if ((rc = residual_launch(m, ly.o, IN_PREQ, st))) return rc;
    }
    FG_HIP(copy(probe->query, m->qkv, width * 4));
    FG_HIP(copy(probe->attended, m->hidden, sh.hidden * 4));
    // the feed-forward: silu(gate)·up captured by its epilogue, then the row it quantized for down
    if ((rc = swiglu_launch(m, ly, st, probe->inner))) return rc;
    FG_HIP(copy(probe->levels, m->xq, sh.ffn));
    FG_HIP(copy(probe->scales, m->xs, groups * 4));
    FG_HIP(copy(probe->corrections, m->xc, groups * 4));
    if ((rc = residual_launch(m, ly.down, IN_PREQ, st))) return rc;
    FG_HIP(copy(probe->out, m->hidden, sh.hidden * 4));
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
    // the embedding row (lm.rs:99-107): in parallel order the first layer's launch reads it
    int rc = FG_OK;
    const bool fast = fast_attention(m);
    if (!fast && (rc = launch_dequantize_row(m->table, size_t(token), m->hidden, st))) return rc;
    for (size_t l = 0; l < sh.layers; l++)
        if ((rc = run_layer(m, l, position, st, l == 0 && fast ? token : -1))) return rc;
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

extern "C" int fg_qwen2_embed(fg_qwen2 *m, const int32_t *ids, size_t count, float *out, void *stream)
{
    if (!m || (count && (!ids || !out))) return set_error(FG_ERR_ARG, "fg_qwen2_embed: a null argument");
    return launch_embed_rows(m->table, ids, count, out, as_stream(stream));
}

extern "C" int fg_qwen2_read(fg_qwen2 *m, const float *embeddings, size_t count, size_t first, size_t chunk, float *hidden,
                             float *logits, int32_t *next_token, void *stream)
{
    if (!m || !embeddings) return set_error(FG_ERR_ARG, "fg_qwen2_read: a null argument");
    const fg_qwen2_shape &sh = m->shape;
    if (count == 0 || chunk == 0) return set_error(FG_ERR_SHAPE, "fg_qwen2_read: no rows, or chunks of none");
    // transformer.rs:329-341: the cache holds every key the span sees
    if (first + count > sh.capacity) return set_error(FG_ERR_SHAPE, "fg_qwen2_read: the cache holds every key the span sees");
    chunk = std::min(std::min(chunk, count), size_t(4096));
    hipStream_t st = as_stream(stream);
    int rc = ensure_prefill(m, chunk);
    if (rc) return rc;
    for (size_t start = 0; start < count; start += chunk) {
        const size_t n = std::min(chunk, count - start);
        FG_HIP(hipMemcpyAsync(m->pre.x, embeddings + start * sh.hidden, n * sh.hidden * 4, hipMemcpyDeviceToDevice, st));
        for (size_t l = 0; l < sh.layers; l++)
            if ((rc = prefill_layer(m, l, first + start, int(n), st))) return rc;
        if (start + n == count)
            FG_HIP(hipMemcpyAsync(m->hidden, m->pre.x + (n - 1) * sh.hidden, sh.hidden * 4, hipMemcpyDeviceToDevice, st));
    }
    // the last row's prediction (Prediction::predict, lm.rs:147-166)
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
    free_prefill(m);
    void *ptrs[] = {m->hidden, m->qkv, m->logits, m->rope, m->xq, m->xs, m->xc, m->pval, m->pidx, m->scores, m->part};
    for (void *p : ptrs)
        if (p) (void)hipFree(p);
    delete m;
    return FG_OK;
}
