// The decode product: a few activation rows (1..4) against a quantized table, HBM-bound, with the
// decoder's neighbours fused in.
//
// Reference: matmul (matmul.rs:265-317) -> quant_tiles / quant_tile / quad_pass / accumulate
// (matmul.rs:521-763) with the scalar backend's arithmetic (arch/scalar.rs:68-90). Per output
// column n and activation row r:  D_g = corr_g + Σ_k u[n,k]·a[r,k]  (int32, exact in any order),
//   s = +0;  for g in order:  s = fl(s + fl(fl((float)D_g) · fl(ws[n,g] · as[r,g])))
// then the bias (linear.rs:63-68) and, for residual projections, h = fl(h + y) (linear.rs:134-143).
//
// Mapping. A workgroup owns `qpw` quads (4 output rows each; consecutive, or a rotary pair D/8
// quads apart) and all of their blocks (in two tables for the gated feed-forward's gate and up).
// Its four waves stream them in 1 KiB chunks (64 lanes x 16 B, coalesced 128-bit loads),
// `kBatch` chunks per wave in flight (the fewest that cover a wave's share), the next batch
// issued before the current one is consumed. The entry is branch-free, so the parameters arrive
// in one scalar round trip ahead of the first vector load.
// Small workgroups (a few quads, about 16 KiB of codes) spread a small table over every CU: a
// CU keeps a bounded number of reads in flight, so a large share per CU costs round trips.
// The first batch is issued before the activations are staged, so the prologue (a copy, an
// in-kernel quantization, or an RMSNorm followed by the quantization) runs under the weights'
// memory latency. Every lane turns its 16 bytes into a partial int32 dot with v_dot4 against the
// activations in LDS, scales its group's total (exact integer; 7/8-bit row-blocks are split over
// two lanes and summed through DPP) into the group's f32 term and parks it in LDS. Once all terms
// are in, one thread per output adds them in group order, the reference's sum to the bit.
//
// Epilogues: store (with bias, or added to a residual row, optionally each workgroup's greedy
// candidate); QKV (bias, rotary embedding by halves of the query and key heads, the key and value
// heads kept in the cache: rope_half ops.rs:77-85, KvCache::keep transformer.rs:166-180); SwiGLU
// (silu(gate)·up as f32, layer.rs:321-341, which the down projection quantizes as its input);
// query attention (one query head's rows rotated, then attended over one chunk of the cached keys,
// ops.rs:301-342 and transformer.rs:185-219 in parallel order; the key and value rows of the position
// kept by the remaining workgroups).
//
// This header holds the kernel and its device helpers; it is instantiated by the translation units
// that dispatch it: matvec.hip (the product's own rows 1..4) and proj_q8.hip / proj_q4.hip (the
// decoder's launches, one per weight format). Everything here has internal linkage.
#pragma once

#include <algorithm>

#include "common.h"
#include "proj.h"

namespace fg {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ int dot16(int4 w, int4 a) { return dot4(w.w, a.w, dot4(w.z, a.z, dot4(w.y, a.y, dot4(w.x, a.x, 0)))); }

// Σ t[g] for g in 0..n, added in index order from +0. `t` is 16-byte aligned and readable up to n
// rounded up to 4. Whole runs of 32 terms come in eight 128-bit reads into two register sets in
// turn: run c + 1's reads (clamped, never past the last run) go out before run c is added, so one
// lane's chain of additions never waits for LDS (no copies between the sets, which would make the
// additions wait for the reads in flight). Then the tail.
__device__ __forceinline__ float ordered_sum(const float *t, int n)
{
    constexpr int V = 8;  // 128-bit reads per run
    const v4f *t4 = reinterpret_cast<const v4f *>(t);
    const int runs = n / (4 * V);
    float s = 0.0f;
    v4f A[V], B[V];
    auto load = [&](v4f *r, int c) {
#pragma unroll
        for (int k = 0; k < V; k++) r[k] = t4[c * V + k];
    };
    auto add = [&](const v4f *r) {
#pragma unroll
        for (int k = 0; k < V; k++) {
            s = s + r[k].x;
            s = s + r[k].y;
            s = s + r[k].z;
            s = s + r[k].w;
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
    const int g0 = runs * 4 * V, rest4 = (n - g0 + 3) / 4;  // uniform
    if (rest4 > 0) {
        v4f cur[V];
#pragma unroll
        for (int k = 0; k < V; k++) cur[k] = t4[runs * V + min(k, rest4 - 1)];
        // the row is zero-padded to whole float4s, and s is never -0 (it starts at +0), so the
        // padding's +0 terms change nothing; whole float4s end on a scalar branch
#pragma unroll
        for (int k = 0; k < V; k++) {
            if (k >= rest4) break;
            s = s + cur[k].x;
            s = s + cur[k].y;
            s = s + cur[k].z;
            s = s + cur[k].w;
        }
    }
    return s;
}

// The activations' global loads, issued before the first weight batch: vector loads complete in
// order, so loads issued after the weights would wait for them.
typedef int v4i __attribute__((ext_vector_type(4)));

struct StageRegs {
    v4i v0, v1, v2, v3;
    float s0, s1, s2, s3;
    int c0, c1, c2, c3;
    v4f f0, f1, f2, f3;  // f32 rows (IN_F32) or the row to normalize (IN_NORM)
    v4f f4, f5, f6, f7;  // more f32 rows (IN_F32)
    v4f pa[kMaxChunks];  // IN_ATTN: this lane's four sums of every chunk, and the chunks' max and total
    float pm[kMaxChunks], pl[kMaxChunks];
    v4f w0, w1, w2, w3;  // the RMSNorm weight (IN_NORM)
    v4f qn, kn, vn;      // IN_ATTN: this lane's four dims of the rotated query, new key and new value
};


template <int FMT, int R, int IN>
__device__ __forceinline__ void stage_issue(const ProjParams &p, StageRegs &g)
{
    const int tid = threadIdx.x;
    const int K = p.K, G = p.G;
    if (IN == IN_PREQ) {
        const v4i *src = reinterpret_cast<const v4i *>(p.q);
        const int n16 = R * K / 16, ng = R * G;
        g.v0 = src[unsigned(min(tid, n16 - 1))];
        g.v1 = src[unsigned(min(tid + kThreads, n16 - 1))];
        g.v2 = src[unsigned(min(tid + 2 * kThreads, n16 - 1))];
        g.v3 = src[unsigned(min(tid + 3 * kThreads, n16 - 1))];
        g.s0 = p.as[unsigned(min(tid, ng - 1))];
        g.s1 = p.as[unsigned(min(tid + kThreads, ng - 1))];
        g.s2 = p.as[unsigned(min(tid + 2 * kThreads, ng - 1))];
        g.s3 = p.as[unsigned(min(tid + 3 * kThreads, ng - 1))];
        g.c0 = p.corr[unsigned(min(tid, ng - 1))];
        g.c1 = p.corr[unsigned(min(tid + kThreads, ng - 1))];
        g.c2 = p.corr[unsigned(min(tid + 2 * kThreads, ng - 1))];
        g.c3 = p.corr[unsigned(min(tid + 3 * kThreads, ng - 1))];
    } else if (IN == IN_F32) {
        const v4f *x4 = reinterpret_cast<const v4f *>(p.x);
        const int n4 = R * K / 4;
        g.f0 = x4[unsigned(min(tid, n4 - 1))];
        g.f1 = x4[unsigned(min(tid + kThreads, n4 - 1))];
        g.f2 = x4[unsigned(min(tid + 2 * kThreads, n4 - 1))];
        g.f3 = x4[unsigned(min(tid + 3 * kThreads, n4 - 1))];
        g.f4 = x4[unsigned(min(tid + 4 * kThreads, n4 - 1))];
        g.f5 = x4[unsigned(min(tid + 5 * kThreads, n4 - 1))];
        g.f6 = x4[unsigned(min(tid + 6 * kThreads, n4 - 1))];
        g.f7 = x4[unsigned(min(tid + 7 * kThreads, n4 - 1))];
    } else if (IN == IN_ATTN) {
        // lane t merges float4 t of the attention row (head t·4 / D); every chunk's record at once
        const int e = min(tid, K / 4 - 1);
        const int h = (e * 4) >> p.dshift, d4 = e * 4 - h * p.D;
        const size_t at = p.layer_base + (size_t(divq(h, p.rcp_group)) * p.capacity + size_t(p.position)) * p.D + d4;
        g.qn = *reinterpret_cast<const v4f *>(p.qkv_out + size_t(h) * p.D + d4);
        g.kn = *reinterpret_cast<const v4f *>(p.kcache + at);
        g.vn = *reinterpret_cast<const v4f *>(p.vcache + at);
#pragma unroll
        for (int c = 0; c < kMaxChunks; c++) {
            const float *rec = p.part + size_t(h * p.chunks + min(c, p.chunks - 1)) * (p.D + 4);
            const float2 ml = *reinterpret_cast<const float2 *>(rec);  // the maximum and total
            g.pm[c] = ml.x;
            g.pl[c] = ml.y;
            g.pa[c] = *reinterpret_cast<const v4f *>(rec + 4 + d4);
        }
    } else if (IN == IN_EMBED) {
        // float4 i of the table row: four codes of block i / 8 as one dword (Q7/Q8 bytes
        // 4·(i % 8) ..; Q4 the nibbles of bytes 4·(i % 4) .. at shift 4·((i % 8) / 4)), and the
        // block's scale
        const int n4 = K / 4;
        const int *c4 = reinterpret_cast<const int *>(p.e_codes);
        const int rowdw = FMT == 8 ? 8 : 4;  // dwords of a row-block
        auto at = [&](int i) { return unsigned((i >> 3) * (4 * rowdw) + p.e_lane * rowdw + (FMT == 8 ? (i & 7) : (i & 3))); };
        auto sc = [&](int i) { return unsigned((i >> 3) * 4 + p.e_lane); };
        const int i0 = min(tid, n4 - 1), i1 = min(tid + kThreads, n4 - 1), i2 = min(tid + 2 * kThreads, n4 - 1),
                  i3 = min(tid + 3 * kThreads, n4 - 1);
        g.c0 = c4[at(i0)];
        g.c1 = c4[at(i1)];
        g.c2 = c4[at(i2)];
        g.c3 = c4[at(i3)];
        g.s0 = p.e_scales[sc(i0)];
        g.s1 = p.e_scales[sc(i1)];
        g.s2 = p.e_scales[sc(i2)];
        g.s3 = p.e_scales[sc(i3)];
        const v4f *w4 = reinterpret_cast<const v4f *>(p.norm_w);
        g.w0 = w4[unsigned(i0)];
        g.w1 = w4[unsigned(i1)];
        g.w2 = w4[unsigned(i2)];
        g.w3 = w4[unsigned(i3)];
    } else {
        // one row of at most 4 · 256 float4s (K <= 4096, checked on the host)
        const v4f *x4 = reinterpret_cast<const v4f *>(p.x);
        const v4f *w4 = reinterpret_cast<const v4f *>(p.norm_w);
        const int n4 = K / 4;
        g.f0 = x4[unsigned(min(tid, n4 - 1))];
        g.f1 = x4[unsigned(min(tid + kThreads, n4 - 1))];
        g.f2 = x4[unsigned(min(tid + 2 * kThreads, n4 - 1))];
        g.f3 = x4[unsigned(min(tid + 3 * kThreads, n4 - 1))];
        g.w0 = w4[unsigned(min(tid, n4 - 1))];
        g.w1 = w4[unsigned(min(tid + kThreads, n4 - 1))];
        g.w2 = w4[unsigned(min(tid + 2 * kThreads, n4 - 1))];
        g.w3 = w4[unsigned(min(tid + 3 * kThreads, n4 - 1))];
    }
}

// Quantize `n` float4 slots per thread (slot k of thread t is float4 t + k·256 of the staged rows;
// eight consecutive threads hold one group of 32) into the staging arrays. Slots are taken two at
// a time, so that two groups' arithmetic interleaves; a wave skips the slots none of its lanes
// holds, and each lane stores only the groups it holds.
template <int S>
__device__ __forceinline__ void quantize_slots(const v4f (&v)[S], int n4, int zp, int8_t *q, float *scales, int32_t *corr)
{
    const int tid = threadIdx.x, first = tid & ~63;
#pragma unroll
    for (int k = 0; k < S; k += 2) {
        if (k + 1 < S && first + (k + 1) * kThreads < n4) {
            Group8 gr[2];
            quantize_groups<2>(&v[k], gr);
            if (tid + k * kThreads < n4) store_group8(gr[0], zp, (tid + k * kThreads) / 8, q, scales, corr);
            if (tid + (k + 1) * kThreads < n4) store_group8(gr[1], zp, (tid + (k + 1) * kThreads) / 8, q, scales, corr);
        } else if (first + k * kThreads < n4) {
            Group8 gr[1];
            quantize_groups<1>(&v[k], gr);
            if (tid + k * kThreads < n4) store_group8(gr[0], zp, (tid + k * kThreads) / 8, q, scales, corr);
        }
    }
}

template <int FMT, int R, int IN, bool EXACT>
__device__ __forceinline__ void stage_finish(const ProjParams &p, const StageRegs &g, int8_t *act_q, float *act_s,
                                             int32_t *act_c, float *nbuf, float *red)
{
    const int tid = threadIdx.x;
    const int K = p.K, G = p.G;
    if (IN == IN_PREQ) {
        const v4i *src = reinterpret_cast<const v4i *>(p.q);
        v4i *dst = reinterpret_cast<v4i *>(act_q);
        const int n16 = R * K / 16, ng = R * G;
#define FG_STASH(k, v, sc, co)                   \
    {                                            \
        const int i = tid + (k) * kThreads;      \
        if (i < n16) dst[i] = (v);               \
        if (i < ng) {                            \
            act_s[i] = (sc);                     \
            act_c[i] = (co);                     \
        }                                        \
    }
        FG_STASH(0, g.v0, g.s0, g.c0)
        FG_STASH(1, g.v1, g.s1, g.c1)
        FG_STASH(2, g.v2, g.s2, g.c2)
        FG_STASH(3, g.v3, g.s3, g.c3)
#undef FG_STASH
        for (int i = tid + 4 * kThreads; i < n16; i += kThreads) dst[i] = src[i];
        for (int i = tid + 4 * kThreads; i < ng; i += kThreads) {
            act_s[i] = p.as[i];
            act_c[i] = p.corr[i];
        }
    } else if (IN == IN_F32) {
        // 8 lanes per group of 32 (quantize_rows): thread t holds float4s t, t + 256, ... of the rows
        const int n4 = R * K / 4;
        const v4f slots[8] = {g.f0, g.f1, g.f2, g.f3, g.f4, g.f5, g.f6, g.f7};
        quantize_slots<8>(slots, n4, p.zp, act_q, act_s, act_c);
        for (int i0 = 8 * kThreads; i0 < n4; i0 += kThreads) {  // rows past 8 float4s per thread
            const int i = min(tid + i0, n4 - 1);
            const v4f rest[1] = {reinterpret_cast<const v4f *>(p.x)[i]};
            Group8 gr[1];
            quantize_groups<1>(rest, gr);
            if (tid + i0 < n4) store_group8(gr[0], p.zp, i / 8, act_q, act_s, act_c);
        }
    } else if (IN == IN_ATTN) {
        // the chunks' softmax states and the new key's (score s_n = q·k_n/√D, total 1, sums v_n)
        // merged (flash decoding): M = max(s_n, m_c), L = e^(s_n − M) + Σ l_c·e^(m_c − M),
        // out = (v_n·e^(s_n − M) + Σ acc_c·e^(m_c − M)) / L; then the row quantized (8 lanes per
        // group of 32). The head's D / 4 lanes are aligned, so its dot product is a group sum.
        const v4f qk = g.qn * g.kn;
        float sn = (qk.x + qk.y) + (qk.z + qk.w);
        sn = sn + __int_as_float(xor1(__float_as_int(sn)));
        sn = sn + __int_as_float(xor2(__float_as_int(sn)));
        sn = sn + __int_as_float(mirror8(__float_as_int(sn)));
        if (p.D >= 64) sn = sn + xor8(sn);
        if (p.D >= 128) {
            const float2 r = row_pair(sn);
            sn = r.x + r.y;
        }
        sn = sn * (1.0f / sqrtf(float(p.D)));
        float M = sn;
#pragma unroll
        for (int c = 0; c < kMaxChunks; c++)
            if (c < p.chunks) M = fmaxf(M, g.pm[c]);
        const float en = ref_exp(sn - M);
        // e^(m_c − M) once per head and row of 16 lanes: lane c of the row (D >= 64: a head fills
        // whole rows) or of the head's D/4 = 8 lanes (D = 32) takes chunk c, and every lane of the
        // head reads them back in chunk order, by a row broadcast or a lane shuffle
        const int head0 = (tid & 63) & ~((p.D >> 2) - 1);
        const bool rows = p.D >= 64;
        const int slot = rows ? (tid & 15) : (tid & 63) - head0;
        float mine = 0.0f;
#pragma unroll
        for (int c = 0; c < kMaxChunks; c++)
            if (slot == c) mine = g.pm[c];
        const float e_mine = slot < p.chunks ? ref_exp(mine - M) : 0.0f;
        float L = en;
        v4f o = g.vn * en;
#pragma unroll
        for (int c = 0; c < kMaxChunks; c++) {
            const float e = rows ? row_broadcast(e_mine, c) : __shfl(e_mine, head0 + c, 64);
            if (c < p.chunks) {
                L = L + g.pl[c] * e;
                o = o + g.pa[c] * e;
            }
        }
        const float inv_L = 1.0f / L;
        const v4f merged[1] = {o * inv_L};
        if (p.merged_out && blockIdx.x == 0 && tid < K / 4) reinterpret_cast<v4f *>(p.merged_out)[tid] = merged[0];
        quantize_slots<1>(merged, K / 4, p.zp, act_q, act_s, act_c);
    } else {
        // rms_norm (ops.rs:7-16): mean of squares, 1/sqrt(mean + eps), x·inverse·weight; then the
        // quantization of the normed row. Thread t holds float4s t, t + 256, ... of the row, so
        // eight consecutive threads hold one group of 32.
        const int n4 = K / 4;
        v4f f[4] = {g.f0, g.f1, g.f2, g.f3};
        if (IN == IN_EMBED) {
            // Matrix::dequantize_row (tensor.rs:247-271): scale · (float)level; workgroup 0 keeps
            // the row for the residual
            const int cw[4] = {g.c0, g.c1, g.c2, g.c3};
            const float cs[4] = {g.s0, g.s1, g.s2, g.s3};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int i = tid + k * kThreads;
                const int lv = FMT == 8 ? cw[k] : nibbles_signed(cw[k] >> (((min(i, n4 - 1) & 7) >> 2) * 4));
                f[k] = v4f{cs[k] * float(int8_t(lv)), cs[k] * float(int8_t(lv >> 8)), cs[k] * float(int8_t(lv >> 16)),
                           cs[k] * float(int8_t(lv >> 24))};
                if (blockIdx.x == 0 && i < n4) reinterpret_cast<v4f *>(p.x_out)[i] = f[k];
            }
        }
        float total;
        if (EXACT) {
            // dot_f32(row, row) in index order from −0 (arch/scalar.rs:340-342): the squares are
            // formed by every thread, then one lane adds them with its reads running ahead (from
            // +0: the squares are never −0, so the start's sign changes nothing)
            v4f *sq = reinterpret_cast<v4f *>(nbuf);
            if (tid < n4) sq[tid] = f[0] * f[0];
            if (tid + kThreads < n4) sq[tid + kThreads] = f[1] * f[1];
            if (tid + 2 * kThreads < n4) sq[tid + 2 * kThreads] = f[2] * f[2];
            if (tid + 3 * kThreads < n4) sq[tid + 3 * kThreads] = f[3] * f[3];
            __syncthreads();
            if (tid == 0) red[4] = ordered_sum(nbuf, K);
            __syncthreads();
            total = red[4];
        } else {
            float part = 0.0f;
#define FG_SQ(v, k) \
    if (tid + (k) * kThreads < n4) part = part + (((v).x * (v).x + (v).y * (v).y) + ((v).z * (v).z + (v).w * (v).w));
            FG_SQ(f[0], 0)
            FG_SQ(f[1], 1)
            FG_SQ(f[2], 2)
            FG_SQ(f[3], 3)
#undef FG_SQ
            part = wave_allsum(part);
            if ((tid & 63) == 0) red[tid >> 6] = part;
            __syncthreads();
            total = ((red[0] + red[1]) + red[2]) + red[3];
        }
        const float inverse = 1.0f / sqrtf(total / float(K) + p.eps);
        const v4f normed[4] = {f[0] * inverse * g.w0, f[1] * inverse * g.w1, f[2] * inverse * g.w2, f[3] * inverse * g.w3};
        quantize_slots<4>(normed, n4, p.zp, act_q, act_s, act_c);
    }
}

// ---------------------------------------------------------------- the fast attention's chunks
//
// One query head over one chunk of the cached keys (flash decoding), 256 threads. Per tile of
// kTileKeys keys, wave w takes keys 16w .. 16w + 15: the scores q·k_j·(1/√D) (ops.rs:310-326;
// four lanes per key), the wave's running maximum m, e^(s_j − m) through ops::exp, the running
// total l and the running weighted sum of values (ops.rs:329-342), both rescaled by e^(m_old − m)
// when the maximum moves; every reduction within the wave (DPP and lane broadcasts). The four
// waves' states are merged once at the end into the chunk's record (m, l, −, −, acc[D]), which the
// output projection's prologue merges with the other chunks' and the new key's.

template <int D>
struct AttnShape {
    static constexpr int DQ = D / 4;                 // dims of a key per lane (scores)
    static constexpr int KPL = D >= 64 ? 16 : 8;     // keys per lane (weighted sum)
    static constexpr int VPL = D >= 64 ? D / 64 : 1; // dims per lane (weighted sum)
};

// A tile's keys and values as one thread holds them: for the scores, key 16w + (lane / 4), dims
// (lane % 4)·D/4 ..; for the weighted sum, dims lane·VPL .. of the wave's 16 keys (D = 32: dim
// lane % 32 of keys 16w + (lane / 32)·8 ..).
template <int D>
struct KVTile {
    v4f k[D >= 16 ? D / 16 : 1];
    float v[D >= 64 ? 16 * (D / 64) : 8];
};

template <int D>
__device__ __forceinline__ void value_slot(int lane, int wave, int &key0, int &dim0)
{
    if (D >= 64) {
        key0 = 16 * wave;
        dim0 = lane * AttnShape<D>::VPL;
    } else {
        key0 = 16 * wave + (lane >> 5) * 8;
        dim0 = lane & 31;
    }
}

// The tile of keys j0 .. j0 + n - 1 of KV head `kv` (branch-free: keys past n re-read key j0);
// KEYS: the keys alone (the exact scores).
template <int D, bool KEYS = false>
__device__ __forceinline__ void load_kv_tile(const ProjParams &p, int kv, int j0, int n, KVTile<D> &t)
{
    if (D == 0) return;
    using S = AttnShape<D>;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), jk = tid >> 2, part = tid & 3;
    const size_t row0 = p.layer_base + (size_t(kv) * p.capacity + size_t(j0)) * D;  // the tile's first key
    const float *kt = p.kcache + row0, *vt = p.vcache + row0;
    const unsigned koff = unsigned((jk < n ? jk : 0) * D + part * S::DQ);
#pragma unroll
    for (int i = 0; i < S::DQ / 4; i++) t.k[i] = *reinterpret_cast<const v4f *>(kt + (koff + 4u * i));
    if (KEYS) return;
    int key0, dim0;
    value_slot<D>(lane, wave, key0, dim0);
#pragma unroll
    for (int e = 0; e < S::KPL; e++) {
        const int j = key0 + e;
        const unsigned at = unsigned((j < n ? j : 0) * D + dim0);
        if (S::VPL == 2) {
            const float2 v2 = *reinterpret_cast<const float2 *>(vt + at);
            t.v[2 * e] = v2.x;
            t.v[2 * e + 1] = v2.y;
        } else {
            t.v[e] = vt[at];
        }
    }
}

// Chunk c of query head h: keys [c·per_chunk, min((c + 1)·per_chunk, position)); the first tile is
// already in `tile`. `scratch` holds 8 + 4·D floats of LDS.
template <int D>
__device__ __forceinline__ void attend_chunk(const ProjParams &p, const float *qrot, int h, int c, KVTile<D> &tile,
                                             float *scratch)
{
    if (D == 0) return;
    using S = AttnShape<D>;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), jk = tid >> 2, part = tid & 3;
    const int kv = divq(h, p.rcp_group);
    const int first = c * p.per_chunk, last = min(p.position, first + p.per_chunk);
    int key0, dim0;
    value_slot<D>(lane, wave, key0, dim0);
    v4f q[S::DQ / 4 > 0 ? S::DQ / 4 : 1];
#pragma unroll
    for (int i = 0; i < S::DQ / 4; i++) q[i] = *reinterpret_cast<const v4f *>(qrot + part * S::DQ + 4 * i);
    const float scale = 1.0f / sqrtf(float(D));
    float m = -INFINITY, l = 0.0f;
    float acc[S::VPL];
#pragma unroll
    for (int i = 0; i < S::VPL; i++) acc[i] = 0.0f;
    for (int j0 = first; j0 < last; j0 += kTileKeys) {
        const int n = min(kTileKeys, last - j0);
        if (j0 != first) load_kv_tile<D>(p, kv, j0, n, tile);
        v4f sv = q[0] * tile.k[0];
#pragma unroll
        for (int i = 1; i < S::DQ / 4; i++) sv = sv + q[i] * tile.k[i];
        float sc = (sv.x + sv.y) + (sv.z + sv.w);
        sc = sc + __int_as_float(xor1(__float_as_int(sc)));
        sc = sc + __int_as_float(xor2(__float_as_int(sc)));
        sc = jk < n ? sc * scale : -INFINITY;
        const float m_new = fmaxf(m, wave_allmax(sc));
        if (m_new == -INFINITY) continue;  // no key of this tile in this wave (uniform)
        const float r = m == -INFINITY ? 0.0f : ref_exp(m - m_new);
        const float pj = jk < n ? ref_exp(sc - m_new) : 0.0f;
        l = l * r + wave_allsum(part == 0 ? pj : 0.0f);
        m = m_new;
#pragma unroll
        for (int i = 0; i < S::VPL; i++) acc[i] = acc[i] * r;
#pragma unroll
        for (int e = 0; e < S::KPL; e++) {
            // key key0 + e's weight, from lane 4·(key0 + e − 16·wave) of this wave
            float w;
            if (D >= 64) w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pj), 4 * e));
            else w = __shfl(pj, 4 * (key0 + e - 16 * wave), 64);
#pragma unroll
            for (int i = 0; i < S::VPL; i++) acc[i] = acc[i] + w * tile.v[S::VPL * e + i];
        }
    }
    if (D < 64) {
        const float2 h = half_pair(acc[0]);  // the two halves' keys, same dims
        acc[0] = h.x + h.y;
    }
    // the waves' states merged: M = max m_w, L = Σ l_w·e^(m_w − M), acc = Σ acc_w·e^(m_w − M)
    float *wm = scratch, *wl = scratch + 4, *wacc = scratch + 8;  // [4], [4], [4][D]
    if (lane == 0) {
        wm[wave] = m;
        wl[wave] = l;
    }
    if (D >= 64 || lane < 32) {
#pragma unroll
        for (int i = 0; i < S::VPL; i++) wacc[wave * D + dim0 + i] = acc[i];
    }
    __syncthreads();
    float *rec = p.states + size_t(h * p.chunks + c) * (D + 4);
    if (tid < D) {
        const float M = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
        float L = 0.0f, o = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float e = wm[w] == -INFINITY ? 0.0f : ref_exp(wm[w] - M);
                L = L + wl[w] * e;
                o = o + wacc[w * D + tid] * e;
            }
        }
        rec[4 + tid] = o;
        if (tid == 0) {
            rec[0] = M;
            rec[1] = L;
        }
    }
}

// The exact order's scores of chunk c of query head h (ops.rs:310-326): for each key j in
// [c·per_chunk, min((c + 1)·per_chunk, position)), dot_f32(q, k_j) in index order from −0, times
// 1/√D, into scores[h][j]. The four lanes of a key hold a quarter of its dimensions each, in order:
// the quarters' products are added one quarter after another, each lane continuing the sum that
// the previous quarter's lane passes on. The first tile is already in `tile`.
template <int D>
__device__ __forceinline__ void score_chunk(const ProjParams &p, const float *qrot, int h, int c, KVTile<D> &tile)
{
    if (D == 0) return;
    using S = AttnShape<D>;
    const int tid = threadIdx.x, lane = tid & 63, jk = tid >> 2, part = tid & 3;
    const int kv = divq(h, p.rcp_group);
    const int first = c * p.per_chunk, last = min(p.position, first + p.per_chunk);
    v4f q[S::DQ / 4 > 0 ? S::DQ / 4 : 1];
#pragma unroll
    for (int i = 0; i < S::DQ / 4; i++) q[i] = *reinterpret_cast<const v4f *>(qrot + part * S::DQ + 4 * i);
    const float scale = 1.0f / sqrtf(float(D));
    float *out = p.scores + size_t(h) * p.capacity;
    for (int j0 = first; j0 < last; j0 += kTileKeys) {
        const int n = min(kTileKeys, last - j0);
        if (j0 != first) load_kv_tile<D, true>(p, kv, j0, n, tile);
        v4f prod[S::DQ / 4 > 0 ? S::DQ / 4 : 1];
#pragma unroll
        for (int i = 0; i < S::DQ / 4; i++) prod[i] = q[i] * tile.k[i];
        float s = -0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            // every lane continues from quarter t − 1's sum; quarter t's lane holds the real one
            float run = s;
#pragma unroll
            for (int i = 0; i < S::DQ / 4; i++) {
                run = run + prod[i].x;
                run = run + prod[i].y;
                run = run + prod[i].z;
                run = run + prod[i].w;
            }
            s = quad_broadcast(run, t);
        }
        if (part == 0 && jk < n) out[j0 + jk] = s * scale;
    }
}

// The (head, chunk) unit, head·chunks + chunk, of query workgroup w. Workgroups go to the eight
// XCDs in turn (w % 8), so consecutive units are spread over w = x, x + 8, ... of one XCD: the
// chunk workgroups of a head then share that XCD's L2 for the head's rows.
__device__ __forceinline__ int qattn_unit(const ProjParams &p, int w, int qwgs)
{
    return qwgs % 8 ? w : (w % 8) * (qwgs / 8) + w / 8;
}

// FMT: 8 for signed 8-bit levels (Q7b32 folded, Q8b32), 4 for offset nibbles (Q4b32).
// TREE: each output's group terms summed by a team of lanes and a lane reduction instead of in
// group order (the decoder's parallel-order mode; the product's own entry points never use it).
template <int FMT, int R, int IN, int OUT, bool EXACT, int kBatch, bool TREE, int HD>
__global__ __launch_bounds__(kThreads) void proj_kernel(ProjParams p)
{
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int NT = OUT == OUT_SWIGLU ? 2 : 1;  // tables streamed
    const int K = p.K, G = p.G, B = p.B;
    const int Gp = (G + 3) & ~3;  // terms per output, padded for 128-bit reads
    // OUT_QATTN: the query workgroups own their head's D/4 quads, the others a rotary pair of the
    // key and value rows (quads D/8 apart). Branch-free, so that the parameters' loads issue at once.
    const int w = int(blockIdx.x);
    const int qwgs = OUT == OUT_QATTN ? p.heads * p.chunks : 0;
    const bool query = OUT == OUT_QATTN && w < qwgs;
    int qs, base, nq;
    if (OUT == OUT_QATTN) {
        constexpr int hq = HD / 8;
        const int b = w - qwgs;
        qs = query ? 1 : hq;
        base = query ? divq(qattn_unit(p, w, qwgs), p.rcp_chunks) * (HD / 4) : p.heads * (HD / 4) + b / hq * hq * 2 + b % hq;
        nq = query ? HD / 4 : 2;
    } else {
        qs = p.qstride;
        base = p.quad_begin + ((w >> p.qshift) << p.qshift) * p.qpw + (w & (qs - 1));
        nq = min(p.qpw, (p.quad_end - base + qs - 1) >> p.qshift);
    }
    // The host's grids leave no workgroup without quads. No early exit (it would put a round trip
    // for the parameters ahead of every load): the clamp only keeps any access in bounds.
    nq = max(nq, 1);
    const int NW = p.qpw * 4;
    auto output_of = [&](int nl) { return (base + (nl >> 2) * qs) * 4 + (nl & 3); };  // local -> column
    const ProjLayout lay = proj_layout(R, K, G, NW, IN, OUT);
    int8_t *act_q = reinterpret_cast<int8_t *>(smem);
    float *act_s = reinterpret_cast<float *>(smem + lay.off_s);      // [R][G]
    int32_t *act_c = reinterpret_cast<int32_t *>(smem + lay.off_c);  // [R][G]
    float *red = reinterpret_cast<float *>(smem + lay.off_red);      // [16]
    float *ybuf = reinterpret_cast<float *>(smem + lay.off_y);       // [NT (+1)][R][NW]
    float *terms = reinterpret_cast<float *>(smem + lay.off_terms);  // [NT][R][NW][Gp]
    float *nbuf = reinterpret_cast<float *>(smem + lay.off_n);       // [K] (IN_NORM)

    // the wave index in a scalar register: what depends only on it (a wave's chunks, its batch
    // count, the slots it skips) becomes scalar work and branches rather than per-lane masks
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    constexpr int QB = FMT == 8 ? 128 : 64;         // device bytes per quad block
    constexpr int QB_PER_CHUNK = 1024 / QB;         // quad blocks per 1 KiB chunk
    const int total_qb = nq * B;
    const int per_table = (total_qb + QB_PER_CHUNK - 1) / QB_PER_CHUNK;  // chunks per table
    const int L = FMT == 8 ? (lane >> 1) & 3 : lane & 3;
    const int h = FMT == 8 ? lane & 1 : 0;
    const int qb_in_chunk = FMT == 8 ? lane >> 3 : lane >> 2;
    const int piece = FMT == 8 ? lane & 7 : lane & 3;  // this lane's 16 bytes of its quad block
    // Chunk k of a wave is chunk wt + k·stride of table tb: with two tables, waves 0 and 2 stream
    // the gate, 1 and 3 the up table.
    constexpr int stride = 4 / NT;
    const int tb = NT == 2 ? (wave & 1) : 0;
    const int wt = NT == 2 ? (wave >> 1) : wave;
    const int mine = per_table > wt ? (per_table - wt + stride - 1) / stride : 0;  // chunks of this wave
    const int batches = (mine + kBatch - 1) / kBatch;
    const int8_t *codes = tb ? p.codes2 : p.codes;
    const float *wsc = tb ? p.wscales2 : p.wscales;
    // The lane's quad block (local quad ql, block blk) walks by `stride` chunks at a time: one
    // division up front, then a quotient and a remainder step.
    const int qb0 = wt * QB_PER_CHUNK + qb_in_chunk;
    const int step_q = stride * QB_PER_CHUNK / B, step_r = stride * QB_PER_CHUNK - step_q * B;
    // ti: the lane's term slot (ql·4 + L)·Gp + blk in the first table's first row, kept in step
    struct Cursor {
        int ql, blk, ti;
    };
    const int step_t = step_q * 4 * Gp + step_r, wrap_t = 4 * Gp - B;
    auto advance = [&](Cursor &cu) {
        cu.ql += step_q;
        cu.blk += step_r;
        cu.ti += step_t;
        if (cu.blk >= B) {
            cu.blk -= B;
            cu.ql++;
            cu.ti += wrap_t;
        }
    };
    const int ql0 = divq(qb0, p.rcp_B);
    Cursor ccur{ql0, qb0 - ql0 * B, (ql0 * 4 + L) * Gp + (qb0 - ql0 * B)};
    // the term slot of a quad block past the run's end (its store lands there, never read)
    const int spare = NT * R * NW * Gp;

    // The workgroup's quad blocks, numbered ql·B + blk, sit contiguously from its first quad, but
    // for a strided pair (qs > 1, two quads) whose second half starts (qs − 1)·B blocks later.
    // Lanes address them as 32-bit offsets from the workgroup's base (the loads' scalar-base form),
    // a few instructions per chunk. Branch-free: past the run's end every lane reloads the last
    // block (always in bounds), so a batch issues back to back with a single wait when consumed;
    // `consume` skips what was not valid.
    const int8_t *wq = codes + size_t(base) * B * QB;
    const float *sq = wsc + size_t(base) * G * 4;
    const unsigned skip = unsigned(qs - 1) * unsigned(B), last_qb = unsigned(nq * B - 1);
    unsigned lqb = unsigned(qb0);
    // The query-head workgroups' 16-chunk batch issues in two halves, the second after the
    // prologue: a wave issues its loads one after another and the prologue's wait for the row
    // sits behind all of them (decode 588 -> 580 us per token)
    constexpr bool kSplit = OUT == OUT_QATTN && kBatch == 16;
    auto load = [&](int4 *w, float *ws, int part = -1) {
#pragma unroll
        for (int u = 0; u < kBatch; u++) {
            if (part == 0 && u >= kBatch / 2) break;
            if (part == 1 && u < kBatch / 2) continue;
            const unsigned qb = min(lqb, last_qb);
            const unsigned at = qb + (qb >= unsigned(B) ? skip : 0u);
            w[u] = *reinterpret_cast<const int4 *>(wq + (at * QB + unsigned(piece) * 16u));
            ws[u] = sq[at * 4u + unsigned(L)];
            lqb += unsigned(stride * QB_PER_CHUNK);
        }
    };

    // A batch is consumed U chunks at a time: the chunks' activation reads from LDS first, then
    // their dots and term stores. LDS reads are not moved above possibly aliasing LDS stores, so
    // reading per chunk would serialize two LDS round trips per chunk.
    constexpr int U = R == 1 ? (FMT == 8 ? (kBatch < 8 ? kBatch : 8) : (kBatch < 8 ? (kBatch + 1) / 2 : 4))
                             : (R == 2 ? (kBatch < 4 ? kBatch : 4) : (kBatch < 2 ? kBatch : 2));
    auto consume = [&](int b, const int4 *w, const float *ws) {
#pragma unroll
        for (int u0 = 0; u0 < kBatch; u0 += U) {
            int qls[U], blks[U], tis[U];
            int4 a0[U][R], a1[U][R];
            float asc[U][R];
            int acr[U][R];
#pragma unroll
            for (int v = 0; v < U; v++) {
                qls[v] = ccur.ql;
                blks[v] = ccur.blk;
                tis[v] = ccur.ti;
                advance(ccur);
                const int blk = blks[v];  // < B always: every read is in bounds
#pragma unroll
                for (int r = 0; r < R; r++) {
                    if (FMT == 8) {
                        a0[v][r] = *reinterpret_cast<const int4 *>(act_q + r * K + blk * 32 + h * 16);
                    } else {
                        a0[v][r] = *reinterpret_cast<const int4 *>(act_q + r * K + blk * 32);
                        a1[v][r] = *reinterpret_cast<const int4 *>(act_q + r * K + blk * 32 + 16);
                        acr[v][r] = act_c[r * G + blk];
                    }
                    if (OUT != OUT_DOTS) asc[v][r] = act_s[r * G + blk];
                }
            }
#pragma unroll
            for (int v = 0; v < U; v++) {
                const int u = u0 + v;
                if (b * kBatch + u >= mine) continue;  // uniform across the wave
                const int ql = qls[v], blk = blks[v];
                const bool valid = ql < nq;
#pragma unroll
                for (int r = 0; r < R; r++) {
                    int D;
                    if (FMT == 8) {
                        D = dot16(w[u], a0[v][r]);
                        D += xor1(D);  // the row-block's other half
                    } else {
                        const int4 lo = make_int4(w[u].x & 0x0F0F0F0F, w[u].y & 0x0F0F0F0F, w[u].z & 0x0F0F0F0F, w[u].w & 0x0F0F0F0F);
                        const int4 hi = make_int4((w[u].x >> 4) & 0x0F0F0F0F, (w[u].y >> 4) & 0x0F0F0F0F,
                                                  (w[u].z >> 4) & 0x0F0F0F0F, (w[u].w >> 4) & 0x0F0F0F0F);
                        D = dot16(lo, a0[v][r]) + dot16(hi, a1[v][r]) + acr[v][r];
                    }
                    if (OUT == OUT_DOTS) {
                        if (valid && h == 0) {
                            const int n = (base + ql * qs) * 4 + L;
                            p.dots[(size_t(r) * p.dots_cols + (n - p.col_begin)) * G + blk] = D;
                        }
                    } else {
                        // both lanes of a pair hold the same total and scale, so both store the
                        // same term; a block past the run's end stores to the spare slot
                        const float scale = ws[u] * asc[v][r];
                        terms[valid ? tis[v] + (tb * R + r) * NW * Gp : spare] = float(D) * scale;
                    }
                }
            }
        }
    };

    // Batches of up to 8 chunks are double-buffered (the next batch in flight while one is
    // consumed); a deeper batch, sized to cover a wave's whole share, has a single buffer.
    constexpr bool kDouble = kBatch <= 8;
    constexpr int kSecond = kDouble ? kBatch : 1;
    int4 wa[kBatch], wb[kSecond];
    float sa[kBatch], sb[kSecond];
    StageRegs g;
    stage_issue<FMT, R, IN>(p, g);
    // Who sums which output: one thread per output, or (TREE) a team of `team` lanes per output.
    const int outs = NT * R * NW;
    // the largest power of two (at most 64) with outs·team <= 256: no loop ahead of the loads
    // and no more lanes than the output's float4 runs of terms (the rest would add zeros)
    const int runs4 = Gp / 4;
    const int team = TREE ? min(min(64, int(0x80000000u >> __builtin_clz(unsigned(max(1, kThreads / outs))))),
                                runs4 <= 1 ? 1 : int(2u << (31 - __builtin_clz(unsigned(runs4 - 1)))))
                          : 1;
    const int my_out = TREE ? int(threadIdx.x) >> __builtin_ctz(unsigned(team)) : int(threadIdx.x);
    const int sub = int(threadIdx.x) - my_out * team;
    // the residual row this workgroup adds to, read early (linear.rs:139-142); read whether or not
    // it is added, so that no branch splits the loads before the weights' first batch
    float resid = 0.0f, bias0 = 0.0f;
    if (OUT != OUT_SWIGLU && OUT != OUT_DOTS) {
        const int r = R == 1 ? 0 : my_out / NW, nl = my_out - r * NW;
        const bool mine = r < R && nl < nq * 4;
        const int n = output_of(nl);
        // 32-bit offsets, selected rather than branched on, so no branch splits the loads
        const unsigned at = unsigned(r) * unsigned(p.ld_out) + unsigned(n - p.col_begin);
        if (OUT == OUT_STORE) resid = p.out[mine ? at : 0u];
        // and the bias of that output (a table without bias reads its own scales instead, unused)
        bias0 = (p.bias ? p.bias : p.wscales)[mine ? unsigned(min(n, p.n_rows - 1)) : 0u];
    }
    // keep the activation loads ahead of the weights': loads return in order, and the prologue
    // waits only for the activations
    __builtin_amdgcn_sched_barrier(0);
    load(wa, sa, kSplit ? 0 : -1);  // every wave, in bounds even without chunks of its own
    __builtin_amdgcn_sched_barrier(0);  // and all of them issued before the prologue's first wait
    stage_finish<FMT, R, IN, EXACT>(p, g, act_q, act_s, act_c, nbuf, red);
    if (!TREE && OUT != OUT_DOTS && Gp != G) {
        // term rows zero-padded to whole float4s (the ordered sum reads them whole)
        for (int i = threadIdx.x; i < NT * R * NW; i += kThreads)
            for (int g2 = G; g2 < Gp; g2++) terms[i * Gp + g2] = 0.0f;
    }
    __syncthreads();
    // OUT_QATTN: the first tile of the chunk's cached keys and values, issued once the prologue
    // is done (a wave issues its loads one after another, and the prologue waits behind every
    // load issued before it) and behind the weights, so it arrives while the query rows are
    // computed. Every workgroup loads one, in bounds, so that no branch splits the loads.
    if constexpr (kSplit) {
        load(wa, sa, 1);
        __builtin_amdgcn_sched_barrier(0);
    }
    KVTile<HD> tile;
    int head = 0, chunk = 0;
    if (OUT == OUT_QATTN) {
        const int unit = query ? qattn_unit(p, int(blockIdx.x), qwgs) : 0;
        head = divq(unit, p.rcp_chunks);
        chunk = unit - head * p.chunks;
        const int first = chunk * p.per_chunk;
        load_kv_tile<HD, EXACT>(p, divq(head, p.rcp_group), first,
                                max(0, min(kTileKeys, min(p.position, first + p.per_chunk) - first)), tile);
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (kDouble) {
        for (int b = 0; b < batches; b += 2) {
            if (b + 1 < batches) load(wb, sb);
            consume(b, wa, sa);
            if (b + 1 < batches) {
                if (b + 2 < batches) load(wa, sa);
                consume(b + 1, wb, sb);
            }
        }
    } else {
        for (int b = 0; b < batches; b++) {
            if (b > 0) load(wa, sa);
            consume(b, wa, sa);
        }
    }
    if (OUT == OUT_DOTS) return;
    __syncthreads();

    // Output i of (table, row, column): bias, then stored (written or added to the residual row).
    auto finish = [&](int i, float s) {
        const int tb = NT == 1 ? 0 : i / (R * NW), rem = i - tb * R * NW;  // no division where fixed
        const int r = R == 1 ? 0 : rem / NW, nl = rem - r * NW;
        const int n = output_of(nl);
        if (OUT != OUT_SWIGLU && p.bias && n < p.n_rows) s = s + (i == my_out ? bias0 : p.bias[n]);
        if (OUT == OUT_STORE) {
            float *o = p.out + r * p.ld_out + (n - p.col_begin);
            float prior = resid;
            if (p.accumulate && i >= kThreads) prior = *o;  // rows past the prefetched ones
            *o = p.accumulate ? prior + s : s;
        }
        ybuf[i] = s;
    };
    auto live = [&](int i) { return i < outs && (NT * R == 1 ? i : i % NW) < nq * 4; };
    if (TREE) {
        // strided partial sums, then the team's lanes reduced (lanes of one wave)
        float s = 0.0f;
        if (live(my_out)) {
            // [tb][r][nl] rows in output order, 16-byte aligned: four terms per read
            const v4f *t4 = reinterpret_cast<const v4f *>(terms + my_out * Gp);
            for (int k = sub; 4 * k < G; k += team) {
                const v4f v = t4[k];
                const int g = 4 * k;
                s = s + ((v.x + (g + 1 < G ? v.y : 0.0f)) + ((g + 2 < G ? v.z : 0.0f) + (g + 3 < G ? v.w : 0.0f)));
            }
        }
        if (team >= 2) s = s + __int_as_float(xor1(__float_as_int(s)));
        if (team >= 4) s = s + __int_as_float(xor2(__float_as_int(s)));
        if (team >= 8) s = s + __int_as_float(mirror8(__float_as_int(s)));
        if (team >= 16) s = s + xor8(s);
        if (team >= 32) {
            const float2 r = row_pair(s);
            s = r.x + r.y;
        }
        if (team >= 64) {
            const float2 h = half_pair(s);
            s = h.x + h.y;
        }
        if (sub == 0 && live(my_out)) finish(my_out, s);
    } else {
        // group order: the reference's sequential sum, one thread per (table, row, output)
        for (int i = threadIdx.x; i < outs; i += kThreads)
            if (live(i)) finish(i, ordered_sum(terms + i * Gp, G));
    }

    if (OUT == OUT_STORE) {
        if (p.pval) {
            // this workgroup's greedy candidate (lm.rs:169-179): the first largest, NaN never wins.
            // Its outputs (at most 64, checked on the host) are one per lane of the first wave in
            // column order: the wave's maximum (NaN ignored), then the first lane holding it.
            __syncthreads();
            if (wave == 0) {
                float v = __builtin_nanf("");
                if (lane < nq * 4 && output_of(lane) < p.n_rows) v = ybuf[lane];
                const float best = wave_allmax(v);
                const unsigned long long hit = __ballot(v == best);
                const int first = hit ? __ffsll((long long)hit) - 1 : 0;
                if (lane == first) {
                    p.pval[blockIdx.x] = hit ? v : 0.0f;
                    p.pidx[blockIdx.x] = hit ? output_of(lane) : -1;
                }
            }
        }
        return;
    }
    __syncthreads();
    if (OUT == OUT_QATTN && query) {
        // the query head: rotated by halves (rope_half, ops.rs:77-85), kept for the output
        // projection's new-key term by the chunk-0 workgroup, then attended over the chunk
        float *qrot = reinterpret_cast<float *>(smem + lay.off_att);
        constexpr int half = HD / 2;
        if (threadIdx.x < half) {
            const int j = int(threadIdx.x);
            const float x = ybuf[j] , y = ybuf[half + j];
            const float c = p.rope[j], sn = p.rope[half + j];
            const float nx = x * c - y * sn, ny = y * c + x * sn;
            qrot[j] = nx;
            qrot[j + half] = ny;
            if (chunk == 0) {
                p.qkv_out[head * HD + j] = nx;
                p.qkv_out[head * HD + j + half] = ny;
            }
        }
        __syncthreads();
        if (EXACT) score_chunk<HD>(p, qrot, head, chunk, tile);
        else attend_chunk<HD>(p, qrot, head, chunk, tile, qrot + HD);
    } else if (OUT == OUT_QKV || OUT == OUT_QATTN) {
        // a rotary pair per workgroup (qstride = D/8, qpw = 2): outputs 0..3 are dimensions
        // j0..j0+3 of a head, outputs 4..7 the same dimensions + D/2. The bias is in; query and key
        // heads rotate by halves, key and value heads go to the cache.
        const int D = p.D, half = D / 2;
        const int unit = base * 4 / D, j0 = base * 4 - unit * D;
        if (threadIdx.x < 4) {
            const int j = j0 + int(threadIdx.x);
            float x = ybuf[threadIdx.x], y = ybuf[4 + threadIdx.x];
            if (unit < p.heads + p.kv_heads) {
                const float c = p.rope[j], sn = p.rope[half + j];
                const float nx = x * c - y * sn;
                const float ny = y * c + x * sn;
                x = nx;
                y = ny;
            }
            p.qkv_out[unit * D + j] = x;
            p.qkv_out[unit * D + j + half] = y;
            if (unit >= p.heads) {
                const bool key = unit < p.heads + p.kv_heads;
                const int kv = (unit - p.heads) % p.kv_heads;
                float *cache = key ? p.kcache : p.vcache;
                const size_t at = p.layer_base + (size_t(kv) * p.capacity + size_t(p.position % p.capacity)) * D;
                cache[at + j] = x;
                cache[at + j + half] = y;
            }
        }
    } else if (OUT == OUT_SWIGLU) {
        // silu(gate)·up (layer.rs:321-341); the down projection quantizes the row
        for (int nl = threadIdx.x; nl < nq * 4; nl += kThreads) {
            const float y = ref_silu(ybuf[nl]) * ybuf[NW + nl];
            if (p.act_out) p.act_out[output_of(nl)] = y;
            ybuf[nl] = y;  // in place of the gate: slot nl is this thread's alone
        }
        if (p.q_out && wave == 0) {
            // the workgroup's 32 outputs are one group (written above by lanes 0..31 of this
            // wave): lanes 0..7 take four consecutive products each and quantize them as the
            // next projection's prologue would (the other lanes' groups are not stored)
            const v4f v[1] = {*reinterpret_cast<const v4f *>(ybuf + 4 * (lane & 7))};
            Group8 gr[1];
            quantize_groups<1>(v, gr);
            if (lane < 8) store_group8(gr[0], p.zp, output_of(0) / 32, p.q_out, p.s_out, p.c_out);
        }
    }
}

template <int FMT, int R, int IN, int OUT, bool EXACT, int NB = 8, bool TREE = false, int HD = 0>
int launch_one(const ProjParams &p, size_t smem, unsigned grid, hipStream_t s)
{
    auto kernel = proj_kernel<FMT, R, IN, OUT, EXACT, NB, TREE, HD>;
    // past 64 KiB of LDS the kernel's limit is raised on the current device, every time (a host
    // call with no stream work: no per-device state to keep, safe from concurrent callers)
    if (smem > 64 * 1024)
        FG_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                   160 * 1024));
    kernel<<<grid, kThreads, smem, s>>>(p);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

}  // namespace
}  // namespace fg
