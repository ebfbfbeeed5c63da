// The decode product: a few activation rows (1..4) against a quantized table, HBM-bound, with the
// decoder's neighbours fused in.
//
// Reference: matmul (matmul.rs:265-317) -> quant_tiles / quant_tile / quad_pass / accumulate
// (matmul.rs:521-763) with the scalar backend's arithmetic (arch/scalar.rs:68-90). Per output
// column n and activation row r:  D_g = corr_g + Σ_k u[n,k]·a[r,k]  (int32, exact in any order),
//   s = +0;  for g in order:  s = fl(s + fl(fl((float)D_g) · fl(ws[n,g] · as[r,g])))
// then the bias (linear.rs:63-68) and, for residual projections, h = fl(h + y) (linear.rs:134-143).
//
// Mapping. A workgroup owns `qpw` consecutive quads (4 output rows each) and all of their blocks:
// a contiguous run of the table (two runs for the gated feed-forward's gate and up tables). Its
// four waves stream the run in 1 KiB chunks (64 lanes x 16 B, fully coalesced 128-bit loads),
// `kBatch` chunks per wave in flight, the next batch issued before the current one is consumed.
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
// (silu(gate)·up quantized per group of 32 for the down projection, layer.rs:321-341).
#include "common.h"
#include "proj.h"

namespace fg {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ int dot16(int4 w, int4 a) { return dot4(w.w, a.w, dot4(w.z, a.z, dot4(w.y, a.y, dot4(w.x, a.x, 0)))); }

// Quantize `n` LDS floats (a multiple of 32) into levels / scales / corrections, 8 lanes per group
// (quantize_rows, matmul.rs:233-257). Every thread of the block calls it.
__device__ void quantize_lds_to(const float *v, int n, int zp, int8_t *q, float *scales, int32_t *corr)
{
    const int sub = threadIdx.x & 7;
    const int groups = n / 32;
    const int per_round = kThreads / 8;
    for (int g0 = 0; g0 < groups; g0 += per_round) {
        const int g = g0 + int(threadIdx.x >> 3);
        const bool active = g < groups;
        float x0 = 0, x1 = 0, x2 = 0, x3 = 0;
        if (active) {
            const float4 f = *reinterpret_cast<const float4 *>(v + g * 32 + sub * 4);
            x0 = f.x, x1 = f.y, x2 = f.z, x3 = f.w;
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
            reinterpret_cast<int *>(q)[g * 8 + sub] = pack4(l0, l1, l2, l3);
            if (sub == 0) {
                scales[g] = d;
                corr[g] = -zp * sum;
            }
        }
    }
}

// Σ t[g·stride] for g in 0..n, added in index order from +0; loads issued 16 at a time so that
// the dependent additions do not wait on each load.
__device__ __forceinline__ float ordered_sum(const float *t, int n, int stride)
{
    float s = 0.0f;
    int g = 0;
    for (; g + 16 <= n; g += 16) {
        float v[16];
#pragma unroll
        for (int k = 0; k < 16; k++) v[k] = t[(g + k) * stride];
#pragma unroll
        for (int k = 0; k < 16; k++) s = s + v[k];
    }
    for (; g < n; g++) s = s + t[g * stride];
    return s;
}

__device__ float block_sum256(float v, float *red)
{
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return ((red[0] + red[1]) + red[2]) + red[3];
}

// The activations' global loads, issued before the first weight batch: vector loads complete in
// order, so loads issued after the weights would wait for them.
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

struct StageRegs {
    v4i v0, v1, v2, v3;
    float s0, s1, s2, s3;
    int c0, c1, c2, c3;
    v4f f0, f1, f2, f3;
    float x[8], w[8];
};


template <int R, int IN>
__device__ __forceinline__ void stage_issue(const ProjParams &p, StageRegs &g)
{
    const int tid = threadIdx.x;
    const int K = p.K, G = p.G;
    if (IN == IN_PREQ) {
        const v4i *src = reinterpret_cast<const v4i *>(p.q);
        const int n16 = R * K / 16, ng = R * G;
        g.v0 = src[min(tid, n16 - 1)];
        g.v1 = src[min(tid + kThreads, n16 - 1)];
        g.v2 = src[min(tid + 2 * kThreads, n16 - 1)];
        g.v3 = src[min(tid + 3 * kThreads, n16 - 1)];
        g.s0 = p.as[min(tid, ng - 1)];
        g.s1 = p.as[min(tid + kThreads, ng - 1)];
        g.s2 = p.as[min(tid + 2 * kThreads, ng - 1)];
        g.s3 = p.as[min(tid + 3 * kThreads, ng - 1)];
        g.c0 = p.corr[min(tid, ng - 1)];
        g.c1 = p.corr[min(tid + kThreads, ng - 1)];
        g.c2 = p.corr[min(tid + 2 * kThreads, ng - 1)];
        g.c3 = p.corr[min(tid + 3 * kThreads, ng - 1)];
    } else if (IN == IN_F32) {
        const v4f *x4 = reinterpret_cast<const v4f *>(p.x);
        const int n4 = R * K / 4;
        g.f0 = x4[min(tid, n4 - 1)];
        g.f1 = x4[min(tid + kThreads, n4 - 1)];
        g.f2 = x4[min(tid + 2 * kThreads, n4 - 1)];
        g.f3 = x4[min(tid + 3 * kThreads, n4 - 1)];
    } else {
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int i = min(tid + k * kThreads, K - 1);
            g.x[k] = p.x[i];
            g.w[k] = p.norm_w[i];
        }
    }
}

// Quantize one group of 32 held by 8 lanes (four values each) at `grp` of the staged rows.
__device__ __forceinline__ void quantize8(v4f v, int zp, int grp, int8_t *q, float *scales, int32_t *corr)
{
    const int sub = threadIdx.x & 7;
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(0.0f, amax);
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
    const float d = group_scale(amax, 127.0f);
    const int l0 = quantize_level(v.x, d), l1 = quantize_level(v.y, d), l2 = quantize_level(v.z, d), l3 = quantize_level(v.w, d);
    int sum = l0 + l1 + l2 + l3;
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    sum += __shfl_xor(sum, 4, 64);
    reinterpret_cast<int *>(q)[grp * 8 + sub] = pack4(l0, l1, l2, l3);
    if (sub == 0) {
        scales[grp] = d;
        corr[grp] = -zp * sum;
    }
}

template <int R, int IN, bool EXACT>
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
        // 8 lanes per group of 32 (quantize_rows): thread t holds float4 t of the rows; every lane
        // of an 8-lane group is active together (the float4 count is a multiple of 8)
        const int n4 = R * K / 4;
        if (tid < n4) quantize8(g.f0, p.zp, tid / 8, act_q, act_s, act_c);
        if (tid + kThreads < n4) quantize8(g.f1, p.zp, (tid + kThreads) / 8, act_q, act_s, act_c);
        if (tid + 2 * kThreads < n4) quantize8(g.f2, p.zp, (tid + 2 * kThreads) / 8, act_q, act_s, act_c);
        if (tid + 3 * kThreads < n4) quantize8(g.f3, p.zp, (tid + 3 * kThreads) / 8, act_q, act_s, act_c);
        for (int i = tid + 4 * kThreads; i < n4; i += kThreads)
            quantize8(reinterpret_cast<const v4f *>(p.x)[i], p.zp, i / 8, act_q, act_s, act_c);
    } else {
        // rms_norm (ops.rs:7-16): mean of squares, 1/sqrt(mean + eps), x·inverse·weight; then the
        // quantization of the normed row
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int i = tid + k * kThreads;
            if (i < K) nbuf[i] = g.x[k];
        }
        for (int i = tid + 8 * kThreads; i < K; i += kThreads) nbuf[i] = p.x[i];
        __syncthreads();
        float total;
        if (EXACT) {
            if (tid == 0) {
                float s = -0.0f;  // dot_f32(row, row) in index order (arch/scalar.rs:340-342)
                for (int i = 0; i < K; i += 32) {
                    float4 f[8];
#pragma unroll
                    for (int k = 0; k < 8; k++) f[k] = *reinterpret_cast<const float4 *>(nbuf + i + 4 * k);
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        s = s + f[k].x * f[k].x;
                        s = s + f[k].y * f[k].y;
                        s = s + f[k].z * f[k].z;
                        s = s + f[k].w * f[k].w;
                    }
                }
                red[4] = s;
            }
            __syncthreads();
            total = red[4];
        } else {
            float part = 0.0f;
            for (int i = tid; i < K; i += kThreads) part = part + nbuf[i] * nbuf[i];
            total = block_sum256(part, red);
        }
        const float inverse = 1.0f / sqrtf(total / float(K) + p.eps);
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int i = tid + k * kThreads;
            if (i < K) nbuf[i] = nbuf[i] * inverse * g.w[k];
        }
        for (int i = tid + 8 * kThreads; i < K; i += kThreads) nbuf[i] = nbuf[i] * inverse * p.norm_w[i];
        __syncthreads();
        quantize_lds_to(nbuf, K, p.zp, act_q, act_s, act_c);
    }
}

// FMT: 8 for signed 8-bit levels (Q7b32 folded, Q8b32), 4 for offset nibbles (Q4b32).
template <int FMT, int R, int IN, int OUT, bool EXACT, int kBatch>
__global__ __launch_bounds__(kThreads) void proj_kernel(ProjParams p)
{
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int NT = OUT == OUT_SWIGLU ? 2 : 1;  // tables streamed
    const int K = p.K, G = p.G, B = p.B;
    const int qa = p.quad_begin + int(blockIdx.x) * p.qpw;
    const int nq = min(p.qpw, p.quad_end - qa);
    const int NW = p.qpw * 4;
    const ProjLayout lay = proj_layout(R, K, G, NW, IN, OUT);
    int8_t *act_q = reinterpret_cast<int8_t *>(smem);
    float *act_s = reinterpret_cast<float *>(smem + lay.off_s);      // [R][G]
    int32_t *act_c = reinterpret_cast<int32_t *>(smem + lay.off_c);  // [R][G]
    float *red = reinterpret_cast<float *>(smem + lay.off_red);      // [16]
    float *ybuf = reinterpret_cast<float *>(smem + lay.off_y);       // [NT (+1)][R][NW]
    float *terms = reinterpret_cast<float *>(smem + lay.off_terms);  // [NT][R][G][NW]
    float *nbuf = reinterpret_cast<float *>(smem + lay.off_n);       // [K] (IN_NORM)

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int QB = FMT == 8 ? 128 : 64;         // device bytes per quad block
    constexpr int QB_PER_CHUNK = 1024 / QB;         // quad blocks per 1 KiB chunk
    const int total_qb = nq * B;
    const int per_table = (total_qb + QB_PER_CHUNK - 1) / QB_PER_CHUNK;
    const int chunks = NT * per_table;
    const int L = FMT == 8 ? (lane >> 1) & 3 : lane & 3;
    const int h = FMT == 8 ? lane & 1 : 0;
    const int qb_in_chunk = FMT == 8 ? lane >> 3 : lane >> 2;
    const int mine = chunks > wave ? (chunks - wave + 3) / 4 : 0;  // chunks of this wave
    const int batches = (mine + kBatch - 1) / kBatch;

    // Branch-free: every lane loads, from its own address when its chunk exists and from the
    // run's first bytes otherwise (always in bounds), so the loads of a batch issue back to back
    // with a single wait when consumed; `consume` skips what was not valid.
    auto load = [&](int b, int4 *w, float *ws) {
#pragma unroll
        for (int u = 0; u < kBatch; u++) {
            const int c = wave + 4 * (b * kBatch + u);
            const int tb = NT == 2 ? (c >= per_table) : 0;
            const int cc = c - tb * per_table;
            const int qb = cc * QB_PER_CHUNK + qb_in_chunk;
            const bool ok = c < chunks && qb < total_qb;
            const int8_t *codes = tb ? p.codes2 : p.codes;
            const float *wsc = tb ? p.wscales2 : p.wscales;
            const int ql = qb / B, blk = qb - ql * B;
            const size_t coff = ok ? size_t(qa) * B * QB + size_t(cc) * 1024 + lane * 16 : size_t(qa) * B * QB;
            const size_t soff = ok ? (size_t(qa + ql) * G + blk) * 4 + L : size_t(qa) * G * 4;
            w[u] = *reinterpret_cast<const int4 *>(codes + coff);
            ws[u] = wsc[soff];
        }
    };

    auto consume = [&](int b, const int4 *w, const float *ws) {
#pragma unroll
        for (int u = 0; u < kBatch; u++) {
            const int c = wave + 4 * (b * kBatch + u);
            if (c >= chunks) continue;  // uniform across the wave
            const int tb = NT == 2 ? (c >= per_table) : 0;
            const int cc = c - tb * per_table;
            const int qb = cc * QB_PER_CHUNK + qb_in_chunk;
            const bool valid = qb < total_qb;
            const int ql = valid ? qb / B : 0, blk = valid ? qb - ql * B : 0;
#pragma unroll
            for (int r = 0; r < R; r++) {
                int D;
                if (FMT == 8) {
                    const int4 a = *reinterpret_cast<const int4 *>(act_q + r * K + blk * 32 + h * 16);
                    D = dot16(w[u], a);
                    D += xor1(D);  // the row-block's other half
                } else {
                    const int4 a0 = *reinterpret_cast<const int4 *>(act_q + r * K + blk * 32);
                    const int4 a1 = *reinterpret_cast<const int4 *>(act_q + r * K + blk * 32 + 16);
                    const int4 lo = make_int4(w[u].x & 0x0F0F0F0F, w[u].y & 0x0F0F0F0F, w[u].z & 0x0F0F0F0F, w[u].w & 0x0F0F0F0F);
                    const int4 hi = make_int4((w[u].x >> 4) & 0x0F0F0F0F, (w[u].y >> 4) & 0x0F0F0F0F,
                                              (w[u].z >> 4) & 0x0F0F0F0F, (w[u].w >> 4) & 0x0F0F0F0F);
                    D = dot16(lo, a0) + dot16(hi, a1) + act_c[r * G + blk];
                }
                if (valid && h == 0) {
                    if (OUT == OUT_DOTS) {
                        const int n = (qa + ql) * 4 + L;
                        p.dots[(size_t(r) * p.dots_cols + (n - p.col_begin)) * G + blk] = D;
                    } else {
                        const float scale = ws[u] * act_s[r * G + blk];
                        terms[((tb * R + r) * G + blk) * NW + ql * 4 + L] = float(D) * scale;
                    }
                }
            }
        }
    };

    int4 wa[kBatch], wb[kBatch];
    float sa[kBatch], sb[kBatch];
    StageRegs g;
    stage_issue<R, IN>(p, g);
    // the residual row this workgroup adds to, read early (linear.rs:139-142)
    float resid = 0.0f;
    if (OUT == OUT_STORE && p.accumulate) {
        const int r = int(threadIdx.x) / NW, nl = int(threadIdx.x) - r * NW;
        const bool mine = r < R && nl < nq * 4;
        resid = p.out[mine ? r * p.ld_out + (qa * 4 + nl - p.col_begin) : 0];
    }
    if (batches > 0) load(0, wa, sa);
    stage_finish<R, IN, EXACT>(p, g, act_q, act_s, act_c, nbuf, red);
    __syncthreads();
    for (int b = 0; b < batches; b += 2) {
        if (b + 1 < batches) load(b + 1, wb, sb);
        consume(b, wa, sa);
        if (b + 1 < batches) {
            if (b + 2 < batches) load(b + 2, wa, sa);
            consume(b + 1, wb, sb);
        }
    }
    if (OUT == OUT_DOTS) return;
    __syncthreads();

    // Group order: the reference's sequential sum, one thread per (table, row, output).
    for (int i = threadIdx.x; i < NT * R * NW; i += kThreads) {
        const int tb = i / (R * NW), rem = i - tb * R * NW;
        const int r = rem / NW, nl = rem - r * NW;
        if (nl >= nq * 4) continue;
        const float *t = terms + (tb * R + r) * G * NW + nl;
        float s = ordered_sum(t, G, NW);
        const int n = qa * 4 + nl;
        if (OUT != OUT_SWIGLU && p.bias && n < p.n_rows) s = s + p.bias[n];
        if (OUT == OUT_STORE) {
            float *o = p.out + r * p.ld_out + (n - p.col_begin);
            float prior = resid;
            if (p.accumulate && i >= kThreads) prior = *o;  // rows past the prefetched ones
            *o = p.accumulate ? prior + s : s;
        }
        ybuf[i] = s;
    }

    if (OUT == OUT_STORE) {
        if (p.pval) {
            // this workgroup's greedy candidate (lm.rs:169-179): the first largest, NaN never wins
            __syncthreads();
            float best = 0.0f;
            int idx = -1;
            for (int nl = threadIdx.x; nl < nq * 4; nl += kThreads) {
                const int n = qa * 4 + nl;
                const float v = ybuf[nl];
                if (n < p.n_rows && v == v && (idx < 0 || v > best)) {
                    best = v;
                    idx = n;
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
            if (lane == 0) {
                red[wave] = best;
                reinterpret_cast<int *>(red)[8 + wave] = idx;
            }
            __syncthreads();
            if (threadIdx.x == 0) {
                for (int w = 1; w < kThreads / 64; w++) {
                    const float ob = red[w];
                    const int oi = reinterpret_cast<int *>(red)[8 + w];
                    if (oi >= 0 && (idx < 0 || ob > best || (ob == best && oi < idx))) {
                        best = ob;
                        idx = oi;
                    }
                }
                p.pval[blockIdx.x] = best;
                p.pidx[blockIdx.x] = idx;
            }
        }
        return;
    }
    __syncthreads();
    if (OUT == OUT_QKV) {
        // whole heads per workgroup: bias is in; rotate query and key heads, keep keys and values
        const int D = p.D, half = D / 2;
        const int first_unit = qa * 4 / D;
        for (int i = threadIdx.x; i < nq * 4 / 2; i += kThreads) {
            const int u = i / half, j = i - u * half;
            const int unit = first_unit + u;
            float x = ybuf[u * D + j], y = ybuf[u * D + j + half];
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
        // silu(gate)·up (layer.rs:321-341), quantized per group of 32 for the down projection
        for (int nl = threadIdx.x; nl < nq * 4; nl += kThreads) ybuf[2 * NW + nl] = ref_silu(ybuf[nl]) * ybuf[NW + nl];
        __syncthreads();
        const int g0 = qa * 4 / 32;
        quantize_lds_to(ybuf + 2 * NW, nq * 4, p.zp_out, p.q_out + g0 * 32, p.s_out + g0, p.c_out + g0);
    }
}

template <int FMT, int R, int IN, int OUT, bool EXACT, int NB = 8>
int launch_one(const ProjParams &p, size_t smem, unsigned grid, hipStream_t s)
{
    auto kernel = proj_kernel<FMT, R, IN, OUT, EXACT, NB>;
    if (smem > 64 * 1024) {
        static bool raised = false;
        if (!raised) {
            FG_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       160 * 1024));
            raised = true;
        }
    }
    kernel<<<grid, kThreads, smem, s>>>(p);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

template <int FMT, int R>
int dispatch_generic(const ProjParams &p, int in, bool dots, size_t smem, unsigned grid, hipStream_t s)
{
    if (dots) return in == IN_F32 ? launch_one<FMT, R, IN_F32, OUT_DOTS, false>(p, smem, grid, s)
                                  : launch_one<FMT, R, IN_PREQ, OUT_DOTS, false>(p, smem, grid, s);
    return in == IN_F32 ? launch_one<FMT, R, IN_F32, OUT_STORE, false>(p, smem, grid, s)
                        : launch_one<FMT, R, IN_PREQ, OUT_STORE, false>(p, smem, grid, s);
}

template <int FMT>
int dispatch_rows(const ProjParams &p, int rows, int in, bool dots, size_t smem, unsigned grid, hipStream_t s)
{
    switch (rows) {
    case 1: return dispatch_generic<FMT, 1>(p, in, dots, smem, grid, s);
    case 2: return dispatch_generic<FMT, 2>(p, in, dots, smem, grid, s);
    case 3: return dispatch_generic<FMT, 3>(p, in, dots, smem, grid, s);
    default: return dispatch_generic<FMT, 4>(p, in, dots, smem, grid, s);
    }
}

// The decoder's launches: 16 chunks per wave in flight where workgroups are few (one per head or
// per 32 outputs), 8 where they are many.
template <int FMT, int IN, int OUT, int NB>
int dispatch_exact(const ProjParams &p, bool exact, size_t smem, unsigned grid, hipStream_t s)
{
    return exact ? launch_one<FMT, 1, IN, OUT, true, NB>(p, smem, grid, s) : launch_one<FMT, 1, IN, OUT, false, NB>(p, smem, grid, s);
}

}  // namespace

size_t proj_smem(const ProjParams &p, int rows, int in, int out)
{
    return size_t(proj_layout(rows, p.K, p.G, p.qpw * 4, in, out).total);
}

int launch_proj(const ProjParams &p0, int dtype, int in, int out, bool exact, hipStream_t s)
{
    ProjParams p = p0;
    const int nq = p.quad_end - p.quad_begin;
    if (nq <= 0) return FG_OK;
    const unsigned grid = unsigned((nq + p.qpw - 1) / p.qpw);
    const size_t smem = proj_smem(p, 1, in, out);
    if (smem > 160 * 1024) return set_error(FG_ERR_SHAPE, "rows too wide for the matrix-vector kernel");
    const bool q4 = dtype == FG_Q4B32;
    switch (out) {
    case OUT_QKV:
        return q4 ? dispatch_exact<4, IN_NORM, OUT_QKV, 16>(p, exact, smem, grid, s)
                  : dispatch_exact<8, IN_NORM, OUT_QKV, 16>(p, exact, smem, grid, s);
    case OUT_SWIGLU:
        return q4 ? dispatch_exact<4, IN_NORM, OUT_SWIGLU, 16>(p, exact, smem, grid, s)
                  : dispatch_exact<8, IN_NORM, OUT_SWIGLU, 16>(p, exact, smem, grid, s);
    default:
        if (in == IN_NORM)
            return q4 ? dispatch_exact<4, IN_NORM, OUT_STORE, 8>(p, exact, smem, grid, s)
                      : dispatch_exact<8, IN_NORM, OUT_STORE, 8>(p, exact, smem, grid, s);
        return q4 ? launch_one<4, 1, IN_PREQ, OUT_STORE, false, 8>(p, smem, grid, s)
                  : launch_one<8, 1, IN_PREQ, OUT_STORE, false, 8>(p, smem, grid, s);
    }
}

// Rows 1..4 of a Q7b32 / Q8b32 / Q4b32 product (fg_matmul, fg_matmul_dots).
int launch_matvec(const ProductArgs &a, hipStream_t s)
{
    const fg_table *t = a.t;
    const int rows = int(a.rows);
    if (rows < 1 || rows > 4) return set_error(FG_ERR_SHAPE, "the matrix-vector kernel takes 1 to 4 rows");
    if (t->dtype == FG_T2B128) return set_error(FG_ERR_FORMAT, "the matrix-vector kernel takes Q7b32, Q8b32 and Q4b32 tables");
    ProjParams p{};
    p.codes = t->codes;
    p.wscales = t->scales;
    p.B = int(t->blocks);
    p.G = int(t->groups);
    p.K = int(t->cols);
    p.quad_begin = int(a.quad_begin);
    p.quad_end = int(a.quad_end);
    p.n_rows = int(t->rows);
    p.x = a.x;
    p.q = a.q;
    p.as = a.as;
    p.corr = a.corr;
    p.zp = zero_point_of(t->dtype);
    p.bias = a.bias;
    p.out = a.out;
    p.ld_out = long(a.ld_out);
    p.col_begin = int(a.quad_begin * 4);
    p.accumulate = a.accumulate;
    p.dots = a.dots;
    p.dots_cols = int((a.quad_end - a.quad_begin) * 4);
    const int nq = p.quad_end - p.quad_begin;
    if (nq <= 0) return FG_OK;
    const int in = a.x ? IN_F32 : IN_PREQ;
    const int out = a.dots ? OUT_DOTS : OUT_STORE;
    // Quads per workgroup: enough workgroups to cover the chip, more quads per group when
    // activations are quantized in-kernel (each group quantizes them once).
    int qpw = in == IN_F32 ? nq / 512 : nq / 1024;
    qpw = qpw < 1 ? 1 : (qpw > 16 ? 16 : qpw);
    p.qpw = qpw;
    while (qpw > 1 && proj_smem(p, rows, in, out) > 64 * 1024) p.qpw = qpw = qpw / 2;
    const size_t smem = proj_smem(p, rows, in, out);
    if (smem > 160 * 1024) return set_error(FG_ERR_SHAPE, "rows too wide for the matrix-vector kernel");
    const unsigned grid = unsigned((nq + qpw - 1) / qpw);
    if (t->dtype == FG_Q4B32) return dispatch_rows<4>(p, rows, in, a.dots != nullptr, smem, grid, s);
    return dispatch_rows<8>(p, rows, in, a.dots != nullptr, smem, grid, s);
}

}  // namespace fg
