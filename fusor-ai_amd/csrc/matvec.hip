// The decode product: a few activation rows (1..4) against a quantized table, HBM-bound.
//
// Reference: matmul (matmul.rs:265-317) -> quant_tiles / quant_tile / quad_pass / accumulate
// (matmul.rs:521-763) with the scalar backend's arithmetic (arch/scalar.rs:68-90). Per output
// column n and activation row r:  D_g = corr_g + Σ_k u[n,k]·a[r,k]  (int32, exact in any order),
//   s = +0;  for g in order:  s = fl(s + fl(fl((float)D_g) · fl(ws[n,g] · as[r,g])))
// then the bias (linear.rs:63-68) and, for residual projections, h = fl(h + y) (linear.rs:134-143).
//
// Mapping. A workgroup owns `qpw` consecutive quads (4 output rows each) and all of their blocks:
// a contiguous run of the table. Its four waves stream that run in 1 KiB chunks (64 lanes x 16 B,
// fully coalesced 128-bit loads). Every lane turns its 16 bytes into a partial int32 dot with
// v_dot4 against activations staged once in LDS (quantized in-kernel when the input is f32),
// scales its group's total (exact integer, pair-summed through DPP for 7/8-bit codes) into the
// group's f32 term and parks it in LDS. Once all terms are in, one thread per output adds them in
// group order: the only order-dependent step, done exactly as the reference does it.
#include "common.h"

namespace fg {
namespace {

constexpr int kThreads = 256;

struct MatvecParams {
    const int8_t *codes;
    const float *wscales;
    int B, G;  // blocks and groups per row (equal for the 7/8/4-bit formats)
    int K;
    int quad_begin, quad_end, qpw;
    int n_rows;  // the table's rows: bias applies below them only (linear.rs:63-68)
    const float *x;
    const int8_t *q;
    const float *as;
    const int32_t *corr;
    int zp;
    const float *bias;
    float *out;
    long ld_out;
    int col_begin;
    int accumulate;
    int32_t *dots;
    int dots_cols;
};

__device__ __forceinline__ int dot16(int4 w, int4 a) { return dot4(w.w, a.w, dot4(w.z, a.z, dot4(w.y, a.y, dot4(w.x, a.x, 0)))); }

// Stage the activation rows in LDS: copy pre-quantized rows, or quantize f32 rows (8 lanes per
// group of 32, as quantize_rows does it).
template <int R, bool FUSED>
__device__ __forceinline__ void stage_activations(const MatvecParams &p, int8_t *act_q, float *act_s, int32_t *act_c)
{
    const int tid = threadIdx.x;
    const int K = p.K, G = p.G;
    if (FUSED) {
        const int sub = tid & 7;
        for (int grp = tid >> 3; grp < R * G; grp += kThreads / 8) {
            const int r = grp / G, g = grp - r * G;
            float4 v = *reinterpret_cast<const float4 *>(p.x + size_t(r) * K + g * 32 + sub * 4);
            float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
            amax = fmaxf(0.0f, amax);
            amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
            amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
            amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
            const float d = group_scale(amax, 127.0f);
            const int l0 = quantize_level(v.x, d), l1 = quantize_level(v.y, d);
            const int l2 = quantize_level(v.z, d), l3 = quantize_level(v.w, d);
            int sum = l0 + l1 + l2 + l3;
            sum += __shfl_xor(sum, 1, 64);
            sum += __shfl_xor(sum, 2, 64);
            sum += __shfl_xor(sum, 4, 64);
            reinterpret_cast<int *>(act_q)[(r * K + g * 32) / 4 + sub] = pack4(l0, l1, l2, l3);
            if (sub == 0) {
                act_s[grp] = d;
                act_c[grp] = -p.zp * sum;
            }
        }
    } else {
        const int4 *src = reinterpret_cast<const int4 *>(p.q);
        int4 *dst = reinterpret_cast<int4 *>(act_q);
        for (int i = tid; i < R * K / 16; i += kThreads) dst[i] = src[i];
        for (int i = tid; i < R * G; i += kThreads) {
            act_s[i] = p.as[i];
            act_c[i] = p.corr[i];
        }
    }
}

// FMT: 8 for signed 8-bit levels (Q7b32 folded, Q8b32), 4 for offset nibbles (Q4b32).
template <int FMT, int R, bool FUSED, bool DOTS>
__global__ __launch_bounds__(kThreads) void matvec_kernel(MatvecParams p)
{
    extern __shared__ __align__(16) unsigned char smem[];
    const int K = p.K, G = p.G, B = p.B;
    const int qa = p.quad_begin + int(blockIdx.x) * p.qpw;
    const int nq = min(p.qpw, p.quad_end - qa);
    const int NW = p.qpw * 4;
    int8_t *act_q = reinterpret_cast<int8_t *>(smem);
    float *act_s = reinterpret_cast<float *>(smem + ((R * K + 15) & ~15));
    int32_t *act_c = reinterpret_cast<int32_t *>(act_s + R * G);
    float *terms = reinterpret_cast<float *>(act_c + R * G);  // [R][G][NW]

    stage_activations<R, FUSED>(p, act_q, act_s, act_c);
    __syncthreads();

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int QB = FMT == 8 ? 128 : 64;         // device bytes per quad block
    constexpr int QB_PER_CHUNK = 1024 / QB;         // quad blocks per 1 KiB chunk
    const int total_qb = nq * B;
    const int chunks = (total_qb + QB_PER_CHUNK - 1) / QB_PER_CHUNK;
    const int8_t *region = p.codes + size_t(qa) * B * QB;
    const int L = FMT == 8 ? (lane >> 1) & 3 : lane & 3;
    const int h = FMT == 8 ? lane & 1 : 0;
    const int qb_in_chunk = FMT == 8 ? lane >> 3 : lane >> 2;

    constexpr int U = 4;
    for (int c0 = wave; c0 < chunks; c0 += 4 * U) {
        int4 w[U];
        float ws[U];
        int qbs[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int c = c0 + 4 * u;
            const int qb = c * QB_PER_CHUNK + qb_in_chunk;
            qbs[u] = qb;
            if (c < chunks && qb < total_qb) {
                w[u] = *reinterpret_cast<const int4 *>(region + size_t(c) * 1024 + lane * 16);
                const int ql = qb / B, b = qb - ql * B;
                ws[u] = p.wscales[(size_t(qa + ql) * G + b) * 4 + L];
            } else {
                w[u] = make_int4(0, 0, 0, 0);
                ws[u] = 0.0f;
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int c = c0 + 4 * u;
            if (c >= chunks) break;  // uniform across the wave
            const int qb = qbs[u];
            const bool valid = qb < total_qb;
            const int ql = valid ? qb / B : 0, b = valid ? qb - ql * B : 0;
#pragma unroll
            for (int r = 0; r < R; r++) {
                int D;
                if (FMT == 8) {
                    const int4 a = *reinterpret_cast<const int4 *>(act_q + r * K + b * 32 + h * 16);
                    D = dot16(w[u], a);
                    D += xor1(D);  // the row-block's other half
                } else {
                    const int4 a0 = *reinterpret_cast<const int4 *>(act_q + r * K + b * 32);
                    const int4 a1 = *reinterpret_cast<const int4 *>(act_q + r * K + b * 32 + 16);
                    const int4 lo = make_int4(w[u].x & 0x0F0F0F0F, w[u].y & 0x0F0F0F0F, w[u].z & 0x0F0F0F0F, w[u].w & 0x0F0F0F0F);
                    const int4 hi = make_int4((w[u].x >> 4) & 0x0F0F0F0F, (w[u].y >> 4) & 0x0F0F0F0F,
                                              (w[u].z >> 4) & 0x0F0F0F0F, (w[u].w >> 4) & 0x0F0F0F0F);
                    D = dot16(lo, a0) + dot16(hi, a1) + act_c[r * G + b];
                }
                if (valid && h == 0) {
                    if (DOTS) {
                        const int n = (qa + ql) * 4 + L;
                        p.dots[(size_t(r) * p.dots_cols + (n - p.col_begin)) * G + b] = D;
                    } else {
                        const float scale = ws[u] * act_s[r * G + b];
                        terms[(r * G + b) * NW + ql * 4 + L] = float(D) * scale;
                    }
                }
            }
        }
    }
    if (DOTS) return;
    __syncthreads();

    // Group order: the reference's sequential sum, one thread per (row, output).
    for (int i = threadIdx.x; i < R * NW; i += kThreads) {
        const int r = i / NW, nl = i - r * NW;
        if (nl >= nq * 4) continue;
        float s = 0.0f;
        const float *t = terms + r * G * NW + nl;
        for (int g = 0; g < G; g++) s = s + t[g * NW];
        const int n = qa * 4 + nl;
        if (p.bias && n < p.n_rows) s = s + p.bias[n];
        float *o = p.out + r * p.ld_out + (n - p.col_begin);
        *o = p.accumulate ? *o + s : s;
    }
}

template <int FMT, int R, bool FUSED, bool DOTS>
int launch(const MatvecParams &p, size_t smem, unsigned grid, hipStream_t s)
{
    matvec_kernel<FMT, R, FUSED, DOTS><<<grid, kThreads, smem, s>>>(p);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

template <int FMT, int R>
int dispatch(const MatvecParams &p, bool fused, bool dots, size_t smem, unsigned grid, hipStream_t s)
{
    if (dots) return fused ? launch<FMT, R, true, true>(p, smem, grid, s) : launch<FMT, R, false, true>(p, smem, grid, s);
    return fused ? launch<FMT, R, true, false>(p, smem, grid, s) : launch<FMT, R, false, false>(p, smem, grid, s);
}

template <int FMT>
int dispatch_rows(const MatvecParams &p, int rows, bool fused, bool dots, size_t smem, unsigned grid, hipStream_t s)
{
    switch (rows) {
    case 1: return dispatch<FMT, 1>(p, fused, dots, smem, grid, s);
    case 2: return dispatch<FMT, 2>(p, fused, dots, smem, grid, s);
    case 3: return dispatch<FMT, 3>(p, fused, dots, smem, grid, s);
    default: return dispatch<FMT, 4>(p, fused, dots, smem, grid, s);
    }
}

}  // namespace

// Rows 1..4 of a Q7b32 / Q8b32 / Q4b32 product.
int launch_matvec(const ProductArgs &a, hipStream_t s)
{
    const fg_table *t = a.t;
    const int rows = int(a.rows);
    if (rows < 1 || rows > 4) return set_error(FG_ERR_SHAPE, "the matrix-vector kernel takes 1 to 4 rows");
    if (t->dtype == FG_T2B128) return set_error(FG_ERR_FORMAT, "T2b128 products are not built on the GPU");
    MatvecParams p{};
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
    const bool fused = a.x != nullptr;
    // Quads per workgroup: enough workgroups to cover the chip, more quads per group when
    // activations are quantized in-kernel (each group quantizes them once).
    int qpw = fused ? nq / 512 : nq / 1024;
    qpw = qpw < 1 ? 1 : (qpw > 16 ? 16 : qpw);
    const size_t act_bytes = size_t((rows * p.K + 15) & ~15) + size_t(rows) * p.G * 8;
    auto smem_for = [&](int qq) { return act_bytes + (a.dots ? 0 : size_t(rows) * p.G * qq * 4 * 4); };
    while (qpw > 1 && smem_for(qpw) > 64 * 1024) qpw /= 2;
    if (smem_for(qpw) > 160 * 1024) return set_error(FG_ERR_SHAPE, "rows too wide for the matrix-vector kernel");
    p.qpw = qpw;
    const unsigned grid = unsigned((nq + qpw - 1) / qpw);
    const size_t smem = smem_for(qpw);
    if (smem > 64 * 1024) {
        // Larger than the default dynamic LDS limit: raise it for this instantiation.
        return set_error(FG_ERR_SHAPE, "rows too wide for the matrix-vector kernel");
    }
    if (t->dtype == FG_Q4B32) return dispatch_rows<4>(p, rows, fused, a.dots != nullptr, smem, grid, s);
    return dispatch_rows<8>(p, rows, fused, a.dots != nullptr, smem, grid, s);
}

}  // namespace fg
