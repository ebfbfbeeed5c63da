// The batched (prefill) product on the int8 matrix cores.
//
// Reference: the same arithmetic as the matrix-vector product (matmul.rs:628-763,
// arch/scalar.rs:68-90), reached through quant_tiles with 4-row tiles (matmul.rs:521-577) and
// conv::project_rows for many rows (conv.rs:563-606). Per (row r, output n):
//   s = +0;  for g in order:  s = fl(s + fl(fl((float)D_g) · fl(ws[n,g] · as[r,g])))
//
// v_mfma_i32_32x32x32_i8 multiplies a 32x32 tile of activation levels by a 32x32 tile of weight
// levels over K = 32, exactly one block: its int32 results are the group accumulators D_g of a
// 32x32 output tile, exact. Weight levels are signed on the device (Q7b32 stored as u - 64; Q4b32
// nibbles widened to u - 8 in registers), so no correction term is needed. Each wave owns a 32 x
// 64 output tile (two MFMAs per block) and keeps the running f32 sums in registers; the K loop
// walks the blocks in order, so the sums are the reference's to the bit.
//
// MFMA operand layout (32x32xK): lane l feeds row (or column) l % 32 and K-half l / 32; the same
// K positions are used for both operands, so the sum covers the block's 32 inputs. Result:
// lane l holds column l % 32, rows 8·(v/4) + 4·(l/32) + v%4 for v = 0..15.
#include "common.h"

namespace fg {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

struct GemmParams {
    const int8_t *codes;
    const float *wscales;
    int B, G, K;
    int M, Mpad;
    int col_begin, col_end;
    int n_rows;
    const int8_t *q;      // [M][K] levels
    const float *as_t;    // [G][Mpad] activation scales, block-major
    const float *bias;
    float *out;
    long ld_out;
    int accumulate;
    int32_t *dots;
    int dots_cols;
};

template <int FMT>
__device__ __forceinline__ v4i load_weights(const GemmParams &p, int n, int b, int h, bool valid)
{
    if (!valid) return v4i{0, 0, 0, 0};
    const int quad = n >> 2, L = n & 3;
    if (FMT == 8) return *reinterpret_cast<const v4i *>(p.codes + (size_t(quad) * p.B + b) * 128 + L * 32 + h * 16);
    v4i raw = *reinterpret_cast<const v4i *>(p.codes + (size_t(quad) * p.B + b) * 64 + L * 16);
    const int sh = h * 4;
    return v4i{nibbles_signed(raw.x >> sh), nibbles_signed(raw.y >> sh), nibbles_signed(raw.z >> sh),
               nibbles_signed(raw.w >> sh)};
}

// WM waves along M (a 32·WM-row tile), 4 / WM along N (64 columns each).
template <int FMT, int WM, bool DOTS>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams p)
{
    constexpr int WN = 4 / WM;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave % WM, wn = wave / WM;
    const int i = lane & 31, h = lane >> 5;
    const int m0 = int(blockIdx.y) * 32 * WM + wm * 32;
    const int n0 = p.col_begin + int(blockIdx.x) * 64 * WN + wn * 64;
    if (m0 >= p.M || n0 >= p.col_end) return;

    const int row = m0 + i;
    const bool row_ok = row < p.M;
    const int n_a = n0 + i, n_b = n0 + 32 + i;
    const bool ok_a = n_a < p.col_end, ok_b = n_b < p.col_end;
    const int8_t *arow = p.q + size_t(row) * p.K + h * 16;

    float s0[16], s1[16];
#pragma unroll
    for (int v = 0; v < 16; v++) s0[v] = s1[v] = 0.0f;

    for (int b = 0; b < p.B; b++) {
        const v4i a = row_ok ? *reinterpret_cast<const v4i *>(arow + b * 32) : v4i{0, 0, 0, 0};
        const v4i wa = load_weights<FMT>(p, n_a, b, h, ok_a);
        const v4i wb = load_weights<FMT>(p, n_b, b, h, ok_b);
        const float ws_a = ok_a ? p.wscales[(size_t(n_a >> 2) * p.G + b) * 4 + (n_a & 3)] : 0.0f;
        const float ws_b = ok_b ? p.wscales[(size_t(n_b >> 2) * p.G + b) * 4 + (n_b & 3)] : 0.0f;
        const float *asb = p.as_t + size_t(b) * p.Mpad + m0 + 4 * h;
        float4 as4[4];
#pragma unroll
        for (int u = 0; u < 4; u++) as4[u] = *reinterpret_cast<const float4 *>(asb + 8 * u);
        const v16i zero = {0};
        const v16i da = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, wa, zero, 0, 0, 0);
        const v16i db = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, wb, zero, 0, 0, 0);
        if (DOTS) {
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int r = m0 + 8 * (v >> 2) + 4 * h + (v & 3);
                if (r < p.M) {
                    if (ok_a) p.dots[(size_t(r) * p.dots_cols + (n_a - p.col_begin)) * p.G + b] = da[v];
                    if (ok_b) p.dots[(size_t(r) * p.dots_cols + (n_b - p.col_begin)) * p.G + b] = db[v];
                }
            }
            continue;
        }
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const float4 f = as4[v >> 2];
            const float asv = (v & 3) == 0 ? f.x : (v & 3) == 1 ? f.y : (v & 3) == 2 ? f.z : f.w;
            s0[v] = s0[v] + float(da[v]) * (ws_a * asv);
            s1[v] = s1[v] + float(db[v]) * (ws_b * asv);
        }
    }
    if (DOTS) return;
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int r = m0 + 8 * (v >> 2) + 4 * h + (v & 3);
        if (r >= p.M) continue;
        float *orow = p.out + size_t(r) * p.ld_out - p.col_begin;
        if (ok_a) {
            float y = s0[v];
            if (p.bias && n_a < p.n_rows) y = y + p.bias[n_a];
            orow[n_a] = p.accumulate ? orow[n_a] + y : y;
        }
        if (ok_b) {
            float y = s1[v];
            if (p.bias && n_b < p.n_rows) y = y + p.bias[n_b];
            orow[n_b] = p.accumulate ? orow[n_b] + y : y;
        }
    }
}

// as [M][G] -> as_t [G][Mpad] (zeros past M).
__global__ void transpose_scales_kernel(const float *__restrict__ as, int M, int G, int Mpad, float *__restrict__ as_t)
{
    const size_t id = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= size_t(G) * Mpad) return;
    const int g = int(id / Mpad), r = int(id % Mpad);
    as_t[id] = r < M ? as[size_t(r) * G + g] : 0.0f;
}

template <int FMT, int WM>
int launch_tiles(const GemmParams &p, bool dots, hipStream_t s)
{
    constexpr int WN = 4 / WM;
    const int ncols = p.col_end - p.col_begin;
    dim3 grid(unsigned((ncols + 64 * WN - 1) / (64 * WN)), unsigned((p.M + 32 * WM - 1) / (32 * WM)));
    if (dots) gemm_kernel<FMT, WM, true><<<grid, 256, 0, s>>>(p);
    else gemm_kernel<FMT, WM, false><<<grid, 256, 0, s>>>(p);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

// T2b128 (ternary levels, one scale per 128 inputs: matmul.rs:461-469, quant.rs:168-177): one
// thread per (row, output), the groups in order, each group's four blocks summed as integers
// before the scaling (matmul.rs:671-709). Device row-block of 8 bytes: byte i holds the offset
// codes of inputs i, i + 8, i + 16, i + 24 in its bit pairs. Not tuned: no workload uses it.
__global__ __launch_bounds__(256) void t2_product_kernel(const uint8_t *__restrict__ codes, const float *__restrict__ wscales,
                                                         int B, int G, int K, int n_rows, const int8_t *__restrict__ q,
                                                         const float *__restrict__ as, const int32_t *__restrict__ corr,
                                                         int rows, int col_begin, int ncols, const float *__restrict__ bias,
                                                         float *out, long ld_out, int accumulate, int32_t *dots)
{
    const long id = long(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= long(rows) * ncols) return;
    const int r = int(id / ncols), c = int(id % ncols);
    const int n = col_begin + c, quad = n >> 2, L = n & 3;
    const int8_t *qa = q + size_t(r) * K;
    float s = 0.0f;
    for (int g = 0; g < G; g++) {
        int D = corr[size_t(r) * G + g];
        for (int b = 4 * g; b < 4 * g + 4; b++) {
            const uint8_t *rb = codes + (size_t(quad) * B + b) * 32 + L * 8;
            const int lo = *reinterpret_cast<const int *>(rb), hi = *reinterpret_cast<const int *>(rb + 4);
            const int *ad = reinterpret_cast<const int *>(qa + b * 32);
            for (int t = 0; t < 4; t++) {
                D = dot4((lo >> (2 * t)) & 0x03030303, ad[2 * t], D);
                D = dot4((hi >> (2 * t)) & 0x03030303, ad[2 * t + 1], D);
            }
        }
        if (dots) {
            dots[(size_t(r) * ncols + c) * G + g] = D;
            continue;
        }
        s = s + float(D) * (wscales[(size_t(quad) * G + g) * 4 + L] * as[size_t(r) * G + g]);
    }
    if (dots) return;
    if (bias && n < n_rows) s = s + bias[n];
    float *o = out + size_t(r) * ld_out + c;
    *o = accumulate ? *o + s : s;
}

}  // namespace

int launch_t2(const ProductArgs &a, hipStream_t s)
{
    const fg_table *t = a.t;
    const int M = int(a.rows), K = int(t->cols), G = int(t->groups);
    const int col_begin = int(a.quad_begin * 4), ncols = int((a.quad_end - a.quad_begin) * 4);
    int8_t *q = const_cast<int8_t *>(a.q);
    const float *as = a.as;
    const int32_t *corr = a.corr;
    void *ws = nullptr;
    int rc = FG_OK;
    if (a.x) {  // quantize the f32 rows first (groups of 128)
        const size_t qb = (size_t(M) * K + 255) / 256 * 256, sb = (size_t(M) * G * 4 + 255) / 256 * 256;
        FG_HIP(hipMallocAsync(&ws, qb + 2 * sb, s));
        q = static_cast<int8_t *>(ws);
        float *sc = reinterpret_cast<float *>(static_cast<char *>(ws) + qb);
        int32_t *co = reinterpret_cast<int32_t *>(static_cast<char *>(ws) + qb + sb);
        rc = launch_quantize_rows(a.x, size_t(M) * K, FG_T2B128, q, sc, co, s);
        as = sc;
        corr = co;
    }
    if (rc == FG_OK) {
        const long n = long(M) * ncols;
        t2_product_kernel<<<unsigned((n + 255) / 256), 256, 0, s>>>(reinterpret_cast<const uint8_t *>(t->codes), t->scales, int(t->blocks),
                                                                   G, K, int(t->rows), q, as, corr, M, col_begin, ncols, a.bias,
                                                                   a.out, long(a.ld_out), a.accumulate, a.dots);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) rc = check_hip(e, "t2_product_kernel");
    }
    if (ws) {
        hipError_t e = hipFreeAsync(ws, s);
        if (rc == FG_OK && e != hipSuccess) rc = check_hip(e, "hipFreeAsync");
    }
    return rc;
}

int launch_gemm(const ProductArgs &a, hipStream_t s)
{
    const fg_table *t = a.t;
    if (t->dtype == FG_T2B128) return launch_t2(a, s);
    const int M = int(a.rows), K = int(t->cols), G = int(t->groups);
    const int Mpad = (M + 63) / 64 * 64;
    // Workspace: levels (when the input is f32), scales, corrections, block-major scales.
    const size_t q_bytes = a.x ? (size_t(M) * K + 255) / 256 * 256 : 0;
    const size_t s_bytes = a.x ? (size_t(M) * G * 4 + 255) / 256 * 256 : 0;
    const size_t t_bytes = size_t(G) * Mpad * 4;
    void *ws = nullptr;
    FG_HIP(hipMallocAsync(&ws, q_bytes + 2 * s_bytes + t_bytes, s));
    int8_t *q = const_cast<int8_t *>(a.q);
    const float *as = a.as;
    char *base = static_cast<char *>(ws);
    int rc = FG_OK;
    if (a.x) {
        q = reinterpret_cast<int8_t *>(base);
        float *sc = reinterpret_cast<float *>(base + q_bytes);
        int32_t *co = reinterpret_cast<int32_t *>(base + q_bytes + s_bytes);
        rc = launch_quantize_rows(a.x, size_t(M) * K, t->dtype, q, sc, co, s);
        as = sc;
    }
    float *as_t = reinterpret_cast<float *>(base + q_bytes + 2 * s_bytes);
    if (rc == FG_OK) {
        const size_t n = size_t(G) * Mpad;
        transpose_scales_kernel<<<unsigned((n + 255) / 256), 256, 0, s>>>(as, M, G, Mpad, as_t);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) rc = check_hip(e, "transpose_scales_kernel");
    }
    if (rc == FG_OK) {
        GemmParams p{};
        p.codes = t->codes;
        p.wscales = t->scales;
        p.B = int(t->blocks);
        p.G = G;
        p.K = K;
        p.M = M;
        p.Mpad = Mpad;
        p.col_begin = int(a.quad_begin * 4);
        p.col_end = int(a.quad_end * 4);
        p.n_rows = int(t->rows);
        p.q = q;
        p.as_t = as_t;
        p.bias = a.bias;
        p.out = a.out;
        p.ld_out = long(a.ld_out);
        p.accumulate = a.accumulate;
        p.dots = a.dots;
        p.dots_cols = p.col_end - p.col_begin;
        const bool dots = a.dots != nullptr;
        const bool tall = M > 32;
        if (t->dtype == FG_Q4B32) rc = tall ? launch_tiles<4, 2>(p, dots, s) : launch_tiles<4, 1>(p, dots, s);
        else rc = tall ? launch_tiles<8, 2>(p, dots, s) : launch_tiles<8, 1>(p, dots, s);
    }
    hipError_t e = hipFreeAsync(ws, s);
    if (rc == FG_OK && e != hipSuccess) rc = check_hip(e, "hipFreeAsync");
    return rc;
}

// Rows 1..4 stream the weights once through the matrix-vector kernel; more rows go to the
// matrix cores.
int launch_product(const ProductArgs &a, hipStream_t s)
{
    if (a.rows == 0 || a.quad_end <= a.quad_begin) return FG_OK;
    if (a.t->dtype == FG_T2B128) return launch_t2(a, s);
    if (a.rows <= 4) return launch_matvec(a, s);
    return launch_gemm(a, s);
}

}  // namespace fg
