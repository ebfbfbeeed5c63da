// The product's matrix-vector path (fg_matmul, rows 1..4) and the decoder's launch checks, over
// the projection kernel of proj_kernel.h.
#include "proj_kernel.h"

namespace fg {

int launch_proj_q8(const ProjParams &p, int in, int out, bool exact, int nb, size_t smem, unsigned grid, hipStream_t s);
int launch_proj_q4(const ProjParams &p, int in, int out, bool exact, int nb, size_t smem, unsigned grid, hipStream_t s);

namespace {

template <int FMT, int R, int NB = 8>
int dispatch_generic(const ProjParams &p, int in, bool dots, bool tree, size_t smem, unsigned grid, hipStream_t s)
{
    if (dots) return in == IN_F32 ? launch_one<FMT, R, IN_F32, OUT_DOTS, false>(p, smem, grid, s)
                                  : launch_one<FMT, R, IN_PREQ, OUT_DOTS, false>(p, smem, grid, s);
    if constexpr (R == 1) {
        // FG_PARALLEL_SUM: the decoder's parallel-order sums of the same terms
        if (tree) return in == IN_F32 ? launch_one<FMT, 1, IN_F32, OUT_STORE, false, NB, true>(p, smem, grid, s)
                                      : launch_one<FMT, 1, IN_PREQ, OUT_STORE, false, NB, true>(p, smem, grid, s);
    }
    return in == IN_F32 ? launch_one<FMT, R, IN_F32, OUT_STORE, false, NB>(p, smem, grid, s)
                        : launch_one<FMT, R, IN_PREQ, OUT_STORE, false, NB>(p, smem, grid, s);
}

// One row takes the batch depth its workgroups' shares need (batch_depth), more rows 8 chunks.
template <int FMT>
int dispatch_rows(const ProjParams &p, int rows, int in, bool dots, bool tree, int nb, size_t smem, unsigned grid,
                  hipStream_t s)
{
    switch (rows) {
    case 1:
        switch (nb) {
        case 1: return dispatch_generic<FMT, 1, 1>(p, in, dots, tree, smem, grid, s);
        case 2: return dispatch_generic<FMT, 1, 2>(p, in, dots, tree, smem, grid, s);
        case 4: return dispatch_generic<FMT, 1, 4>(p, in, dots, tree, smem, grid, s);
        default: return dispatch_generic<FMT, 1>(p, in, dots, tree, smem, grid, s);
        }
    case 2: return dispatch_generic<FMT, 2>(p, in, dots, false, smem, grid, s);
    case 3: return dispatch_generic<FMT, 3>(p, in, dots, false, smem, grid, s);
    default: return dispatch_generic<FMT, 4>(p, in, dots, false, smem, grid, s);
    }
}

// Batch depth: the fewest chunks in flight per wave (1, 2, 4 or 8) that cover a wave's share in
// one batch. A wave's instructions are its latency at one wave per SIMD, so the address
// arithmetic and reads of unused batch slots would cost time at small shares.
int batch_depth(const ProjParams &p, int dtype, int out)
{
    const int qb_per_chunk = dtype == FG_Q4B32 ? 16 : 8;
    const int per_table = (p.qpw * p.B + qb_per_chunk - 1) / qb_per_chunk;
    const int stride = out == OUT_SWIGLU ? 2 : 4;
    const int mine = (per_table + stride - 1) / stride;
    return mine <= 1 ? 1 : mine <= 2 ? 2 : mine <= 4 ? 4 : 8;
}

// RMSNorm + quantize of one row (the IN_NORM prologue's arithmetic, exact or parallel order) into
// q_out, s_out and c_out: the head's input, formed once instead of in each of its workgroups.
template <bool EXACT>
__global__ __launch_bounds__(kThreads) void norm_quantize_kernel(ProjParams p)
{
    __shared__ __align__(16) float nbuf[4 * 4 * kThreads];
    __shared__ float red[16];
    StageRegs g;
    stage_issue<8, 1, IN_NORM>(p, g);
    stage_finish<8, 1, IN_NORM, EXACT>(p, g, p.q_out, p.s_out, p.c_out, nbuf, red);
}

// The same over rows: workgroup y takes row y of x [rows][K] into its levels [rows][K], scales and
// corrections [rows][G].
template <bool EXACT>
__global__ __launch_bounds__(kThreads) void norm_quantize_rows_kernel(ProjParams p)
{
    __shared__ __align__(16) float nbuf[4 * 4 * kThreads];
    __shared__ float red[16];
    const size_t y = blockIdx.x;
    p.x += y * p.K;
    p.q_out += y * p.K;
    p.s_out += y * p.G;
    p.c_out += y * p.G;
    StageRegs g;
    stage_issue<8, 1, IN_NORM>(p, g);
    stage_finish<8, 1, IN_NORM, EXACT>(p, g, p.q_out, p.s_out, p.c_out, nbuf, red);
}

}  // namespace

int launch_norm_quantize_rows(const ProjParams &p, int rows, bool exact, hipStream_t s)
{
    if (p.K % 32 || p.K > 4 * 4 * kThreads || p.G * 32 != p.K)
        return set_error(FG_ERR_SHAPE, "the RMSNorm prologue takes rows of at most 4096");
    if (rows <= 0) return FG_OK;
    if (exact) norm_quantize_rows_kernel<true><<<unsigned(rows), kThreads, 0, s>>>(p);
    else norm_quantize_rows_kernel<false><<<unsigned(rows), kThreads, 0, s>>>(p);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

int launch_norm_quantize(const ProjParams &p, bool exact, hipStream_t s)
{
    if (p.K % 32 || p.K > 4 * 4 * kThreads || p.G * 32 != p.K)
        return set_error(FG_ERR_SHAPE, "the RMSNorm prologue takes rows of at most 4096");
    if (exact) norm_quantize_kernel<true><<<1, kThreads, 0, s>>>(p);
    else norm_quantize_kernel<false><<<1, kThreads, 0, s>>>(p);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

size_t proj_smem(const ProjParams &p, int rows, int in, int out)
{
    return size_t(proj_layout(rows, p.K, p.G, p.qpw * 4, in, out).total);
}

int launch_proj(const ProjParams &p0, int dtype, int in, int out, bool exact, hipStream_t s)
{
    ProjParams p = p0;
    const int nq = p.quad_end - p.quad_begin;
    if (nq <= 0) return FG_OK;
    if (p.qstride < 1) p.qstride = 1;
    if (p.qstride & (p.qstride - 1)) return set_error(FG_ERR_SHAPE, "the quad stride is a power of two");
    p.qshift = __builtin_ctz(unsigned(p.qstride));
    proj_derive(p);
    const int span = p.qstride * p.qpw;
    if (p.qstride > 1 && (nq % span || p.qpw != 2)) return set_error(FG_ERR_SHAPE, "strided quads come in whole pairs");
    if (p.pval && (out != OUT_STORE || p.qpw > 16 || p.qstride != 1))
        return set_error(FG_ERR_SHAPE, "greedy candidates take at most 16 consecutive quads per workgroup");
    if (out == OUT_QKV && (p.qpw != 2 || p.qstride * 8 != p.D))
        return set_error(FG_ERR_SHAPE, "the QKV epilogue takes one rotary pair per workgroup");
    if (out == OUT_SWIGLU && p.q_out && (p.qpw != 8 || p.qstride != 1 || nq % 8))
        return set_error(FG_ERR_SHAPE, "the quantized SwiGLU row takes 8 quads (one group) per workgroup");
    if ((in == IN_NORM || in == IN_EMBED) && p.K > 4 * 4 * kThreads)
        return set_error(FG_ERR_SHAPE, "the RMSNorm prologue takes rows of at most 4096");
    if (in == IN_EMBED && (out != OUT_QATTN || !p.e_codes || !p.e_scales || !p.x_out || p.e_lane < 0 || p.e_lane > 3))
        return set_error(FG_ERR_ARG, "a table row as input takes the query attention, its quad's codes and scales and an output row");
    if (in == IN_ATTN && (p.K > 4 * kThreads || p.chunks < 1 || p.chunks > kMaxChunks || p.heads * p.D != p.K ||
                          (p.D != 32 && p.D != 64 && p.D != 128) || p.kv_heads < 1 || p.heads % p.kv_heads))
        return set_error(FG_ERR_SHAPE, "the attention merge takes rows of at most 1024, head_dim 32/64/128 and 1 to 8 chunks");
    if (out == OUT_QATTN &&
        ((p.D != 32 && p.D != 64 && p.D != 128) || p.qpw * 4 != p.D || p.qstride != 1 || p.kv_heads < 1 || p.heads % p.kv_heads ||
         (p.heads + 2 * p.kv_heads) * p.D != p.n_rows || p.n_rows % 4 || p.chunks < 1 || p.chunks > kMaxChunks ||
         p.per_chunk < kTileKeys || size_t(p.chunks) * p.per_chunk < size_t(p.position) || p.position >= p.capacity))
        return set_error(FG_ERR_SHAPE, "the query attention takes head_dim 32/64/128, whole query and key heads and 1 to 8 chunks");
    const unsigned grid = out == OUT_QATTN ? unsigned(p.heads * p.chunks + 2 * p.kv_heads * (p.D / 8))
                          : p.qstride == 1 ? unsigned((nq + p.qpw - 1) / p.qpw)
                                           : unsigned(nq / span * p.qstride);
    const size_t smem = proj_smem(p, 1, in, out);
    if (smem > 160 * 1024) return set_error(FG_ERR_SHAPE, "rows too wide for the matrix-vector kernel");
    const int nb = batch_depth(p, dtype, out);
    if (out == OUT_QATTN && ((in != IN_NORM && in != IN_EMBED) || (exact && (in != IN_NORM || !p.scores))))
        return set_error(FG_ERR_SHAPE, "the query attention takes a normed row (in the exact order, and its scores' buffer)");
    return dtype == FG_Q4B32 ? launch_proj_q4(p, in, out, exact, nb, smem, grid, s)
                             : launch_proj_q8(p, in, out, exact, nb, smem, grid, s);
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
    // Quads per workgroup: the most (a power of two, at most 16) whose codes fit in 64 KiB,
    // halved while fewer than 128 workgroups would cover the chip. Measured on 4864 x 896 Q8b32
    // (8 quads: 4.1 us against 4.6 at 4), 14336 x 4096 Q4b32 (8: 10.3 us against 13.1 at 2) and
    // 151936 x 896 (16).
    const int run = int(t->blocks) * (t->dtype == FG_Q4B32 ? 64 : 128);  // code bytes per quad
    int qpw = 16;
    while (qpw > 1 && qpw * run > 65536) qpw /= 2;
    while (qpw > 1 && (nq + qpw - 1) / qpw < 128) qpw /= 2;
    p.qpw = qpw;
    p.qstride = 1;
    proj_derive(p);
    while (qpw > 1 && proj_smem(p, rows, in, out) > 64 * 1024) p.qpw = qpw = qpw / 2;
    const size_t smem = proj_smem(p, rows, in, out);
    if (smem > 160 * 1024) return set_error(FG_ERR_SHAPE, "rows too wide for the matrix-vector kernel");
    const unsigned grid = unsigned((nq + qpw - 1) / qpw);
    const int nb = batch_depth(p, t->dtype, out);
    const bool tree = a.parallel && rows == 1 && !a.dots;
    if (t->dtype == FG_Q4B32) return dispatch_rows<4>(p, rows, in, a.dots != nullptr, tree, nb, smem, grid, s);
    return dispatch_rows<8>(p, rows, in, a.dots != nullptr, tree, nb, smem, grid, s);
}

}  // namespace fg
