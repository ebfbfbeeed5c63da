// The decoder's dispatch of proj_kernel for one weight format (FMT), instantiated by
// proj_q8.hip and proj_q4.hip so the two formats compile in parallel.
#pragma once

#include "proj_kernel.h"

namespace fg {
namespace {

// The decoder's launches, in the reference's reduction order (exact) or with parallel f32 sums.
template <int FMT, int IN, int OUT, int NB>
int dispatch_exact(const ProjParams &p, bool exact, size_t smem, unsigned grid, hipStream_t s)
{
    return exact ? launch_one<FMT, 1, IN, OUT, true, NB, false>(p, smem, grid, s)
                 : launch_one<FMT, 1, IN, OUT, false, NB, true>(p, smem, grid, s);
}

template <int FMT, int IN, int OUT>
int dispatch_depth(const ProjParams &p, bool exact, int depth, size_t smem, unsigned grid, hipStream_t s)
{
    switch (depth) {
    case 1: return dispatch_exact<FMT, IN, OUT, 1>(p, exact, smem, grid, s);
    case 2: return dispatch_exact<FMT, IN, OUT, 2>(p, exact, smem, grid, s);
    case 4: return dispatch_exact<FMT, IN, OUT, 4>(p, exact, smem, grid, s);
    default: return dispatch_exact<FMT, IN, OUT, 8>(p, exact, smem, grid, s);
    }
}

// The query workgroups stream a whole head (D rows): one batch of up to 16 chunks per wave. In
// the exact order (a normed row) they write their chunk's scores instead of attending over it.
template <int FMT, int IN, int HD, bool EXACT>
int dispatch_qattn_depth(const ProjParams &p, int depth, size_t smem, unsigned grid, hipStream_t s)
{
    return depth <= 1 ? launch_one<FMT, 1, IN, OUT_QATTN, EXACT, 1, !EXACT, HD>(p, smem, grid, s)
                      : launch_one<FMT, 1, IN, OUT_QATTN, EXACT, 16, !EXACT, HD>(p, smem, grid, s);
}

// The query heads of a normed row, or (IN_EMBED, the first layer) of a table row normed.
template <int FMT, int IN, bool EXACT>
int dispatch_qattn_in(const ProjParams &p, int depth, size_t smem, unsigned grid, hipStream_t s)
{
    switch (p.D) {
    case 32: return dispatch_qattn_depth<FMT, IN, 32, EXACT>(p, depth, smem, grid, s);
    case 64: return dispatch_qattn_depth<FMT, IN, 64, EXACT>(p, depth, smem, grid, s);
    default: return dispatch_qattn_depth<FMT, IN, 128, EXACT>(p, depth, smem, grid, s);
    }
}

template <int FMT>
int dispatch_qattn(const ProjParams &p, int in, bool exact, int depth, size_t smem, unsigned grid, hipStream_t s)
{
    if (exact) return dispatch_qattn_in<FMT, IN_NORM, true>(p, depth, smem, grid, s);
    return in == IN_EMBED ? dispatch_qattn_in<FMT, IN_EMBED, false>(p, depth, smem, grid, s)
                          : dispatch_qattn_in<FMT, IN_NORM, false>(p, depth, smem, grid, s);
}

template <int FMT>
int dispatch_attn(const ProjParams &p, int depth, size_t smem, unsigned grid, hipStream_t s)
{
    switch (depth) {  // the merge is the parallel-order attention's
    case 1: return launch_one<FMT, 1, IN_ATTN, OUT_STORE, false, 1, true>(p, smem, grid, s);
    case 2: return launch_one<FMT, 1, IN_ATTN, OUT_STORE, false, 2, true>(p, smem, grid, s);
    case 4: return launch_one<FMT, 1, IN_ATTN, OUT_STORE, false, 4, true>(p, smem, grid, s);
    default: return launch_one<FMT, 1, IN_ATTN, OUT_STORE, false, 8, true>(p, smem, grid, s);
    }
}


// The launch of proj_kernel for the decoder's input and output modes (the checks, grid, LDS size
// and batch depth come from launch_proj).
template <int FMT>
int launch_proj_format(const ProjParams &p, int in, int out, bool exact, int nb, size_t smem, unsigned grid, hipStream_t s)
{
    switch (out) {
    case OUT_QKV: return dispatch_depth<FMT, IN_NORM, OUT_QKV>(p, exact, nb, smem, grid, s);
    case OUT_SWIGLU: return dispatch_depth<FMT, IN_NORM, OUT_SWIGLU>(p, exact, nb, smem, grid, s);
    case OUT_QATTN: return dispatch_qattn<FMT>(p, in, exact, nb, smem, grid, s);
    default:
        if (in == IN_NORM) return dispatch_depth<FMT, IN_NORM, OUT_STORE>(p, exact, nb, smem, grid, s);
        if (in == IN_F32) return dispatch_depth<FMT, IN_F32, OUT_STORE>(p, exact, nb, smem, grid, s);
        if (in == IN_ATTN) return dispatch_attn<FMT>(p, nb, smem, grid, s);
        return dispatch_depth<FMT, IN_PREQ, OUT_STORE>(p, exact, nb, smem, grid, s);
    }
}

}  // namespace
}  // namespace fg
