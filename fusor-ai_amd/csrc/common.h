// Shared definitions of the MI355X (gfx950) quantized matrix-product library.
//
// Device layout of a table (the device mirror of a fusor-ai Table, tensor.rs:1-9). The host hands
// over the reference bytes (quad-major codes, then f32 scales); the upload rewrites the codes so
// that every kernel reads a row's codes of one 32-input block contiguously:
//   * quad q (rows 4q..4q+3), block b: a "quad block" of 4 row-blocks, [lane][codes];
//   * Q7b32 / Q8b32: 32 signed int8 levels per row-block (Q7b32 stores u - 64, so the
//     correction -64·Σa is folded into the levels: Σ(u-64)·a == corr + Σu·a exactly);
//   * Q4b32: 16 bytes per row-block, byte i holding code i in its low nibble and code i + 16 in
//     its high nibble, offset-binary as the reference stores them (u = q + 8);
//   * scales: unchanged, f32 at ((q·G + g)·4 + lane).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/fusor_gpu.h"

namespace fg {

constexpr int kBlock = 32;
constexpr int kQuad = 4;
constexpr int kTernaryGroup = 128;

inline int group_of(int dtype) { return dtype == FG_T2B128 ? kTernaryGroup : kBlock; }
inline int zero_point_of(int dtype)
{
    switch (dtype) {
    case FG_Q7B32: return 64;
    case FG_Q4B32: return 8;
    case FG_T2B128: return 1;
    default: return 0;
    }
}
inline int codes_per_byte(int dtype) { return dtype == FG_Q4B32 ? 2 : dtype == FG_T2B128 ? 4 : 1; }
inline bool is_quantized(int dtype) { return dtype >= FG_Q7B32 && dtype <= FG_Q8B32; }
// Bytes of one quad block in the reference layout (tensor.rs:129): 128 / 64 / 32.
inline size_t quad_bytes(int dtype) { return size_t(kQuad * kBlock / codes_per_byte(dtype)); }
inline size_t padded_values(size_t rows, size_t cols) { return (rows + kQuad - 1) / kQuad * kQuad * cols; }

}  // namespace fg

struct fg_table {
    int dtype;
    size_t rows, cols;
    size_t quads, blocks, groups;
    int8_t *codes;   // device layout, quads * blocks * quad_bytes bytes
    float *scales;   // quads * groups * 4
    size_t code_bytes;
    // A run-time matrix (QuantizedMatrix): room for `capacity` rows of `max_cols` values; `rows`
    // and `cols` are the rows appended so far and the current width. 0 for a model's table.
    size_t capacity, max_cols;
};

namespace fg {

// ------------------------------------------------------------------ errors (host side)

int set_error(int code, const std::string &message);
int check_hip(hipError_t e, const char *what);

#define FG_HIP(call)                                                          \
    do {                                                                      \
        hipError_t fg_e_ = (call);                                            \
        if (fg_e_ != hipSuccess) return ::fg::check_hip(fg_e_, #call);        \
    } while (0)

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// ------------------------------------------------------------------ device helpers

typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int dot4(int a, int b, int acc) { return __builtin_amdgcn_sdot4(a, b, acc, false); }

// A workgroup barrier for pipelines of direct global-to-LDS loads. __syncthreads() carries a
// release fence, and that fence waits for every outstanding global load of the wave, the direct
// loads of later stages included, so a pipeline several stages deep would drain to one stage at
// each barrier. Here each wave first waits for its own loads of the stage it needs (an explicit
// vmcnt wait before the call); the barrier then publishes them, and the LDS reads of the stage
// before are complete (lgkmcnt(0)) before any wave refills its buffer.
__device__ __forceinline__ void stage_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// The partner lane's value in pairs (lane ^ 1), through DPP.
__device__ __forceinline__ int xor1(int v) { return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false); }
// lane ^ 2 within a quad, and the mirror lane within 8 (lane ^ 7), through DPP.
__device__ __forceinline__ int xor2(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false); }
__device__ __forceinline__ int mirror8(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false); }

// Reductions over aligned groups of 8 lanes (every lane gets the group's result): after the two
// quad steps each quad holds its own result, and the mirror exchanges the two quads.
__device__ __forceinline__ float max8(float v)
{
    v = fmaxf(v, __int_as_float(xor1(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(xor2(__float_as_int(v))));
    return fmaxf(v, __int_as_float(mirror8(__float_as_int(v))));
}
__device__ __forceinline__ int sum8(int v)
{
    v += xor1(v);
    v += xor2(v);
    return v + mirror8(v);
}
// The value of lane l ^ 8 within its row of 16 lanes (DPP row_ror:8).
__device__ __forceinline__ float xor8(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));
}
// The two rows of 16 lanes that lane l's row pairs with (lanes l and l ^ 16), at l's place in its
// row: .x the even row's value, .y the odd row's. A VALU lane swap (v_permlane16_swap), so
// x + y, or fmaxf(x, y), is the xor-16 exchange with the same operands in both lanes.
__device__ __forceinline__ float2 row_pair(float v)
{
    const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return make_float2(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
// ... and the two halves of 32 lanes (lanes l and l ^ 32): .x the lower half's, .y the upper's
__device__ __forceinline__ float2 half_pair(float v)
{
    const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return make_float2(__uint_as_float(q[0]), __uint_as_float(q[1]));
}

// Lane C of each quad of lanes, to every lane of its quad (DPP quad_perm [C, C, C, C]).
template <int C>
__device__ __forceinline__ float quad_broadcast_of(float x)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), C * 0x55, 0xF, 0xF, false));
}
// ... for a lane index that is a constant where the call is unrolled (0..3)
__device__ __forceinline__ float quad_broadcast(float x, int c)
{
    switch (c) {
    case 0: return quad_broadcast_of<0>(x);
    case 1: return quad_broadcast_of<1>(x);
    case 2: return quad_broadcast_of<2>(x);
    default: return quad_broadcast_of<3>(x);
    }
}

// Lane C of each row of 16 lanes, to every lane of its row (DPP row_newbcast).
template <int C>
__device__ __forceinline__ float row_broadcast_of(float x)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x150 + C, 0xF, 0xF, false));
}
// ... for a lane index that is a constant where the call is unrolled (0..7)
__device__ __forceinline__ float row_broadcast(float x, int c)
{
    switch (c) {
    case 0: return row_broadcast_of<0>(x);
    case 1: return row_broadcast_of<1>(x);
    case 2: return row_broadcast_of<2>(x);
    case 3: return row_broadcast_of<3>(x);
    case 4: return row_broadcast_of<4>(x);
    case 5: return row_broadcast_of<5>(x);
    case 6: return row_broadcast_of<6>(x);
    default: return row_broadcast_of<7>(x);
    }
}

// Maximum / sum over the wave of a value every lane holds, every lane getting the result: DPP
// within rows of 16 lanes, then lane swaps across the rows (no LDS or scalar round trips).
__device__ __forceinline__ float wave_allmax(float v)
{
    v = fmaxf(v, __int_as_float(xor1(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(xor2(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(mirror8(__float_as_int(v))));
    v = fmaxf(v, xor8(v));
    const float2 r = row_pair(v);
    v = fmaxf(r.x, r.y);
    const float2 h = half_pair(v);
    return fmaxf(h.x, h.y);
}
__device__ __forceinline__ float wave_allsum(float v)
{
    v = v + __int_as_float(xor1(__float_as_int(v)));
    v = v + __int_as_float(xor2(__float_as_int(v)));
    v = v + __int_as_float(mirror8(__float_as_int(v)));
    v = v + xor8(v);
    const float2 r = row_pair(v);
    v = r.x + r.y;
    const float2 h = half_pair(v);
    return h.x + h.y;
}

// Activation quantization of one value at scale d (scalar.rs:57-66): ties-to-even rounding of the
// IEEE quotient, clamped to ±127 in float, NaN to 0 (Rust's saturating cast).
__device__ __forceinline__ int quantize_level(float x, float d)
{
    float r = __builtin_rintf(x / d);
    if (r != r) return 0;
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    return int(r);
}

// `extreme == 0 ? 1 : extreme / level` (quant.rs:126-128).
__device__ __forceinline__ float group_scale(float extreme, float level) { return extreme == 0.0f ? 1.0f : extreme / level; }

// The levels of groups of 32 values (activation quantization, scalar.rs:48-66, arch/mod.rs:223-228)
// held by 8 aligned lanes, four values each, to the bit of the reference's IEEE arithmetic.
//
// A correctly rounded a / b costs about a dozen instructions: the compiler's expansion scales both
// operands (v_div_scale), refines a reciprocal of the scaled divisor, corrects the quotient with
// fused multiply-adds and undoes the scaling (v_div_fmas, v_div_fixup). The scaling is the identity
// unless an operand or the quotient is near the ends of the exponent range, so where it provably is,
// the same reciprocal and correction steps alone give the same quotient, and a divisor's
// reciprocal is shared by the values it divides:
//   d = amax / 127 for amax in [2^-52, 2^66];
//   x / d for d in [2^-60, 2^60] and |x| <= amax (|x / d| < 128): the scaling acts only when
//   |x / d| < 2^-43 or |x| < 2^-103, and those quotients are below 1/4, so their level is 0 either
//   way (the remainders of every larger quotient stay normal).
// Groups outside that range take the IEEE division itself.
__device__ __forceinline__ int level_of(float t)
{
    float r = __builtin_rintf(t);
    if (r != r) return 0;
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    return int(r);
}

// The reciprocal of b refined as the division expansion refines it (v_rcp_f32 then one step).
__device__ __forceinline__ float refined_reciprocal(float b)
{
    const float r0 = __builtin_amdgcn_rcpf(b);
    return __builtin_fmaf(__builtin_fmaf(-b, r0, 1.0f), r0, r0);
}
// a / b from the refined reciprocal r of b: the expansion's two correction steps.
__device__ __forceinline__ float corrected_quotient(float a, float b, float r)
{
    const float q = a * r;
    const float q1 = __builtin_fmaf(__builtin_fmaf(-b, q, a), r, q);
    return __builtin_fmaf(__builtin_fmaf(-b, q1, a), r, q1);
}
// The level of a quotient with |t| < 128 or NaN: v_cvt_i32_f32 converts NaN to 0, the reference's
// saturating cast; rounding ties to even first.
__device__ __forceinline__ int level_in_range(float t)
{
    int i;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(i) : "v"(__builtin_rintf(t)));
    return i;
}

// The scale amax / 127 of a group and the levels of four of its values, branching per lane.
__device__ __forceinline__ float scale_and_levels(float amax, float x0, float x1, float x2, float x3, int &l0, int &l1,
                                                  int &l2, int &l3)
{
    if (amax >= 0x1p-52f && amax <= 0x1p66f) {
        float c = 127.0f;
        asm("" : "+v"(c));  // the divisor's reciprocal from v_rcp_f32 at run time, as the expansion takes it
        const float d = corrected_quotient(amax, c, refined_reciprocal(c));
        const float r = refined_reciprocal(d);
        l0 = level_in_range(corrected_quotient(x0, d, r));
        l1 = level_in_range(corrected_quotient(x1, d, r));
        l2 = level_in_range(corrected_quotient(x2, d, r));
        l3 = level_in_range(corrected_quotient(x3, d, r));
        return d;
    }
    const float d = group_scale(amax, 127.0f);
    l0 = quantize_level(x0, d);
    l1 = quantize_level(x1, d);
    l2 = quantize_level(x2, d);
    l3 = quantize_level(x3, d);
    return d;
}

struct Group8 {
    int packed;  // this lane's four levels, lowest first
    int total;   // the sum of the group's 32 levels (every lane of the group)
    float d;     // the group's scale
};

// Maximum over aligned groups of 8 lanes of floats that are >= 0 and not NaN: their bits order as
// unsigned integers do, so one fused DPP integer maximum per step.
__device__ __forceinline__ float max8_nonneg(float v)
{
    unsigned u = __float_as_uint(v);
    u = max(u, unsigned(xor1(int(u))));
    u = max(u, unsigned(xor2(int(u))));
    return __uint_as_float(max(u, unsigned(mirror8(int(u)))));
}

// N groups at once (independent instruction streams the scheduler interleaves). Every lane of the
// wave runs it (the group reductions read neighbouring lanes); callers predicate the stores.
template <int N>
__device__ __forceinline__ void quantize_groups(const v4f *v, Group8 *out)
{
    float amax[N];
    bool fast = true;
#pragma unroll
    for (int n = 0; n < N; n++) {
        // fold(0, max |x|) with NaN ignored (f32::max): fmaxf keeps the non-NaN operand
        float a = fmaxf(fmaxf(fabsf(v[n].x), fabsf(v[n].y)), fmaxf(fabsf(v[n].z), fabsf(v[n].w)));
        amax[n] = max8_nonneg(fmaxf(a, 0.0f));
        fast = fast && amax[n] >= 0x1p-52f && amax[n] <= 0x1p66f;
    }
    // the shared-reciprocal path for every group, then (rarely) the IEEE division for groups outside
    // its range, so the range test is off the arithmetic's critical path
    int l[N][4];
    float c = 127.0f;
    asm("" : "+v"(c));  // the divisor's reciprocal from v_rcp_f32 at run time, as the expansion takes it
    const float r127 = refined_reciprocal(c);
#pragma unroll
    for (int n = 0; n < N; n++) {
        const float d = corrected_quotient(amax[n], c, r127);
        const float r = refined_reciprocal(d);
        out[n].d = d;
        l[n][0] = level_in_range(corrected_quotient(v[n].x, d, r));
        l[n][1] = level_in_range(corrected_quotient(v[n].y, d, r));
        l[n][2] = level_in_range(corrected_quotient(v[n].z, d, r));
        l[n][3] = level_in_range(corrected_quotient(v[n].w, d, r));
    }
    if (!__all(fast)) {
#pragma unroll
        for (int n = 0; n < N; n++) {
            if (!(amax[n] >= 0x1p-52f && amax[n] <= 0x1p66f)) {
                const float d = amax[n] == 0.0f ? 1.0f : amax[n] / 127.0f;
                out[n].d = d;
                l[n][0] = level_of(v[n].x / d);
                l[n][1] = level_of(v[n].y / d);
                l[n][2] = level_of(v[n].z / d);
                l[n][3] = level_of(v[n].w / d);
            }
        }
    }
#pragma unroll
    for (int n = 0; n < N; n++) {
        out[n].packed = (l[n][0] & 0xff) | ((l[n][1] & 0xff) << 8) | ((l[n][2] & 0xff) << 16) | ((l[n][3] & 0xff) << 24);
        out[n].total = sum8(l[n][0] + l[n][1] + l[n][2] + l[n][3]);
    }
}

// A group's levels, scale and correction (−zp · Σ levels) to staging arrays indexed by group.
__device__ __forceinline__ void store_group8(const Group8 &g, int zp, int grp, int8_t *q, float *scales, int32_t *corr)
{
    const int sub = threadIdx.x & 7;
    reinterpret_cast<int *>(q)[grp * 8 + sub] = g.packed;
    if (sub == 0) {
        scales[grp] = g.d;
        corr[grp] = -zp * g.total;
    }
}


// Pack four int8 levels into one dword, lowest first.
__device__ __forceinline__ int pack4(int a, int b, int c, int d)
{
    return (a & 0xff) | ((b & 0xff) << 8) | ((c & 0xff) << 16) | ((d & 0xff) << 24);
}

// One block of 32 values of a run-time Q7b32 matrix (QuantizedMatrix::set_block, matmul.rs:77-90):
// the scale absmax / 63 (1 for a zero block), the levels rint(x / scale) saturated to i8 and
// clamped to ±63, stored signed four to a dword (the device form u − 64 of the codes u).
__device__ __forceinline__ float q7_block(const float *x, int *dst)
{
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i]));
    const float scale = group_scale(amax, 63.0f);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        int l[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float v = __builtin_rintf(x[4 * i + j] / scale);
            const int level = v != v ? 0 : v >= 127.0f ? 127 : v <= -128.0f ? -128 : int(v);
            l[j] = level < -63 ? -63 : (level > 63 ? 63 : level);
        }
        dst[i] = pack4(l[0], l[1], l[2], l[3]);
    }
    return scale;
}

// Offset-binary nibbles (u in [0,15]) of a dword to signed levels u - 8, byte-wise without
// borrows: (u + 0x78) ^ 0x80 == u - 8 as an int8.
__device__ __forceinline__ int nibbles_signed(int packed_nibbles)
{
    return ((packed_nibbles & 0x0F0F0F0F) + 0x78787878) ^ int(0x80808080u);
}

}  // namespace fg

// Host-side launchers shared between translation units.
namespace fg {
int launch_relayout(const uint8_t *ref_codes, fg_table *t, hipStream_t s);
int launch_unrelayout(const fg_table *t, uint8_t *ref_codes, hipStream_t s);
// Reference quad blocks (whole ones, `bytes` long) to device quad blocks at the same offset.
int launch_relayout_range(const uint8_t *ref_codes, uint8_t *dev_codes, int dtype, size_t bytes, hipStream_t s);
// A table's device storage for a shape (codes and scales uninitialised), or an error.
int table_alloc(int dtype, size_t rows, size_t cols, fg_table **out);
size_t table_byte_len(int dtype, size_t rows, size_t cols);
int launch_encode(int dtype, size_t rows, size_t cols, const float *values, uint8_t *bytes, hipStream_t s);
int launch_dequantize_row(const fg_table *t, size_t row, float *out, hipStream_t s);
// The table's rows ids[0..count) (device ids) into out[count][cols].
int launch_embed_rows(const fg_table *t, const int32_t *ids, size_t count, float *out, hipStream_t s);
// quantize_rows for groups of 32 with the scales written block-major, as_t[g][Mpad] (zeros for the
// rows past `rows`), and no corrections: the form the batched product's kernels read.
int launch_quantize_rows_t(const float *x, size_t rows, size_t K, int dtype, int8_t *q, float *as_t, size_t Mpad,
                           hipStream_t s);
int launch_quantize_rows(const float *x, size_t count, int dtype, int8_t *q, float *scales, int32_t *corr,
                         hipStream_t s);
int launch_qmatrix_clear(fg_table *t, size_t first, size_t last, hipStream_t s);
int launch_qmatrix_set(fg_table *t, size_t first, size_t count, size_t b0, size_t nb, const float *values, size_t ld,
                       hipStream_t s);

// One product: rows of int8 levels (q, scales, corrections) or f32 rows x quantized in-kernel.
struct ProductArgs {
    const fg_table *t;
    const float *x;
    const int8_t *q;
    const float *as;
    const int32_t *corr;
    size_t rows;
    size_t quad_begin, quad_end;
    const float *bias;
    float *out;
    size_t ld_out;
    int accumulate;
    int32_t *dots;  // when set, the int32 group accumulators are written instead of out
    int fused;      // FG_FUSED_SCALE: s = fma((float)D, ws·as, s)
    int parallel;   // FG_PARALLEL_SUM: one row, group terms summed as a tree (the decoder's order)
    // scratch the caller provides (fg_matmul_noalloc): used instead of the workspace pool, never
    // allocated or freed; a product that needs more than `workspace_bytes` fails
    void *workspace;
    size_t workspace_bytes;
    // pre-quantized rows may bring their scales block-major as well ([G][as_t_rows], rows past
    // `rows` zero): a kernel that reads that form takes it instead of a transposed copy
    const float *as_t;
    size_t as_t_rows;
};
// Scratch bytes a product needs beyond its inputs and outputs (0 for the matrix-vector rows).
size_t product_scratch_bytes(const ProductArgs &a);
// A stream-ordered allocation from this device's workspace pool (kept across calls).
hipError_t workspace_alloc(void **ptr, size_t bytes, hipStream_t s);
int launch_matvec(const ProductArgs &a, hipStream_t s);
int launch_gemm(const ProductArgs &a, hipStream_t s);
// `items` products of pre-quantized rows of one shape in one launch (the staged kernel): item z's
// levels, scales and outputs at z times the strides (elements) from a's, and its table's codes
// and scales (z + first) / per_table − first / per_table tables on from a.t's.
int launch_gemm_batch(const ProductArgs &a, int items, int per_table, int first, size_t q_stride, size_t as_stride,
                      size_t out_stride, size_t codes_stride, size_t scales_stride, hipStream_t s);
int launch_t2(const ProductArgs &a, hipStream_t s);
int launch_product(const ProductArgs &a, hipStream_t s);
// Two products of the same pre-quantized rows over tables of one shape (a layer's gate and up):
// one launch when both take the same kernel, else one each.
int launch_product_pair(const ProductArgs &a, const ProductArgs &b, hipStream_t s);
}  // namespace fg
