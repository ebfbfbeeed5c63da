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
// 32 or 32 x 64 output tile (one or two MFMAs per block) and keeps the running f32 sums in
// registers; the K loop walks the blocks in order, so the sums are the reference's to the bit.
//
// MFMA operand layout (32x32xK): lane l feeds row (or column) l % 32 and K-half l / 32; the same
// K positions are used for both operands, so the sum covers the block's 32 inputs. Result:
// lane l holds column l % 32, rows 8·(v/4) + 4·(l/32) + v%4 for v = 0..15.
#include "common.h"

#include <cstdint>
#include <cstdlib>
#include <mutex>
#include <type_traits>
#include <vector>

namespace fg {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

struct GemmParams {
    const int8_t *codes;
    const float *wscales;
    int B, G, K;
    int M, Mpad;
    int col_begin, col_end;
    int n_rows;
    const int8_t *q;      // [M][K] levels
    const float *as;      // [M][G] activation scales (row-major, 16-byte rows: staged in LDS)
    const float *as_t;    // [G][Mpad] the same, block-major (when not staged)
    const float *bias;
    float *out;
    long ld_out;
    int accumulate;
    int32_t *dots;
    int dots_cols;
    // a batch of products (the staged kernel's grid y): item z takes the levels, scales and outputs
    // z items on (strides in elements) and table z / per_table's codes and scales
    long q_batch, as_batch, out_batch, codes_batch, wscales_batch;
    // a second product of the same rows in the same launch (the split kernel): workgroups from
    // tiles1 on take this table and output instead (gate and up of one input)
    const int8_t *codes2;
    const float *wscales2;
    float *out2;
    int tiles1;
    int per_table, first;  // item z's table: (z + first) / per_table − first / per_table on
};

// Workgroups in launch order go round-robin to the 8 XCDs, each with its own L2, so neighbouring
// tiles (which share activation rows or weight columns) would land on different L2s. The tile of
// launch index L is renumbered so that each XCD takes a contiguous run of tiles, and the runs
// are laid over the [Y row tiles][X column tiles] grid in groups of kGroupRows row tiles, row
// tile fastest: the waves resident on one XCD at a time share a few weight columns and a band
// of activation rows in its L2. A bijection of [0, X·Y).
constexpr int kGroupRows = 16;

__device__ __forceinline__ void tile_of(int L, int X, int Y, int &tx, int &ty)
{
    const int T = X * Y, per = T >> 3, rem = T & 7, xcd = L & 7, j = L >> 3;
    const int t = xcd < rem ? xcd * (per + 1) + j : rem * (per + 1) + (xcd - rem) * per + j;
    const int g = t / (kGroupRows * X), rows = min(kGroupRows, Y - g * kGroupRows), in = t - g * kGroupRows * X;
    ty = g * kGroupRows + in % rows;
    tx = in / rows;
}

// Activation scales of a tile's rows, transposed to [block][row] in LDS: this thread's row
// `srow` (row-major, whole float4s), float4s c = part, part + parts, ... of n4. Eight loads go
// out before their writes, so a pass waits for memory once rather than once per float4.
template <int ROWS>
__device__ __forceinline__ void stage_scales(float *tile_scales, const float *srow, int n4, int part, int parts, int row_in_tile)
{
    for (int c0 = part; c0 < n4; c0 += 8 * parts) {
        v4f v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = *reinterpret_cast<const v4f *>(srow + 4 * min(c0 + u * parts, n4 - 1));
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int c = c0 + u * parts;
            if (c < n4) {
                tile_scales[(4 * c) * ROWS + row_in_tile] = v[u].x;
                tile_scales[(4 * c + 1) * ROWS + row_in_tile] = v[u].y;
                tile_scales[(4 * c + 2) * ROWS + row_in_tile] = v[u].z;
                tile_scales[(4 * c + 3) * ROWS + row_in_tile] = v[u].w;
            }
        }
    }
}

// One wave per workgroup and per 32 x 32·TN output tile (TN MFMAs per block): enough waves to
// spread the exact rescale, four VALU operations per output per block and the product's bound,
// over every SIMD. Operands stream straight from memory, kDepth blocks ahead of the block being
// multiplied (a ring of registers); rows and columns past the edges re-read the last valid one.
constexpr int kDepth = 4;

template <int TN, bool LDS_SCALES>
struct Stage {
    v4i a;        // this lane's 16 activation levels
    v4i w[TN];    // 16 weight levels (or 32 packed nibbles) of this lane's column in each sub-tile
    float ws[TN]; // the weight scale of those columns
    v4f s0, s1, s2, s3;  // activation scales of this lane's 16 rows (when not staged in LDS)
};

// LDS_SCALES: the tile's activation scales for every block staged in LDS once (32 floats per
// block), so that the ring of registers holds operands only (more waves per SIMD).
template <int FMT, int TN, bool DOTS, bool LDS_SCALES, bool FUSED>
__global__ __launch_bounds__(64) void gemm_kernel(GemmParams p)
{
    extern __shared__ __align__(16) float tile_scales[];  // [B][32] when LDS_SCALES
    constexpr int QB = FMT == 8 ? 128 : 64;  // device bytes per quad block
    const int lane = threadIdx.x, i = lane & 31, h = lane >> 5;
    int tx, ty;
    tile_of(int(blockIdx.x), (p.col_end - p.col_begin + 32 * TN - 1) / (32 * TN), (p.M + 31) / 32, tx, ty);
    const int m0 = ty * 32, n0 = p.col_begin + tx * 32 * TN;
    const int row = min(m0 + i, p.M - 1);
    const int8_t *arow = p.q + size_t(row) * p.K + h * 16;
    const float *asrow = p.as_t + m0 + 4 * h;
    const int8_t *wrow[TN];
    const float *wsrow[TN];
#pragma unroll
    for (int t = 0; t < TN; t++) {
        const int nc = min(n0 + 32 * t + i, p.col_end - 1);
        wrow[t] = p.codes + size_t(nc >> 2) * p.B * QB + (nc & 3) * (QB / 4) + (FMT == 8 ? h * 16 : 0);
        wsrow[t] = p.wscales + size_t(nc >> 2) * p.G * 4 + (nc & 3);
    }
    const int B = p.B;
    if (LDS_SCALES) {
        // rows m0 .. m0 + 31 of as (rows past M re-read the last), transposed to [block][row]:
        // lane l reads four blocks of row l % 32 and writes them to four consecutive-row slots
        stage_scales<32>(tile_scales, p.as + size_t(min(m0 + i, p.M - 1)) * p.G, B / 4, h, 2, i);
        __syncthreads();
    }

    auto fetch = [&](int b, Stage<TN, LDS_SCALES> &st) {
        st.a = *reinterpret_cast<const v4i *>(arow + b * 32);
#pragma unroll
        for (int t = 0; t < TN; t++) {
            st.w[t] = *reinterpret_cast<const v4i *>(wrow[t] + size_t(b) * QB);
            st.ws[t] = wsrow[t][size_t(b) * 4];
        }
        if (!LDS_SCALES) {
            const float *ap = asrow + size_t(b) * p.Mpad;
            st.s0 = *reinterpret_cast<const v4f *>(ap);
            st.s1 = *reinterpret_cast<const v4f *>(ap + 8);
            st.s2 = *reinterpret_cast<const v4f *>(ap + 16);
            st.s3 = *reinterpret_cast<const v4f *>(ap + 24);
        }
    };

    float acc[TN][16];
#pragma unroll
    for (int t = 0; t < TN; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[t][v] = 0.0f;

    // The product of a block (TN MFMAs) is issued one block ahead of its rescale, so that the
    // matrix cores work on block b + 1 while the VALU scales block b, within one wave.
    struct Prod {
        v16i d[TN];
    };
    auto product = [&](const Stage<TN, LDS_SCALES> &st, Prod &pr) {
#pragma unroll
        for (int t = 0; t < TN; t++) {
            v4i w = st.w[t];
            if (FMT == 4) {
                const int sh = h * 4;
                w = v4i{nibbles_signed(w.x >> sh), nibbles_signed(w.y >> sh), nibbles_signed(w.z >> sh), nibbles_signed(w.w >> sh)};
            }
            const v16i zero = {0};
            pr.d[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(st.a, w, zero, 0, 0, 0);
        }
    };
    auto rescale = [&](int b, const Stage<TN, LDS_SCALES> &st, const Prod &pr) {
        v4f s0 = st.s0, s1 = st.s1, s2 = st.s2, s3 = st.s3;
        if (LDS_SCALES) {
            const v4f *ls = reinterpret_cast<const v4f *>(tile_scales + b * 32 + 4 * h);
            s0 = ls[0];
            s1 = ls[2];
            s2 = ls[4];
            s3 = ls[6];
        }
        const float sc[16] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w, s2.x, s2.y, s2.z, s2.w, s3.x, s3.y, s3.z, s3.w};
#pragma unroll
        for (int t = 0; t < TN; t++) {
            const v16i d = pr.d[t];
            if (DOTS) {
                const int n = n0 + 32 * t + i;
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int r = m0 + 8 * (v >> 2) + 4 * h + (v & 3);
                    if (r < p.M && n < p.col_end) p.dots[(size_t(r) * p.dots_cols + (n - p.col_begin)) * p.G + b] = d[v];
                }
                continue;
            }
#pragma unroll
            for (int v = 0; v < 16; v++)
                acc[t][v] = FUSED ? __builtin_fmaf(float(d[v]), st.ws[t] * sc[v], acc[t][v])
                                  : acc[t][v] + float(d[v]) * (st.ws[t] * sc[v]);
        }
    };

    // the ring: block b lives in stage b % kDepth; the fetch of block b + kDepth follows the
    // rescale of block b (clamped at the last block, so the loop body has no branch around
    // loads). Scheduling barriers keep each stage's work below the waits of younger loads.
    static_assert(kDepth % 2 == 0, "two products in flight alternate with the block's parity");
    Stage<TN, LDS_SCALES> st[kDepth];
#pragma unroll
    for (int k = 0; k < kDepth; k++) {
        fetch(min(k, B - 1), st[k]);
        __builtin_amdgcn_sched_barrier(0);
    }
    Prod pr[2];
    product(st[0], pr[0]);
    for (int b = 0; b < B; b += kDepth) {
#pragma unroll
        for (int k = 0; k < kDepth; k++) {
            product(st[(k + 1) % kDepth], pr[(k + 1) & 1]);  // block b + k + 1 (a clamped re-read past the end)
            if (k == 0 || b + k < B) rescale(b + k, st[k], pr[k & 1]);
            fetch(min(b + k + kDepth, B - 1), st[k]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (DOTS) return;
#pragma unroll
    for (int t = 0; t < TN; t++) {
        const int n = n0 + 32 * t + i;
        if (n >= p.col_end) continue;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int r = m0 + 8 * (v >> 2) + 4 * h + (v & 3);
            if (r >= p.M) continue;
            float *o = p.out + size_t(r) * p.ld_out + (n - p.col_begin);
            float y = acc[t][v];
            if (p.bias && n < p.n_rows) y = y + p.bias[n];
            *o = p.accumulate ? *o + y : y;
        }
    }
}

// Four waves per 32 x 32 output tile, for products with too few tiles to give every SIMD a wave
// of the kernel above. The exact order fixes only the additions: the terms
// fl(fl((float)D_g) · fl(ws · as)) of different groups are independent. Wave w takes groups
// w, w + 4, w + 8, ... (its own operands, its own ring of loads), forms its group's 1024 terms
// and writes them to LDS; after one barrier per round of four groups, wave q adds the round's
// four terms in group order to its quarter of the tile's sums (rows 8q + 4·(l/32) + 0..3 of
// the MFMA layout). Every sum sees the reference's additions in the reference's order; the
// rescale's VALU work and the operand waits spread over four SIMDs. Terms live in two buffers
// (round parity): a wave writes round r + 2 only after the barrier of round r + 1, which every
// wave reaches after reading round r.
//
// The scale products fl(ws · as) of a wave's two rounds r, r + 1 (r even) come from one f32
// outer product (v_mfma_f32_32x32x1_2b: lanes 0..31 give round r's row and column scales, lanes
// 32..63 round r + 1's), in the layout of the int8 products: exactly the VALU's rounded products,
// and one scale per lane instead of sixteen LDS reads and multiplies per round. STAGE: the tile's
// activation scales are staged in LDS first (deep products: 1024 x 4864 -> 896 38.5 against 42.5
// us for row-major reads in the ring); else each lane reads its row's scale with the operands
// (K = 896: 512 x 896 -> 896 6.7 against 7.3 us).
constexpr int kSplitDepth = 2;  // rounds each wave's ring of operands runs ahead (one pair)

template <int FMT, bool STAGE>
__global__ __launch_bounds__(256) void gemm_split_kernel(GemmParams p)
{
    extern __shared__ __align__(16) float split_lds[];  // [2][4][4][64] v4f terms, then [B][32] scales
    constexpr int QB = FMT == 8 ? 128 : 64;
    const int B = p.B;
    v4f *terms = reinterpret_cast<v4f *>(split_lds);
    float *tile_scales = split_lds + 2 * 4 * 4 * 64 * 4;
    const int tid = threadIdx.x, lane = tid & 63, i = lane & 31, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int L = int(blockIdx.x);
    if (p.codes2 && L >= p.tiles1) {  // the launch's second product (uniform per workgroup)
        L -= p.tiles1;
        p.codes = p.codes2;
        p.wscales = p.wscales2;
        p.out = p.out2;
    }
    int tx, ty;
    tile_of(L, (p.col_end - p.col_begin + 31) / 32, (p.M + 31) / 32, tx, ty);
    const int m0 = ty * 32, n0 = p.col_begin + tx * 32;
    const int row = min(m0 + i, p.M - 1);
    const int8_t *arow = p.q + size_t(row) * p.K + h * 16;
    const float *asrow = p.as + size_t(row) * p.G;
    const int nc = min(n0 + i, p.col_end - 1);
    const int8_t *wrow = p.codes + size_t(nc >> 2) * B * QB + (nc & 3) * (QB / 4) + (FMT == 8 ? h * 16 : 0);
    const float *wsrow = p.wscales + size_t(nc >> 2) * p.G * 4 + (nc & 3);
    // rows m0 .. m0 + 31 of as, transposed to [block][row] (rows past M re-read the last)
    if (STAGE) stage_scales<32>(tile_scales, asrow, B / 4, tid >> 5, 8, i);
    struct Op {
        v4i a, w;
        float ws, as;
    };
    // Round r of this wave: group 4r + wave's operands, and the scales this lane's half gives the
    // outer product of the round's pair, group 4((r & ~1) + h) + wave. Past the last block:
    // clamped re-reads, never used.
    auto fetch = [&](int r, Op &o) {
        const int b = min(4 * r + wave, B - 1), bh = min(4 * ((r & ~1) + h) + wave, B - 1);
        o.a = *reinterpret_cast<const v4i *>(arow + b * 32);
        o.w = *reinterpret_cast<const v4i *>(wrow + size_t(b) * QB);
        o.ws = wsrow[size_t(bh) * 4];
        if (!STAGE) o.as = asrow[bh];
    };
    Op ring[kSplitDepth];
#pragma unroll
    for (int k = 0; k < kSplitDepth; k++) {
        fetch(k, ring[k]);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (STAGE) __syncthreads();  // the scales
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // The products of round r + 1 (this wave's group 4(r + 1) + wave; B is a multiple of 4, the
    // launch checks it) are issued between the barrier of round r and round r's additions, so
    // their latencies overlap; so is the outer product of the next pair, at its first round.
    v16i d;
    v32f pp;  // the pair's scale products: round r's at [16 (r & 1) + v], laid out as d
    // this lane's activation scale for the outer product of the pair that starts at round r
    auto pair_as = [&](int r, const Op &o) { return STAGE ? tile_scales[min(4 * (r + h) + wave, B - 1) * 32 + i] : o.as; };
    auto issue = [&](const Op &o, auto first_of_pair, float asv) {
        if constexpr (decltype(first_of_pair)::value) {
            const v32f zero32 = {0};
            pp = __builtin_amdgcn_mfma_f32_32x32x1f32(asv, o.ws, zero32, 0, 0, 0);
        }
        v4i w = o.w;
        if (FMT == 4) {
            const int sh = h * 4;
            w = v4i{nibbles_signed(w.x >> sh), nibbles_signed(w.y >> sh), nibbles_signed(w.z >> sh), nibbles_signed(w.w >> sh)};
        }
        const v16i zero = {0};
        d = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a, w, zero, 0, 0, 0);
        asm volatile("" : "+v"(d));  // keeps the product here rather than sunk to its first use
    };
    // round r (parity P): its terms to LDS, `o` refilled with round r + 2, the barrier, then the
    // round's four groups added in order to this wave's quarter of the outputs. The next pair's
    // activation scale is read before the barrier, so that after it the term reads go out first
    // and the products follow without waiting on LDS.
    auto round = [&](int r, Op &o, const Op &o_next, auto parity) {
        constexpr int P = decltype(parity)::value;
        const float asn = P == 1 ? pair_as(r + 1, o_next) : 0.0f;
        v4f *buf = terms + P * (4 * 4 * 64);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int v = 4 * q;
            buf[(wave * 4 + q) * 64 + lane] = v4f{float(d[v]) * pp[16 * P + v], float(d[v + 1]) * pp[16 * P + v + 1],
                                                  float(d[v + 2]) * pp[16 * P + v + 2], float(d[v + 3]) * pp[16 * P + v + 3]};
        }
        fetch(r + kSplitDepth, o);
        __syncthreads();
        const v4f t0 = buf[wave * 64 + lane], t1 = buf[(4 + wave) * 64 + lane], t2 = buf[(8 + wave) * 64 + lane],
                  t3 = buf[(12 + wave) * 64 + lane];
        __builtin_amdgcn_sched_barrier(0);
        issue(o_next, std::integral_constant<bool, P == 1>{}, asn);
        __builtin_amdgcn_sched_barrier(0);  // the products go out before the additions wait
        acc[0] = acc[0] + t0.x + t1.x + t2.x + t3.x;
        acc[1] = acc[1] + t0.y + t1.y + t2.y + t3.y;
        acc[2] = acc[2] + t0.z + t1.z + t2.z + t3.z;
        acc[3] = acc[3] + t0.w + t1.w + t2.w + t3.w;
    };
    // whole pairs of rounds without a branch (the load counts the compiler waits on stay exact),
    // then an odd last round
    const int rounds = B / 4;
    issue(ring[0], std::true_type{}, pair_as(0, ring[0]));
    int r0 = 0;
    for (; r0 + 2 <= rounds; r0 += 2) {
        round(r0, ring[0], ring[1], std::integral_constant<int, 0>{});
        __builtin_amdgcn_sched_barrier(0);
        round(r0 + 1, ring[1], ring[0], std::integral_constant<int, 1>{});
        __builtin_amdgcn_sched_barrier(0);
    }
    if (r0 < rounds) round(r0, ring[0], ring[1], std::integral_constant<int, 0>{});
    const int n = n0 + i;
    if (n >= p.col_end) return;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int r = m0 + 8 * wave + 4 * h + e;
        if (r >= p.M) continue;
        float *o = p.out + size_t(r) * p.ld_out + (n - p.col_begin);
        float y = acc[e];
        if (p.bias && n < p.n_rows) y = y + p.bias[n];
        *o = p.accumulate ? *o + y : y;
    }
}

// LDS of gemm_split_kernel: the two term buffers, and the tile's activation scales when staged
// (products over more than 64 blocks).
inline bool split_stages(int B) { return B > 64; }
inline size_t split_lds_bytes(int B) { return 2 * 4 * 4 * 64 * 16 + (split_stages(B) ? size_t(B) * 32 * 4 : 0); }

template <int FMT>
void launch_split(const GemmParams &p, unsigned groups, hipStream_t s)
{
    if (split_stages(p.B)) gemm_split_kernel<FMT, true><<<dim3{groups}, 256, split_lds_bytes(p.B), s>>>(p);
    else gemm_split_kernel<FMT, false><<<dim3{groups}, 256, split_lds_bytes(p.B), s>>>(p);
}

// At most 16 rows: v_mfma_i32_16x16x32_i8, one wave per 16 x 16 tile. Weights, their scales and
// the activations run kDepthW blocks ahead in rings of registers (loads complete in order, so
// the activations' ring is as deep as the weights'). Deeper rings measured slower: the 16
// activation rows of every block cost a cache line each per wave, and that request rate, not
// the bytes in flight, bounds this shape. Operand layout (16x16x32): lane l feeds row (or column) l % 16 with inputs
// 8·(l/16) .. +7 of the block; result: lane l holds column l % 16, rows 4·(l/16) + v, v = 0..3.
constexpr int kDepthW = 8, kDepthA = 8;

template <int FMT, bool DOTS, bool FUSED>
__global__ __launch_bounds__(64) void gemm16_kernel(GemmParams p)
{
    extern __shared__ __align__(16) float tile_scales[];  // [B][16]
    constexpr int QB = FMT == 8 ? 128 : 64;
    const int lane = threadIdx.x, i = lane & 15, s = lane >> 4;  // s: this lane's slice of 8 inputs
    int tx, ty;
    tile_of(int(blockIdx.x), (p.col_end - p.col_begin + 15) / 16, (p.M + 15) / 16, tx, ty);
    const int m0 = ty * 16, n0 = p.col_begin + tx * 16;
    const int row = min(m0 + i, p.M - 1);
    const int n = n0 + i, nc = min(n, p.col_end - 1);
    const int B = p.B;
    const int8_t *arow = p.q + size_t(row) * p.K + 8 * s;
    // Q8 row-block: 32 levels; Q4: byte j holds inputs j and j + 16 in its nibbles
    const int8_t *wrow = p.codes + size_t(nc >> 2) * B * QB + (nc & 3) * (QB / 4) + (FMT == 8 ? 8 * s : 8 * (s & 1));
    const int shift = FMT == 8 ? 0 : 4 * (s >> 1);
    const float *wsrow = p.wscales + size_t(nc >> 2) * p.G * 4 + (nc & 3);
    if (!DOTS) {
        // the rows' scales, transposed to [block][row] (rows past M re-read the last)
        stage_scales<16>(tile_scales, p.as + size_t(row) * p.G, B / 4, s, 4, i);
        __syncthreads();
    }
    long rw[kDepthW], ra[kDepthA];
    float rs[kDepthW];
    // block by block, in the order the loop refills the ring: waiting for a block's operands then
    // leaves the younger blocks' loads in flight (vector loads complete in order)
    static_assert(kDepthA == kDepthW, "one ring");
#pragma unroll
    for (int k = 0; k < kDepthW; k++) {
        const int bb = min(k, B - 1);
        rw[k] = *reinterpret_cast<const long *>(wrow + size_t(bb) * QB);
        rs[k] = wsrow[size_t(bb) * 4];
        ra[k] = *reinterpret_cast<const long *>(arow + bb * 32);
        __builtin_amdgcn_sched_barrier(0);  // the scheduler would otherwise group the loads by array
    }
    __builtin_amdgcn_sched_barrier(0);
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int b = 0; b < B; b += kDepthW) {
#pragma unroll
        for (int k = 0; k < kDepthW; k++) {
            const int bb = b + k;
            // no branch around a block but for the dots: past the last block the operands are
            // clamped re-reads and the term is +0, which leaves the sum (never −0) as it is
            const bool live = bb < B;
            if (!DOTS || live) {
                long w = rw[k];
                if (FMT == 4) {
                    const int lo = nibbles_signed(int(w) >> shift), hi = nibbles_signed(int(w >> 32) >> shift);
                    w = long(unsigned(lo)) | (long(hi) << 32);
                }
                const v4i zero = {0, 0, 0, 0};
                const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(ra[k % kDepthA], w, zero, 0, 0, 0);
                if (DOTS) {
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const int r = m0 + 4 * s + v;
                        if (r < p.M && n < p.col_end) p.dots[(size_t(r) * p.dots_cols + (n - p.col_begin)) * p.G + bb] = d[v];
                    }
                } else {
                    const float ws = rs[k];
                    const v4f sc = *reinterpret_cast<const v4f *>(tile_scales + min(bb, B - 1) * 16 + 4 * s);
                    const float d0 = live ? float(d[0]) : 0.0f, d1 = live ? float(d[1]) : 0.0f;
                    const float d2 = live ? float(d[2]) : 0.0f, d3 = live ? float(d[3]) : 0.0f;
                    if (FUSED) {
                        acc[0] = __builtin_fmaf(d0, ws * sc.x, acc[0]);
                        acc[1] = __builtin_fmaf(d1, ws * sc.y, acc[1]);
                        acc[2] = __builtin_fmaf(d2, ws * sc.z, acc[2]);
                        acc[3] = __builtin_fmaf(d3, ws * sc.w, acc[3]);
                    } else {
                        acc[0] = acc[0] + d0 * (ws * sc.x);
                        acc[1] = acc[1] + d1 * (ws * sc.y);
                        acc[2] = acc[2] + d2 * (ws * sc.z);
                        acc[3] = acc[3] + d3 * (ws * sc.w);
                    }
                }
            }
            const int nw = min(bb + kDepthW, B - 1), na = min(bb + kDepthA, B - 1);
            rw[k] = *reinterpret_cast<const long *>(wrow + size_t(nw) * QB);
            rs[k] = wsrow[size_t(nw) * 4];
            ra[k % kDepthA] = *reinterpret_cast<const long *>(arow + na * 32);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (DOTS || n >= p.col_end) return;
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const int r = m0 + 4 * s + v;
        if (r >= p.M) continue;
        float *o = p.out + size_t(r) * p.ld_out + (n - p.col_begin);
        float y = acc[v];
        if (p.bias && n < p.n_rows) y = y + p.bias[n];
        *o = p.accumulate ? *o + y : y;
    }
}

// The LDS stage of the small-batch products over many columns (at most 16 rows): a workgroup owns
// 16 rows x 64 columns (16 quads, four 16 x 16 tiles). The operands of kStreamBlocks blocks (a
// stage) arrive by direct global-to-LDS loads (lane l of a load writes 16 bytes, or 4, at its
// base + 16·l, or 4·l), so kilobytes per workgroup are in flight with no register held for
// them. In every load four neighbouring lanes read one run of bytes (lanes that each touch
// another line cost the address unit a cycle apiece), and every layout spreads a wave's reads of
// a block over the banks:
//   W  [16 quads][kStreamBlocks][QB]  the quads' weight bytes, a quad's run of blocks being one run
//                                     of bytes in the table; a quad every WQ bytes;
//   WS [4 tiles][4 quads][16 slots][4] the weight scales of a quad's blocks, slot k holding block
//                                     k + 2·quad (mod 16): the four quads' reads of one block fall
//                                     on different banks;
//   A  [8 groups][16 rows][4][16 B]   the activation levels, group g holding bytes 64g .. 64g + 63
//                                     of each row's stage, row r's piece p at position p ^ (r/2 % 4):
//                                     the 16 rows' pieces of a block fall on eight bank offsets;
//   AS [4 groups][16 rows][4]         the activation scales, group j holding blocks 4j .. 4j + 3.
// Rows and columns past the edges re-read the last valid one; blocks past the last are loaded
// clamped (in bounds) and skipped. The arithmetic is gemm16_kernel's.
constexpr int kStreamBlocks = 16;

template <int FMT>
struct StreamTile {
    static constexpr int QB = FMT == 8 ? 128 : 64;             // device bytes per quad block
    static constexpr int WQ = kStreamBlocks * QB + 64;         // a quad's stage bytes, padded
    static constexpr int W_BYTES = 16 * WQ;
    static constexpr int WS_BYTES = 4 * kStreamBlocks * 4 * 16;
    static constexpr int A_BYTES = kStreamBlocks * 32 * 16;
    static constexpr int AS_BYTES = kStreamBlocks * 16 * 4;
    static constexpr int STAGE = W_BYTES + WS_BYTES + A_BYTES + AS_BYTES;
    static constexpr int W_LOADS = kStreamBlocks * QB / 1024;  // per quad
};

// Bands of 16 rows (the products of at most 16 rows, and of up to 256 over a long K) over many
// columns, two waves per 16 x 16 tile: a workgroup of eight waves owns one band's 16 rows over
// 64 columns (16 quads) with the LDS stages above, and tile t (quads 4t .. 4t + 3) has two
// waves. In each stage of kStreamBlocks blocks, wave t forms the products of blocks
// 0..7 and wave t + 4 those of blocks 8..15; wave t + 4 turns its products into the terms
// fl(fl(D)·fl(ws·as)) and hands them over through LDS, and after the next barrier wave t adds
// the stage's sixteen terms per output in group order (its own eight, then the eight handed
// over). With two waves per SIMD each hides the other's waits (one wave per SIMD leaves every
// LDS read and product latency exposed). The eight waves share each stage's direct loads
// evenly: two quads' weight bytes each, the weight scales (first waves) or the activation
// scales (second waves), and one group of the activation levels. Each wave waits for its own
// loads of a stage, then one barrier publishes the stage (and the terms handed over the stage
// before) and frees the buffer the next issue refills.
template <int FMT>
struct PairTile {
    using S = StreamTile<FMT>;
    static constexpr int HALF = kStreamBlocks / 2;             // blocks per wave and stage
    static constexpr int DEPTH = 2;                            // stages in LDS (measured: 3 slower)
    static constexpr int TERMS = 2 * 4 * HALF * 64 * 16;       // [2][4 tiles][HALF][64 lanes] v4f
    static constexpr int LOADS = 2 * S::W_LOADS + 2;           // per wave and stage
    static constexpr int LDS = DEPTH * S::STAGE + TERMS;
    static_assert(LDS <= 160 * 1024 && (DEPTH - 2) * LOADS < 64 && HALF % 4 == 0, "pair tile");
};

template <int FMT>
__global__ __launch_bounds__(512) void gemm16_pair_kernel(GemmParams p)
{
    using S = StreamTile<FMT>;
    using T = PairTile<FMT>;
    constexpr int QB = S::QB, WQ = S::WQ, DEPTH = T::DEPTH, KS = kStreamBlocks, HALF = T::HALF, kWLoads = S::W_LOADS;
    constexpr int kStage = S::STAGE, kW = S::W_BYTES, kWS = S::WS_BYTES, kA = S::A_BYTES;
    extern __shared__ __align__(16) unsigned char pair_lds[];  // [DEPTH][STAGE], then the handed terms
    v4f *const handed = reinterpret_cast<v4f *>(pair_lds + DEPTH * kStage);
    const int tid = threadIdx.x, lane = tid & 63, c = lane & 15, s = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tile = wave & 3, h = wave >> 2;  // h 0: blocks 0..7 and the sums; h 1: blocks 8..15
    int tx, ty;
    tile_of(int(blockIdx.x), (p.col_end - p.col_begin + 63) / 64, (p.M + 15) / 16, tx, ty);
    const int m0 = ty * 16, q0 = (p.col_begin >> 2) + tx * 16, last_quad = (p.col_end - 1) >> 2;
    const int B = p.B, G = p.G, K = p.K;
    const int stages = (B + KS - 1) / KS;

    auto issue = [&](int st, int buf) {
        unsigned char *base = pair_lds + buf * kStage;
        const int b0 = st * KS;
        // the weight bytes of quads 4·tile + 2h and 4·tile + 2h + 1
#pragma unroll
        for (int qq = 0; qq < 2; qq++) {
            const int ql = 4 * tile + 2 * h + qq;
            const int8_t *qbase = p.codes + size_t(min(q0 + ql, last_quad)) * B * QB;
#pragma unroll
            for (int j = 0; j < kWLoads; j++) {
                const int at = min(b0 * QB + (j * 64 + lane) * 16, B * QB - 16);
                __builtin_amdgcn_global_load_lds(qbase + at, base + ql * WQ + j * 1024, 16, 0, 0);
            }
        }
        if (h == 0) {
            // the tile's weight scales: lane l, quad 4·tile + l / 16, slot l % 16 (block slot +
            // 2·quad mod 16)
            const int qw = lane >> 4, slot = lane & 15;
            const int q = min(q0 + 4 * tile + qw, last_quad), blk = min(b0 + ((slot + 2 * qw) & 15), B - 1);
            __builtin_amdgcn_global_load_lds(p.wscales + (size_t(q) * G + blk) * 4, base + kW + tile * 1024, 16, 0, 0);
        } else {
            // activation scales of group `tile`: lane l, row l / 4, block 4·tile + l % 4
            const int row = min(m0 + (lane >> 2), p.M - 1), blk = min(b0 + 4 * tile + (lane & 3), B - 1);
            __builtin_amdgcn_global_load_lds(p.as + size_t(row) * G + blk, base + kW + kWS + kA + tile * 256, 4, 0, 0);
        }
        {
            // activation group g = wave: lane l, row r = l / 4, position l % 4 holding piece
            // (l % 4) ^ (r / 2 % 4)
            const int r = lane >> 2, piece = (lane & 3) ^ ((r >> 1) & 3);
            const int row = min(m0 + r, p.M - 1), at = min(b0 * 32 + (4 * wave + piece) * 16, K - 16);
            __builtin_amdgcn_global_load_lds(p.q + size_t(row) * K + at, base + kW + kWS + wave * 1024, 16, 0, 0);
        }
    };

    const int shift = FMT == 8 ? 0 : 4 * (s >> 1);
    const int w_off = (4 * tile + (c >> 2)) * WQ + (c & 3) * (QB / 4) + (FMT == 8 ? 8 * s : 8 * (s & 1));
    const int a_row = kW + kWS + c * 64 + 8 * (s & 1), sig = (c >> 1) & 3;
    const int a_off0 = a_row + ((s >> 1) ^ sig) * 16, a_off1 = a_row + ((2 + (s >> 1)) ^ sig) * 16;
    const int blk4 = lane >> 4, qi = c >> 2;
    const int as_off = kW + kWS + kA + (c * 4 + blk4) * 4;
    const int ws_row = kW + tile * 1024 + qi * 256 + (c & 3) * 4;
    struct Ops {
        long w[HALF], a[HALF];
        float as[HALF / 4], ws[HALF / 4];
    };
    struct Prods {
        v4i d[HALF];
        v16f p[HALF / 4];
    };
    // this wave's blocks HALF·h + j of the stage in `base`
    auto read = [&](const unsigned char *base, Ops &o) {
#pragma unroll
        for (int j = 0; j < HALF; j++) {
            const int b = HALF * h + j;
            o.w[j] = *reinterpret_cast<const long *>(base + w_off + b * QB);
            o.a[j] = *reinterpret_cast<const long *>(base + (j & 1 ? a_off1 : a_off0) + (b >> 1) * 1024);
        }
#pragma unroll
        for (int j = 0; j < HALF / 4; j++) {
            const int J = HALF / 4 * h + j;  // group of four blocks
            o.as[j] = *reinterpret_cast<const float *>(base + as_off + J * 256);
            o.ws[j] = *reinterpret_cast<const float *>(base + ws_row + ((4 * J + blk4 - 2 * qi) & 15) * 16);
        }
    };
    auto multiply = [&](const Ops &o, Prods &r) {
#pragma unroll
        for (int j = 0; j < HALF / 4; j++) {
            const v16f zero16 = {0};
            r.p[j] = __builtin_amdgcn_mfma_f32_16x16x1f32(o.as[j], o.ws[j], zero16, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < HALF; j++) {
            long x = o.w[j];
            if (FMT == 4) {
                const int lo = nibbles_signed(int(x) >> shift), hi = nibbles_signed(int(x >> 32) >> shift);
                x = long(unsigned(lo)) | (long(hi) << 32);
            }
            const v4i zero = {0, 0, 0, 0};
            r.d[j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(o.a[j], x, zero, 0, 0, 0);
        }
    };
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // the first wave's own terms of a stage, then the handed-over ones, in group order; in the
    // last stage blocks past the last are skipped (uniform branches, kept out of the loop)
    auto own = [&](const Prods &r, int live) {
#pragma unroll
        for (int j = 0; j < HALF; j++) {
            if (j < live) {
#pragma unroll
                for (int v = 0; v < 4; v++) acc[v] = acc[v] + float(r.d[j][v]) * r.p[j / 4][4 * (j % 4) + v];
            }
        }
    };
    auto theirs = [&](int buf, int live) {
        const v4f *t = handed + (buf * 4 + tile) * HALF * 64 + lane;
        v4f x[HALF];
#pragma unroll
        for (int j = 0; j < HALF; j++) x[j] = t[j * 64];
#pragma unroll
        for (int j = 0; j < HALF; j++) {
            if (j < live) {
                acc[0] = acc[0] + x[j].x;
                acc[1] = acc[1] + x[j].y;
                acc[2] = acc[2] + x[j].z;
                acc[3] = acc[3] + x[j].w;
            }
        }
    };
    auto hand_over = [&](const Prods &r, int buf) {
        v4f *t = handed + (buf * 4 + tile) * HALF * 64 + lane;
#pragma unroll
        for (int j = 0; j < HALF; j++) {
            v4f x;
#pragma unroll
            for (int v = 0; v < 4; v++) x[v] = float(r.d[j][v]) * r.p[j / 4][4 * (j % 4) + v];
            t[j * 64] = x;
        }
    };

#pragma unroll
    for (int k = 0; k < DEPTH - 1; k++)
        if (k < stages) issue(k, k);
    Prods prev;
    for (int st = 0; st < stages; st++) {
        // this wave's loads of stage st: the later stages issued so far may still be in flight
        if (st + DEPTH - 2 < stages) asm volatile("s_waitcnt vmcnt(%0)" ::"n"((DEPTH - 2) * T::LOADS) : "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        // every wave's loads of stage st and the terms of stage st - 1 handed over; every wave done
        // reading stage st - 1 and the terms of stage st - 2
        stage_barrier();
        if (st + DEPTH - 1 < stages) issue(st + DEPTH - 1, (st + DEPTH - 1) % DEPTH);
        Ops o;
        read(pair_lds + (st % DEPTH) * kStage, o);
        if (h == 0) {
            if (st > 0) {
                own(prev, HALF);  // stage st - 1 (whole), while the reads are in flight
                theirs((st - 1) & 1, HALF);
            }
            multiply(o, prev);
        } else {
            Prods mine;
            multiply(o, mine);
            hand_over(mine, st & 1);
        }
    }
    stage_barrier();  // the last stage's handed-over terms
    if (h != 0) return;
    const int live = B - (stages - 1) * KS;
    own(prev, live);
    theirs((stages - 1) & 1, live - HALF);
    const int n = p.col_begin + tx * 64 + tile * 16 + c;
    if (n >= p.col_end) return;
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const int r = m0 + 4 * s + v;
        if (r >= p.M) continue;
        float *out = p.out + size_t(r) * p.ld_out + (n - p.col_begin);
        float y = acc[v];
        if (p.bias && n < p.n_rows) y = y + p.bias[n];
        *out = p.accumulate ? *out + y : y;
    }
}

// At most 16 rows with too few 16 x 16 tiles for two waves per SIMD: four waves per tile, split
// over the groups as in gemm_split_kernel. Wave w forms the 256 terms of groups w, w + 4, ...
// (four per lane: rows 4·(l/16) + v of column l % 16), writes them to LDS, and after the round's
// barrier adds the round's four groups in order for output v = w of every lane.
template <int FMT>
__global__ __launch_bounds__(256) void gemm16_split_kernel(GemmParams p)
{
    extern __shared__ __align__(16) float split16_lds[];  // [B][16] scales, then [2][4][64] v4f terms
    constexpr int QB = FMT == 8 ? 128 : 64;
    const int B = p.B;
    float *tile_scales = split16_lds;
    v4f *terms = reinterpret_cast<v4f *>(split16_lds + B * 16);
    const int tid = threadIdx.x, lane = tid & 63, i = lane & 15, sl = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int tx, ty;
    tile_of(int(blockIdx.x), (p.col_end - p.col_begin + 15) / 16, (p.M + 15) / 16, tx, ty);
    const int m0 = ty * 16, n0 = p.col_begin + tx * 16;
    const int row = min(m0 + i, p.M - 1);
    const int n = n0 + i, nc = min(n, p.col_end - 1);
    const int8_t *arow = p.q + size_t(row) * p.K + 8 * sl;
    const int8_t *wrow = p.codes + size_t(nc >> 2) * B * QB + (nc & 3) * (QB / 4) + (FMT == 8 ? 8 * sl : 8 * (sl & 1));
    const int shift = FMT == 8 ? 0 : 4 * (sl >> 1);
    const float *wsrow = p.wscales + size_t(nc >> 2) * p.G * 4 + (nc & 3);
    stage_scales<16>(tile_scales, p.as + size_t(row) * p.G, B / 4, tid >> 4, 16, i);
    struct Op {
        long a, w;
        float ws;
    };
    auto fetch = [&](int g, Op &o) {
        const int b = min(g, B - 1);
        o.a = *reinterpret_cast<const long *>(arow + b * 32);
        o.w = *reinterpret_cast<const long *>(wrow + size_t(b) * QB);
        o.ws = wsrow[size_t(b) * 4];
    };
    Op ring[kSplitDepth];
#pragma unroll
    for (int k = 0; k < kSplitDepth; k++) {
        fetch(4 * k + wave, ring[k]);
        __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();  // the scales
    float acc = 0.0f;
    // round r (B is a multiple of 4: the launch checks it)
    auto round = [&](int r, Op &o) {
        const int g = 4 * r + wave;
        const v4f sc = *reinterpret_cast<const v4f *>(tile_scales + g * 16 + 4 * sl);
        long w = o.w;
        if (FMT == 4) {
            const int lo = nibbles_signed(int(w) >> shift), hi = nibbles_signed(int(w >> 32) >> shift);
            w = long(unsigned(lo)) | (long(hi) << 32);
        }
        const v4i zero = {0, 0, 0, 0};
        const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(o.a, w, zero, 0, 0, 0);
        const float ws = o.ws;
        v4f *buf = terms + (r & 1) * (4 * 64);
        buf[wave * 64 + lane] = v4f{float(d[0]) * (ws * sc.x), float(d[1]) * (ws * sc.y), float(d[2]) * (ws * sc.z),
                                    float(d[3]) * (ws * sc.w)};
        fetch(4 * (r + kSplitDepth) + wave, o);
        __syncthreads();
        const float *fb = reinterpret_cast<const float *>(buf);
        const float t0 = fb[(0 * 64 + lane) * 4 + wave], t1 = fb[(1 * 64 + lane) * 4 + wave],
                    t2 = fb[(2 * 64 + lane) * 4 + wave], t3 = fb[(3 * 64 + lane) * 4 + wave];
        acc = acc + t0 + t1 + t2 + t3;
    };
    const int rounds = B / 4;
    int r0 = 0;
    for (; r0 + kSplitDepth <= rounds; r0 += kSplitDepth) {
#pragma unroll
        for (int k = 0; k < kSplitDepth; k++) {
            round(r0 + k, ring[k]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int k = 0; k < kSplitDepth - 1; k++)
        if (r0 + k < rounds) round(r0 + k, ring[k]);
    const int r = m0 + 4 * sl + wave;
    if (n >= p.col_end || r >= p.M) return;
    float *o = p.out + size_t(r) * p.ld_out + (n - p.col_begin);
    float y = acc;
    if (p.bias && n < p.n_rows) y = y + p.bias[n];
    *o = p.accumulate ? *o + y : y;
}

// LDS-staged tiles for the products with many tiles (the 4096-row DiT block, 512-row prefill with
// wide outputs). A workgroup of four waves owns a (64·WM) x (64·WN) output tile; wave w owns the
// 32·WM x 32·WN sub-tile (w / 2, w % 2): WM x WN MFMA tiles of 32 x 32. The workgroup's operands
// for kStageBlocks blocks at a time (a stage) are staged in LDS once and read by every wave:
//   A  [kb][BM rows][32 B]   int8 activation levels (q, row-major [M][K]);
//   W  [kb][BN cols][32 B]   weight levels (Q8; Q4: [kb][BN cols][16 B] packed nibbles);
//   AS [kb][BM]              activation scales, from the block-major copy as_t [G][Mpad] (f32
//                            rows are quantized straight into it), or from the pre-quantized
//                            rows' own [M][G] scales by 4-byte loads;
//   WS [kb][BN/4 quads][4]   weight scales, the table's own order ((q·G + g)·4 + lane).
// Every stage arrives by direct global-to-LDS loads (global_load_lds_dwordx4: lane l writes 16 bytes
// at base + 16·l), so no register holds staged data and the loads take no VALU work. Two stage
// buffers: stage s + 1 is loaded while stage s is multiplied; one barrier per stage both publishes
// stage s and frees the buffer of stage s - 1. Rows and columns past the edges re-read the last
// valid one (in bounds, never stored); blocks past the last one are loaded clamped and skipped.
// Per block each wave issues its WM·WN MFMAs, then adds each output's term in group order, the
// reference's sum to the bit (or the NEON backend's fused form).
constexpr int kStageBlocks = 2;

template <int FMT, int WM, int WN>
struct LdsTile {
    static constexpr int BM = 64 * WM, BN = 64 * WN, KB = kStageBlocks;
    static constexpr int RB = FMT == 8 ? 32 : 16;  // bytes of a weight row-block on the device
    static constexpr int A_BYTES = KB * BM * 32, W_BYTES = KB * BN * RB, AS_BYTES = KB * BM * 4, WS_BYTES = KB * BN * 4;
    static constexpr int STAGE = A_BYTES + W_BYTES + AS_BYTES + WS_BYTES;
    static constexpr int A_LOADS = A_BYTES / 1024, W_LOADS = W_BYTES / 1024;
    static constexpr int AS_LANES = AS_BYTES / 16, WS_LANES = WS_BYTES / 16;  // 16 bytes per lane
    static_assert(A_BYTES % 1024 == 0 && W_BYTES % 1024 == 0 && AS_LANES <= 64 && WS_LANES <= 64, "stage shape");
};

template <int FMT, int WM, int WN, bool FUSED>
__global__ __launch_bounds__(256) void gemm_lds_kernel(GemmParams p)
{
    using T = LdsTile<FMT, WM, WN>;
    constexpr int BM = T::BM, BN = T::BN, KB = T::KB, RB = T::RB;
    constexpr int QB = FMT == 8 ? 128 : 64;  // device bytes per quad block
    extern __shared__ __align__(16) unsigned char stage_lds[];  // [2][STAGE]
    if (gridDim.y > 1) {  // item blockIdx.y of a batch
        const long z = blockIdx.y, zt = (z + p.first) / p.per_table - p.first / p.per_table;
        p.q += z * p.q_batch;
        p.as += z * p.as_batch;
        p.out += z * p.out_batch;
        p.codes += zt * p.codes_batch;
        p.wscales += zt * p.wscales_batch;
    }
    const int tid = threadIdx.x, lane = tid & 63, i = lane & 31, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int tx, ty;
    tile_of(int(blockIdx.x), (p.col_end - p.col_begin + BN - 1) / BN, (p.M + BM - 1) / BM, tx, ty);
    const int m0 = ty * BM, n0 = p.col_begin + tx * BN;
    const int B = p.B, G = p.G;
    const int stages = (B + KB - 1) / KB;
    const int last_col = p.col_end - 1;

    // The direct loads of stage s into buffer `buf`, spread over the four waves (uniform branches).
    // (Stage offsets are taken out of the lambda: a static member of the tile type used inside it
    // drops the kernel's host-side launch stub.)
    unsigned char *const w_lds = stage_lds + T::A_BYTES, *const as_lds = w_lds + T::W_BYTES, *const ws_lds = as_lds + T::AS_BYTES;
    constexpr int kStage = T::STAGE, kALoads = T::A_LOADS, kWLoads = T::W_LOADS, kASLanes = T::AS_LANES, kWSLanes = T::WS_LANES;
    constexpr int kASLoads4 = KB * BM / 64;  // 4-byte loads of the row-major scales per stage
    auto issue = [&](int s, int buf) {
        unsigned char *base = stage_lds + buf * kStage;
        const int boff = buf * kStage;
        const int g0 = s * KB;
        for (int k = wave; k < kALoads; k += 4) {
            constexpr int per = BM / 32;  // loads per block
            const int kb = k / per, r = (k - kb * per) * 32 + (lane >> 1);
            const int row = min(m0 + r, p.M - 1), blk = min(g0 + kb, B - 1);
            // row r's two 16-byte halves sit swapped when bit 2 of r is set: a wave's reads of
            // eight consecutive rows then touch 32 distinct banks
            __builtin_amdgcn_global_load_lds(p.q + size_t(row) * p.K + blk * 32 + ((lane ^ (lane >> 3)) & 1) * 16,
                                             base + k * 1024, 16, 0, 0);
        }
        for (int k = wave; k < kWLoads; k += 4) {
            const int8_t *src;
            if (FMT == 8) {
                constexpr int per = BN / 32;
                const int kb = k / per, c = min(n0 + (k - kb * per) * 32 + (lane >> 1), last_col), blk = min(g0 + kb, B - 1);
                src = p.codes + size_t(c >> 2) * B * QB + size_t(blk) * QB + (c & 3) * 32 + ((lane ^ (lane >> 3)) & 1) * 16;
            } else {
                constexpr int per = BN / 64;
                const int kb = k / per, c = min(n0 + (k - kb * per) * 64 + lane, last_col), blk = min(g0 + kb, B - 1);
                src = p.codes + size_t(c >> 2) * B * QB + size_t(blk) * QB + (c & 3) * 16;
            }
            __builtin_amdgcn_global_load_lds(src, w_lds + boff + k * 1024, 16, 0, 0);
        }
        if (p.as_t) {
            if (wave == 2 && lane < kASLanes) {
                // four rows' scales of one block per lane: as_t [G][Mpad], Mpad a multiple of BM
                const int kb = lane / (BM / 4), r = (lane - kb * (BM / 4)) * 4, blk = min(g0 + kb, B - 1);
                __builtin_amdgcn_global_load_lds(p.as_t + size_t(blk) * p.Mpad + m0 + r, as_lds + boff, 16, 0, 0);
            }
        } else {
            // the rows' own scales as [M][G]: one scale per lane (4-byte loads), lane l of load j
            // holding position 64j + l of the stage's [KB][BM] (block pos / BM, row pos % BM)
            for (int j = wave; j < kASLoads4; j += 4) {
                const int pos = 64 * j + lane, kb = pos / BM, r = pos - kb * BM;
                const int row = min(m0 + r, p.M - 1), blk = min(g0 + kb, B - 1);
                __builtin_amdgcn_global_load_lds(p.as + size_t(row) * G + blk, as_lds + boff + j * 256, 4, 0, 0);
            }
        }
        if (wave == 3 && lane < kWSLanes) {
            // the four lanes' scales of one quad and block per lane
            const int kb = lane / (BN / 4), qd = lane - kb * (BN / 4), blk = min(g0 + kb, B - 1);
            const int q = min((n0 >> 2) + qd, last_col >> 2);
            __builtin_amdgcn_global_load_lds(p.wscales + (size_t(q) * G + blk) * 4, ws_lds + boff, 16, 0, 0);
        }
    };

    float acc[WM][WN][16];
#pragma unroll
    for (int a = 0; a < WM; a++)
#pragma unroll
        for (int b = 0; b < WN; b++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[a][b][v] = 0.0f;
    const int wr0 = (wave >> 1) * 32 * WM, wc0 = (wave & 1) * 32 * WN;
    const int half = 16 * (h ^ ((i >> 2) & 1));  // the staged half of this lane's row (see issue)

    issue(0, 0);
    for (int s = 0; s < stages; s++) {
        const int buf = s & 1;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's loads of stage s
        __syncthreads();  // every wave's loads of stage s; every wave done with stage s - 1
        if (s + 1 < stages) issue(s + 1, buf ^ 1);
        const unsigned char *base = stage_lds + buf * kStage;
        const int8_t *As = reinterpret_cast<const int8_t *>(base);
        const int8_t *Ws = As + T::A_BYTES;
        const float *ASs = reinterpret_cast<const float *>(Ws + T::W_BYTES);
        const float *WSs = ASs + KB * BM;
        // Per pair of blocks, the scale products fl(ws·as) come from one f32 MFMA outer product
        // per sub-tile (v_mfma_f32_32x32x1_2b: lanes 0..31 give the first block's row and column
        // scales, lanes 32..63 the second's; exactly the VALU's rounded products, subnormals
        // included), in the layout of the int8 products: one scale read per lane, not sixteen.
#pragma unroll
        for (int pr = 0; pr < KB / 2; pr++) {
            const int kb0 = 2 * pr;
            if (s * KB + kb0 >= B) break;  // uniform
            const bool second = s * KB + kb0 + 1 < B;
            float asv[WM], wsv[WN];
            v4i a[2][WM], w[2][WN];
#pragma unroll
            for (int rt = 0; rt < WM; rt++) asv[rt] = ASs[(kb0 + h) * BM + wr0 + rt * 32 + i];
#pragma unroll
            for (int ct = 0; ct < WN; ct++) wsv[ct] = WSs[(kb0 + h) * BN + wc0 + ct * 32 + i];
#pragma unroll
            for (int k2 = 0; k2 < 2; k2++) {
                const int kb = kb0 + k2;
#pragma unroll
                for (int rt = 0; rt < WM; rt++)
                    a[k2][rt] = *reinterpret_cast<const v4i *>(As + (kb * BM + wr0 + rt * 32 + i) * 32 + half);
#pragma unroll
                for (int ct = 0; ct < WN; ct++) {
                    const int c = wc0 + ct * 32 + i;
                    if (FMT == 8) {
                        w[k2][ct] = *reinterpret_cast<const v4i *>(Ws + (kb * BN + c) * RB + half);
                    } else {
                        const v4i x = *reinterpret_cast<const v4i *>(Ws + (kb * BN + c) * RB);
                        const int sh = h * 4;
                        w[k2][ct] = v4i{nibbles_signed(x.x >> sh), nibbles_signed(x.y >> sh), nibbles_signed(x.z >> sh),
                                        nibbles_signed(x.w >> sh)};
                    }
                }
            }
#pragma unroll
            for (int rt = 0; rt < WM; rt++)
#pragma unroll
                for (int ct = 0; ct < WN; ct++) {
                    const v32f zero32 = {0};
                    const v32f pp = __builtin_amdgcn_mfma_f32_32x32x1f32(asv[rt], wsv[ct], zero32, 0, 0, 0);
#pragma unroll
                    for (int k2 = 0; k2 < 2; k2++) {
                        if (k2 == 1 && !second) break;
                        const v16i zero = {0};
                        const v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[k2][rt], w[k2][ct], zero, 0, 0, 0);
#pragma unroll
                        for (int v = 0; v < 16; v++)
                            acc[rt][ct][v] = FUSED ? __builtin_fmaf(float(d[v]), pp[16 * k2 + v], acc[rt][ct][v])
                                                   : acc[rt][ct][v] + float(d[v]) * pp[16 * k2 + v];
                    }
                }
        }
    }
#pragma unroll
    for (int rt = 0; rt < WM; rt++)
#pragma unroll
        for (int ct = 0; ct < WN; ct++) {
            const int n = n0 + wc0 + ct * 32 + i;
            if (n > last_col) continue;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int r = m0 + wr0 + rt * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                if (r >= p.M) continue;
                float *o = p.out + size_t(r) * p.ld_out + (n - p.col_begin);
                float y = acc[rt][ct][v];
                if (p.bias && n < p.n_rows) y = y + p.bias[n];
                *o = p.accumulate ? *o + y : y;
            }
        }
}

// Few 32 x 32 output tiles (512 x 4864 -> 896: 448 tiles for 1024 SIMDs) under the fused scaling: a
// workgroup of four waves owns one 32 x 32 tile and wave w its 16 x 16 quarter (w / 2, w % 2) over
// every block in group order with v_mfma_i32_16x16x32_i8 (K = one block), so no wave hands a term to
// another and no barrier waits on a term. The tile's operands for kQuarterBlocks blocks at a time (a
// stage) arrive by direct global-to-LDS loads, DEPTH stages in flight, and each wave reads its 16
// rows and 16 columns from them:
//   A  [kb][32 rows][32 B]  activation levels (q [M][K], row-major);
//   W  [kb][32 cols][32 B]  weight levels (Q8; Q4: [kb][32 cols][16 B] packed nibbles);
//   AS [kb][32 rows]        activation scales, from the rows' [M][G] scales by 4-byte loads;
//   WS [kb][32 cols]        weight scales, the table's ((q·G + g)·4 + lane) order per quad.
// Operands (16x16x32): lane l feeds row (or column) l % 16 with inputs 8·(l / 16) .. + 7 of the
// block; the product of lane l is column l % 16, rows 4·(l / 16) + v. The scale products of four
// blocks come from one f32 outer product (v_mfma_f32_16x16x1_4b_f32) in the same layout, exactly
// the VALU's rounded fl(ws·as). Rows and columns past the edges re-read the last valid one; blocks
// past the last are loaded clamped and skipped.
constexpr int kQuarterBlocks = 8;

template <int FMT>
struct QuarterTile {
    static constexpr int KB = kQuarterBlocks;
    static constexpr int RB = FMT == 8 ? 32 : 16;  // weight bytes of a column and block
    static constexpr int A_BYTES = KB * 32 * 32, W_BYTES = KB * 32 * RB, AS_BYTES = KB * 32 * 4, WS_BYTES = KB * 32 * 4;
    static constexpr int STAGE = A_BYTES + W_BYTES + AS_BYTES + WS_BYTES;
    // each wave's direct loads of a stage: A, W (1 KiB each), AS (4 bytes a lane), WS (16 lanes)
    static constexpr int A_LOADS = KB / 4, W_LOADS = KB * RB / 32 / 4;
    static constexpr int LOADS = A_LOADS + W_LOADS + 2;
    static_assert(KB % 4 == 0 && A_LOADS >= 1 && W_LOADS >= 1 && KB * 32 * 4 == 4 * 256, "quarter stage shape");
};

template <int FMT, int DEPTH, bool FUSED>
__global__ __launch_bounds__(256) void gemm_quarter_kernel(GemmParams p)
{
    using T = QuarterTile<FMT>;
    constexpr int KB = T::KB, QB = FMT == 8 ? 128 : 64, kALoads = T::A_LOADS, kWLoads = T::W_LOADS, kLoads = T::LOADS;
    constexpr int kStage = T::STAGE, kA = T::A_BYTES, kW = T::W_BYTES, kAS = T::AS_BYTES;
    extern __shared__ __align__(16) unsigned char quarter_lds[];  // [DEPTH][STAGE]
    const int tid = threadIdx.x, lane = tid & 63, c = lane & 15, s = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int tx, ty;
    tile_of(int(blockIdx.x), (p.col_end - p.col_begin + 31) / 32, (p.M + 31) / 32, tx, ty);
    const int m0 = ty * 32, n0 = p.col_begin + tx * 32;
    const int B = p.B, G = p.G, K = p.K, last_col = p.col_end - 1;
    const int stages = (B + KB - 1) / KB;

    auto issue = [&](int st, int buf) {
        unsigned char *base = quarter_lds + buf * kStage;
        const int b0 = st * KB;
#pragma unroll
        for (int j = 0; j < kALoads; j++) {  // block kb; lane l: row l / 2, half l % 2
            const int kb = wave * kALoads + j;
            const int row = min(m0 + (lane >> 1), p.M - 1), blk = min(b0 + kb, B - 1);
            __builtin_amdgcn_global_load_lds(p.q + size_t(row) * K + blk * 32 + (lane & 1) * 16, base + kb * 1024, 16, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < kWLoads; j++) {  // 1 KiB piece k of the stage's weight levels
            const int k = wave * kWLoads + j;
            const int8_t *src;
            if (FMT == 8) {  // block k; lane l: column l / 2, half l % 2
                const int col = min(n0 + (lane >> 1), last_col), blk = min(b0 + k, B - 1);
                src = p.codes + size_t(col >> 2) * B * QB + size_t(blk) * QB + (col & 3) * 32 + (lane & 1) * 16;
            } else {  // blocks 2k + l / 32; lane l: column l % 32
                const int col = min(n0 + (lane & 31), last_col), blk = min(b0 + 2 * k + (lane >> 5), B - 1);
                src = p.codes + size_t(col >> 2) * B * QB + size_t(blk) * QB + (col & 3) * 16;
            }
            __builtin_amdgcn_global_load_lds(src, base + kA + k * 1024, 16, 0, 0);
        }
        {  // AS position 64·wave + lane: block pos / 32, row pos % 32
            const int pos = 64 * wave + lane;
            const int row = min(m0 + (pos & 31), p.M - 1), blk = min(b0 + (pos >> 5), B - 1);
            __builtin_amdgcn_global_load_lds(p.as + size_t(row) * G + blk, base + kA + kW + wave * 256, 4, 0, 0);
        }
        if (lane < 16) {  // WS: blocks 2·wave + l / 8, quad l % 8 (its four columns' scales)
            const int q = min((n0 >> 2) + (lane & 7), last_col >> 2), blk = min(b0 + 2 * wave + (lane >> 3), B - 1);
            __builtin_amdgcn_global_load_lds(p.wscales + (size_t(q) * G + blk) * 4, base + kA + kW + kAS + wave * 256, 16, 0, 0);
        }
    };

    const int wr = 16 * (wave >> 1), wc = 16 * (wave & 1);
    const int a_off = (wr + c) * 32 + 8 * s;
    const int w_off = kA + (FMT == 8 ? (wc + c) * 32 + 8 * s : (wc + c) * 16 + 8 * (s & 1));
    const int shift = FMT == 8 ? 0 : 4 * (s >> 1);
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // the blocks [0, live) of the stage in `base`, in order (CHECK: live < KB, the last stage)
    auto compute = [&](const unsigned char *base, int live, auto check) {
        constexpr bool CHECK = decltype(check)::value;
#pragma unroll
        for (int j4 = 0; j4 < KB / 4; j4++) {
            const float as = *reinterpret_cast<const float *>(base + kA + kW + ((4 * j4 + s) * 32 + wr + c) * 4);
            const float ws = *reinterpret_cast<const float *>(base + kA + kW + kAS + ((4 * j4 + s) * 32 + wc + c) * 4);
            long a[4], w[4];
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int kb = 4 * j4 + b;
                a[b] = *reinterpret_cast<const long *>(base + kb * 1024 + a_off);
                w[b] = *reinterpret_cast<const long *>(base + kb * (32 * T::RB) + w_off);
            }
            const v16f zero16 = {0};
            const v16f pp = __builtin_amdgcn_mfma_f32_16x16x1f32(as, ws, zero16, 0, 0, 0);
#pragma unroll
            for (int b = 0; b < 4; b++) {
                if (CHECK && 4 * j4 + b >= live) break;  // uniform
                long x = w[b];
                if (FMT == 4) {
                    const int lo = nibbles_signed(int(x) >> shift), hi = nibbles_signed(int(x >> 32) >> shift);
                    x = long(unsigned(lo)) | (long(hi) << 32);
                }
                const v4i zero = {0, 0, 0, 0};
                const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[b], x, zero, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; v++)
                    acc[v] = FUSED ? __builtin_fmaf(float(d[v]), pp[4 * b + v], acc[v]) : acc[v] + float(d[v]) * pp[4 * b + v];
            }
        }
    };

#pragma unroll
    for (int k = 0; k < DEPTH - 1; k++)
        if (k < stages) issue(k, k);
    for (int st = 0; st < stages; st++) {
        // this wave's loads of stage st (the later stages issued may still be in flight)
        if (st + DEPTH - 2 < stages) asm volatile("s_waitcnt vmcnt(%0)" ::"n"((DEPTH - 2) * kLoads) : "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        // every wave's loads of stage st; every wave done reading the buffer refilled next
        stage_barrier();
        if (st + DEPTH - 1 < stages) issue(st + DEPTH - 1, (st + DEPTH - 1) % DEPTH);
        const unsigned char *base = quarter_lds + (st % DEPTH) * kStage;
        if (st + 1 < stages) compute(base, KB, std::false_type{});
        else compute(base, B - st * KB, std::true_type{});
    }
    const int n = n0 + wc + c;
    if (n > last_col) return;
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const int r = m0 + wr + 4 * s + v;
        if (r >= p.M) continue;
        float *o = p.out + size_t(r) * p.ld_out + (n - p.col_begin);
        float y = acc[v];
        if (p.bias && n < p.n_rows) y = y + p.bias[n];
        *o = p.accumulate ? *o + y : y;
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

// One workgroup per 32 x 32 tile, four waves on its 16 x 16 quarters (gemm_quarter_kernel).
template <int FMT, int DEPTH, bool FUSED>
int launch_quarter(const GemmParams &p, hipStream_t s)
{
    const long tiles = long((p.col_end - p.col_begin + 31) / 32) * ((p.M + 31) / 32);
    const size_t smem = size_t(DEPTH) * QuarterTile<FMT>::STAGE;
    if (smem > 64 * 1024)
        FG_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_quarter_kernel<FMT, DEPTH, FUSED>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
    gemm_quarter_kernel<FMT, DEPTH, FUSED><<<unsigned(tiles), 256, smem, s>>>(p);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

// 32 x 64 tiles per wave where they still give every SIMD a wave or more, else 32 x 32.
template <int FMT, bool FUSED>
int launch_tiles_as(const GemmParams &p, bool dots, bool lds, hipStream_t s)
{
    const int ncols = p.col_end - p.col_begin;
    const long narrow_waves = long((ncols + 31) / 32) * ((p.M + 31) / 32);
    if (p.M <= 16 && (dots || lds)) {
        const dim3 grid(unsigned(((ncols + 15) / 16) * ((p.M + 15) / 16)));
        // fewer than 512 tiles: four waves per tile (16 x 4864 -> 896: 18.5 -> 11.6 us; at 896
        // tiles, 16 x 4096 -> 14336 Q4, one wave per tile is faster: 27.8 against 31.5 us)
        const size_t split16_smem = size_t(p.B) * 16 * 4 + 2 * 4 * 64 * 16;
        if (!dots && !FUSED && p.B % 4 == 0 && grid.x < 512 && split16_smem <= 64 * 1024) {
            gemm16_split_kernel<FMT><<<grid, 256, split16_smem, s>>>(p);
            FG_HIP(hipGetLastError());
            return FG_OK;
        }
        // more tiles: four adjacent column tiles per workgroup, their operands streamed through LDS
        if (!dots && !FUSED) {
            const dim3 sgrid(unsigned(((ncols + 63) / 64) * ((p.M + 15) / 16)));
            constexpr int lds = PairTile<FMT>::LDS;
            FG_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gemm16_pair_kernel<FMT>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds));
            gemm16_pair_kernel<FMT><<<sgrid, 512, size_t(lds), s>>>(p);
            FG_HIP(hipGetLastError());
            return FG_OK;
        }
        if (dots) gemm16_kernel<FMT, true, false><<<grid, 64, 0, s>>>(p);
        else gemm16_kernel<FMT, false, FUSED><<<grid, 64, size_t(p.B) * 16 * 4, s>>>(p);
        FG_HIP(hipGetLastError());
        return FG_OK;
    }
    // 17 to 256 rows over a long K (64 blocks or more), e.g. a prefill chunk's down projection:
    // the paired 16-row tiles in row bands stream each band's operands through LDS once per 64
    // columns (158 x 4864 -> 896: 15.8 against 18.9 us on the four-wave split kernel; at 512 rows,
    // or K = 896, the kernels below are as fast or faster)
    if (!dots && !FUSED && lds && p.M > 16 && p.M <= 256 && p.B >= 64) {
        const dim3 sgrid(unsigned(((ncols + 63) / 64) * ((p.M + 15) / 16)));
        constexpr int plds = PairTile<FMT>::LDS;
        FG_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gemm16_pair_kernel<FMT>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, plds));
        gemm16_pair_kernel<FMT><<<sgrid, 512, size_t(plds), s>>>(p);
        FG_HIP(hipGetLastError());
        return FG_OK;
    }
    // the fused scaling over few 32 x 32 tiles: four waves per tile on its quarters (512 x 4864 ->
    // 896: 25.7 against 33.2 us for one wave per tile; the exact order keeps the split kernel below,
    // as fast or faster there: 24.0 against 27.3 us)
    if (FUSED && !dots && lds && p.M > 16 && narrow_waves < 2048) return launch_quarter<FMT, 2, true>(p, s);
    const size_t smem = size_t(p.B) * 32 * 4;
    // too few 32 x 32 tiles for two waves per SIMD: four waves per tile
    if (!dots && lds && !FUSED && p.B % 4 == 0 && narrow_waves < 2048 && split_lds_bytes(p.B) <= 64 * 1024) {
        launch_split<FMT>(p, unsigned(narrow_waves), s);
        FG_HIP(hipGetLastError());
        return FG_OK;
    }
    const long wide_waves = long((ncols + 63) / 64) * ((p.M + 31) / 32);
    if (wide_waves >= 1024) {
        const dim3 grid{unsigned(wide_waves)};
        if (dots) gemm_kernel<FMT, 2, true, false, false><<<grid, 64, 0, s>>>(p);
        else if (lds) gemm_kernel<FMT, 2, false, true, FUSED><<<grid, 64, smem, s>>>(p);
        else gemm_kernel<FMT, 2, false, false, FUSED><<<grid, 64, 0, s>>>(p);
    } else {
        const dim3 grid{unsigned(narrow_waves)};
        if (dots) gemm_kernel<FMT, 1, true, false, false><<<grid, 64, 0, s>>>(p);
        else if (lds) gemm_kernel<FMT, 1, false, true, FUSED><<<grid, 64, smem, s>>>(p);
        else gemm_kernel<FMT, 1, false, false, FUSED><<<grid, 64, 0, s>>>(p);
    }
    FG_HIP(hipGetLastError());
    return FG_OK;
}

// 32 x 64 tiles per wave where they still give every SIMD a wave or more, else 32 x 32.
template <int FMT>
int launch_tiles(const GemmParams &p, bool dots, bool lds, bool fused, hipStream_t s)
{
    return fused && !dots ? launch_tiles_as<FMT, true>(p, dots, lds, s) : launch_tiles_as<FMT, false>(p, dots, lds, s);
}

template <int FMT, int WM, int WN>
int launch_lds_as(const GemmParams &p, bool fused, hipStream_t s)
{
    using T = LdsTile<FMT, WM, WN>;
    const long groups = long((p.col_end - p.col_begin + T::BN - 1) / T::BN) * ((p.M + T::BM - 1) / T::BM);
    const size_t smem = 2 * size_t(T::STAGE);
    if (fused) gemm_lds_kernel<FMT, WM, WN, true><<<unsigned(groups), 256, smem, s>>>(p);
    else gemm_lds_kernel<FMT, WM, WN, false><<<unsigned(groups), 256, smem, s>>>(p);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

// tiles: 10·WM + WN (workgroup tiles of 64·WM rows x 64·WN columns)
template <int FMT>
int launch_lds(const GemmParams &p, int tiles, bool fused, hipStream_t s)
{
    return tiles == 21 ? launch_lds_as<FMT, 2, 1>(p, fused, s) : launch_lds_as<FMT, 1, 1>(p, fused, s);
}

// T2b128 (ternary levels, one scale per 128 inputs: matmul.rs:461-469, quant.rs:168-177): one
// thread per (row, output), the groups in order, each group's four blocks summed as integers
// before the scaling (matmul.rs:671-709). Device row-block of 8 bytes: byte i holds the offset
// codes of inputs i, i + 8, i + 16, i + 24 in its bit pairs. Not tuned: no workload uses it.
__global__ __launch_bounds__(256) void t2_product_kernel(const uint8_t *__restrict__ codes, const float *__restrict__ wscales,
                                                         int B, int G, int K, int n_rows, const int8_t *__restrict__ q,
                                                         const float *__restrict__ as, const int32_t *__restrict__ corr,
                                                         int rows, int col_begin, int ncols, const float *__restrict__ bias,
                                                         float *out, long ld_out, int accumulate, int32_t *dots, int fused)
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
        const float sc = wscales[(size_t(quad) * G + g) * 4 + L] * as[size_t(r) * G + g];
        s = fused ? __builtin_fmaf(float(D), sc, s) : s + float(D) * sc;
    }
    if (dots) return;
    if (bias && n < n_rows) s = s + bias[n];
    float *o = out + size_t(r) * ld_out + c;
    *o = accumulate ? *o + s : s;
}

// T2b128 products, streamed: R activation rows per slice of the grid's second dimension, one
// wave per quad of 4 outputs. A quad's codes are one run of B·32 bytes (matmul.rs:461-469: per
// block, each output's 8 bytes hold 4 two-bit parts of 8 inputs), read 1 KiB (32 blocks, 8
// groups of 128) per load instruction with a ring of kT2Ring chunks in flight. Lane l takes
// block 4·(l/8) + l%4 of the chunk and outputs 2·((l/4)%2) + {0, 1}, so the four blocks of a
// group sit in one quad of lanes and their int32 dots sum by two DPP steps. Each group's term
// goes to the wave's LDS row for its (row, output); after the last chunk lanes 0..4R-1, one per
// (row, output), add their row in group order: s = fl(s + fl(fl((float)D_g) · fl(ws · as))),
// or s = fma((float)D_g, ws · as, s) under the fused scaling.
struct T2Params {
    const uint8_t *codes;
    const float *wscales;
    int B, G, K, n_rows;
    const int8_t *q;  // [rows][K] levels, 16-byte aligned rows
    const float *as;  // [rows][G]
    const int32_t *corr;
    int rows;
    int quad_begin, quad_end, col_begin;
    const float *bias;
    float *out;
    long ld_out;
    int accumulate;
};

constexpr int kT2Ring = 4;

// A (row, output)'s LDS row of group terms: G floats padded to whole float4s and 4 more, so the
// rows of neighbouring lanes start in different banks.
__host__ __device__ inline int t2_row_stride(int G) { return (G + 3) / 4 * 4 + 4; }

// Dynamic LDS of one workgroup: R rows of levels, R rows of (scale, correction), and per wave R
// x 4 rows of group terms (two floats a group, D and ws·as, under the fused scaling).
inline size_t t2_lds_bytes(int R, int K, int G, bool fused)
{
    return size_t(R) * K + size_t(R) * G * 8 + 4 * size_t(R) * 4 * t2_row_stride(G) * 4 * (fused ? 2 : 1);
}

template <int R, bool FUSED>
__global__ __launch_bounds__(256) void t2_rows_kernel(T2Params p)
{
    extern __shared__ __align__(16) unsigned char t2_lds[];
    const int G = p.G, Gp = t2_row_stride(G);
    int4 *act = reinterpret_cast<int4 *>(t2_lds);
    float *rs = reinterpret_cast<float *>(t2_lds + size_t(R) * p.K);
    int *rc = reinterpret_cast<int *>(rs + R * G);
    float *tb = reinterpret_cast<float *>(rc + R * G);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = blockIdx.y * R, nr = min(R, p.rows - row0);
    const int quad = p.quad_begin + blockIdx.x * 4 + wave;
    const bool live = quad < p.quad_end;
    const int jj = lane & 3, hh = (lane >> 2) & 1, gq = lane >> 3;
    const int blk = 4 * gq + jj;        // this lane's block in a chunk of 32
    // its 16 bytes of the block (half hh: outputs 2·hh and 2·hh + 1) are the chunk's piece 2·blk + hh
    const int col = 2 * hh + (jj & 1);  // the output whose term this lane writes
    const int nchunks = (p.B + 31) >> 5;
    const int4 *wq = reinterpret_cast<const int4 *>(p.codes + size_t(live ? quad : 0) * p.B * 32);
    const float *wsq = p.wscales + size_t(live ? quad : 0) * G * 4;

    // Every lane loads on every slot, chunks past the end included, from its block clamped into
    // the quad's run (the same count of loads on every path keeps the waits per load exact); the
    // terms of a block past the end are zeroed where they are formed.
    int4 ring[kT2Ring];
    float wsr[kT2Ring];
    auto fetch = [&](int c, int4 &w, float &ws) {
        const int bs = min(32 * c + blk, p.B - 1);
        w = wq[2 * bs + hh];
        ws = wsq[(bs >> 2) * 4 + col];
    };

    // The rows' levels, scales and corrections are loaded before the codes and stored to LDS
    // after them: loads complete in order, so the stores wait for these loads only, while the
    // codes stay in flight. The first R int4s and one (scale, correction) pair per thread go this
    // way (R rows of up to 4096 levels, up to 256 groups), from clamped addresses (rows past the
    // slice are zeroed at the store); larger slices finish with plain loops.
    constexpr int kStage16 = R, kStageG = 1;
    const int kv = p.K >> 4, n16 = R * kv, ng = R * G;
    const int4 *q4 = reinterpret_cast<const int4 *>(p.q);
    int4 st[kStage16];
    float sts[kStageG];
    int stc[kStageG];
#pragma unroll
    for (int k = 0; k < kStage16; k++) {
        const int i = min(int(threadIdx.x) + 256 * k, n16 - 1), r = i / kv;
        st[k] = q4[size_t(row0 + min(r, nr - 1)) * kv + (i - r * kv)];
    }
#pragma unroll
    for (int k = 0; k < kStageG; k++) {
        const int i = min(int(threadIdx.x) + 256 * k, ng - 1), r = i / G;
        const size_t at = size_t(row0 + min(r, nr - 1)) * G + (i - r * G);
        sts[k] = p.as[at];
        stc[k] = p.corr[at];
    }
    __builtin_amdgcn_sched_barrier(0);  // the staging loads go out first
#pragma unroll
    for (int i = 0; i < kT2Ring; i++) fetch(i, ring[i], wsr[i]);
    __builtin_amdgcn_sched_barrier(0);  // then the codes, then the stores
#pragma unroll
    for (int k = 0; k < kStage16; k++) {
        const int i = threadIdx.x + 256 * k;
        if (i < n16) act[i] = i / kv < nr ? st[k] : make_int4(0, 0, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < kStageG; k++) {
        const int i = threadIdx.x + 256 * k;
        if (i < ng) {
            const bool in = i / G < nr;
            rs[i] = in ? sts[k] : 0.0f;
            rc[i] = in ? stc[k] : 0;
        }
    }
    for (int i = threadIdx.x + 256 * kStage16; i < n16; i += 256) {
        const int r = i / kv;
        act[i] = r < nr ? q4[size_t(row0 + r) * kv + (i - r * kv)] : make_int4(0, 0, 0, 0);
    }
    for (int i = threadIdx.x + 256 * kStageG; i < ng; i += 256) {
        const int r = i / G;
        rs[i] = r < nr ? p.as[size_t(row0 + r) * G + (i - r * G)] : 0.0f;
        rc[i] = r < nr ? p.corr[size_t(row0 + r) * G + (i - r * G)] : 0;
    }
    __syncthreads();
    if (!live) return;

    // this wave's term rows: [R x 4][Gp] floats (D), and under the fused scaling [R x 4][Gp] of ws·as
    float *tw = tb + size_t(wave) * R * 4 * Gp * (FUSED ? 2 : 1);
    auto process = [&](int c, const int4 w, const float ws) {
        const int b = min(32 * c + blk, p.B - 1), g = min(8 * c + gq, G - 1);
        const bool real = 8 * c + gq < G;
        int cw[16];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            cw[4 * t + 0] = (w.x >> (2 * t)) & 0x03030303;
            cw[4 * t + 1] = (w.y >> (2 * t)) & 0x03030303;
            cw[4 * t + 2] = (w.z >> (2 * t)) & 0x03030303;
            cw[4 * t + 3] = (w.w >> (2 * t)) & 0x03030303;
        }
        // every LDS read of the chunk first (indices clamped into range, so no read is skipped)
        int4 a0[R], a1[R];
        int cv[R];
        float sv[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            a0[r] = act[((r * p.K) >> 4) + 2 * b];
            a1[r] = act[((r * p.K) >> 4) + 2 * b + 1];
            cv[r] = rc[r * G + g];
            sv[r] = rs[r * G + g];
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int a[8] = {a0[r].x, a0[r].y, a0[r].z, a0[r].w, a1[r].x, a1[r].y, a1[r].z, a1[r].w};
            int d0 = 0, d1 = 0;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                d0 = dot4(cw[4 * t + 0], a[2 * t], d0);
                d0 = dot4(cw[4 * t + 1], a[2 * t + 1], d0);
                d1 = dot4(cw[4 * t + 2], a[2 * t], d1);
                d1 = dot4(cw[4 * t + 3], a[2 * t + 1], d1);
            }
            d0 += xor1(d0);
            d0 += xor2(d0);
            d1 += xor1(d1);
            d1 += xor2(d1);
            const float f = real ? float(cv[r] + ((jj & 1) ? d1 : d0)) : 0.0f;
            const float sc = real ? ws * sv[r] : 0.0f;
            // lanes jj and jj + 2 hold the same group, output and values: both write them
            float *row = tw + (r * 4 + col) * Gp * (FUSED ? 2 : 1);
            if (FUSED) {
                row[8 * c + gq] = f;
                row[Gp + 8 * c + gq] = sc;
            } else {
                row[8 * c + gq] = f * sc;
            }
        }
    };

    if (nchunks <= kT2Ring) {  // the whole run is in flight already: no refills, no loop
#pragma unroll
        for (int i = 0; i < kT2Ring; i++)
            if (i < nchunks) process(i, ring[i], wsr[i]);
    } else {
        for (int c0 = 0; c0 < nchunks; c0 += kT2Ring) {
#pragma unroll
            for (int i = 0; i < kT2Ring; i++) {
                const int c = c0 + i;
                const int4 w = ring[i];
                const float ws = wsr[i];
                fetch(c + kT2Ring, ring[i], wsr[i]);
                if (c < nchunks) process(c, w, ws);
            }
        }
    }
    __builtin_amdgcn_wave_barrier();

    // the group-order sums, one (row, output) per lane; terms of groups past G are +0, which
    // leaves every sum as it is (a sum that starts at +0 is never -0)
    if (lane < 4 * R && (lane >> 2) < nr) {
        const float *tl = tw + lane * Gp * (FUSED ? 2 : 1);
        float s = 0.0f;
        for (int g = 0; g < G; g += 4) {
            const float4 v = *reinterpret_cast<const float4 *>(tl + g);
            if (FUSED) {
                const float4 u = *reinterpret_cast<const float4 *>(tl + Gp + g);
                s = __builtin_fmaf(v.x, u.x, s);
                s = __builtin_fmaf(v.y, u.y, s);
                s = __builtin_fmaf(v.z, u.z, s);
                s = __builtin_fmaf(v.w, u.w, s);
            } else {
                s = s + v.x;
                s = s + v.y;
                s = s + v.z;
                s = s + v.w;
            }
        }
        const int n = quad * 4 + (lane & 3);
        if (p.bias && n < p.n_rows) s = s + p.bias[n];
        float *o = p.out + size_t(row0 + (lane >> 2)) * p.ld_out + (n - p.col_begin);
        *o = p.accumulate ? *o + s : s;
    }
}

// T2b128 products of many rows on the int8 matrix cores: one wave per 32 x 32 output tile. Per
// group of 128 inputs, four v_mfma_i32_32x32x32_i8 (one per block of 32) chain the group's int32
// dots of a column's codes (0, 1, 2 as they are) with the rows' levels; the group total adds
// the row's correction (matmul.rs:461-469 with the quantizer's Backend::seed), and the exact
// rescale follows once per group: s = fl(s + fl(fl((float)D_g) · fl(ws · as))), or one fma
// under the fused scaling. Lane l feeds row (or column) l % 32 and the block's inputs
// 16·(l/32) .. + 15: from the column's 8 bytes (lo: inputs 8t + 0..3 at bits 2t, hi: 8t + 4..7),
// parts 2·(l/32) and 2·(l/32) + 1. Result: lane l holds column l % 32, rows 8·(v/4) + 4·(l/32)
// + v%4. The tile's scales and corrections sit in LDS ([G][32] each); operands stream two groups
// ahead in registers, rows and columns past the edges re-reading the last valid one.
constexpr int kT2GemmDepth = 2;  // groups in flight
// rows from which the 32 x 32 tiles take a T2b128 product; 5 to 16 rows go to the 16 x 16 tiles
// below (14336 x 4096: 11.4 µs at 9 rows, 15.1 at 16, against 17.6 for one row of 32 x 32 tiles
// and 17.1 for the streamed kernel's 8-row slice)
constexpr int kT2GemmRows = 17;
#ifndef FG_T2_WIDE_TILES
#define FG_T2_WIDE_TILES 2048
#endif
constexpr long kT2WideTiles = FG_T2_WIDE_TILES;

template <int TN>
struct T2Stage {
    v4i a[4];       // this lane's 16 levels of each of the group's blocks
    int2 w[TN][4];  // its column's 8 code bytes of each block, per 32-column sub-tile
    float ws[TN];   // the column's scale for the group
};

// TN: 32-column sub-tiles per wave (TN MFMA chains share the rows' operands, halving their
// reads at TN = 2).
template <int TN, bool FUSED>
__global__ __launch_bounds__(64) void t2_gemm_kernel(T2Params p)
{
    extern __shared__ __align__(16) float t2_tile[];  // [G][32] scales, then [G][32] corrections
    const int G = p.G, K = p.K;
    float *tsc = t2_tile;
    int *tco = reinterpret_cast<int *>(t2_tile + G * 32);
    const int lane = threadIdx.x, i = lane & 31, h = lane >> 5;
    const int ncol = (p.quad_end - p.quad_begin) * 4, col_begin = p.quad_begin * 4;
    int tx, ty;
    tile_of(int(blockIdx.x), (ncol + 32 * TN - 1) / (32 * TN), (p.rows + 31) / 32, tx, ty);
    const int m0 = ty * 32, n0 = col_begin + tx * 32 * TN;
    const int row = min(m0 + i, p.rows - 1);
    const int8_t *arow = p.q + size_t(row) * K + h * 16;
    const uint8_t *wcol[TN];
    const float *wscol[TN];
#pragma unroll
    for (int t = 0; t < TN; t++) {
        const int nc = min(n0 + 32 * t + i, col_begin + ncol - 1);
        wcol[t] = p.codes + size_t(nc >> 2) * p.B * 32 + (nc & 3) * 8;
        wscol[t] = p.wscales + size_t(nc >> 2) * G * 4 + (nc & 3);
    }

    // rows m0 .. m0 + 31's scales and corrections, transposed to [group][row]: lane l takes row
    // l % 32 and the groups of parity l / 32, eight loads (clamped) before their stores
    for (int g0 = h; g0 < G; g0 += 16) {
        float a8[8];
        int c8[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const size_t at = size_t(row) * G + min(g0 + 2 * u, G - 1);
            a8[u] = p.as[at];
            c8[u] = p.corr[at];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int g = g0 + 2 * u;
            if (g < G) {
                tsc[g * 32 + i] = a8[u];
                tco[g * 32 + i] = c8[u];
            }
        }
    }
    __syncthreads();

    auto fetch = [&](int g, T2Stage<TN> &st) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            st.a[k] = *reinterpret_cast<const v4i *>(arow + (4 * g + k) * 32);
#pragma unroll
            for (int t = 0; t < TN; t++) st.w[t][k] = *reinterpret_cast<const int2 *>(wcol[t] + size_t(4 * g + k) * 32);
        }
#pragma unroll
        for (int t = 0; t < TN; t++) st.ws[t] = wscol[t][size_t(g) * 4];
    };
    auto product = [&](const T2Stage<TN> &st, int t) {
        v16i d = {0};
        const int sh = 4 * h;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int lo = st.w[t][k].x, hi = st.w[t][k].y;
            const v4i w = {(lo >> sh) & 0x03030303, (hi >> sh) & 0x03030303, (lo >> (sh + 2)) & 0x03030303,
                           (hi >> (sh + 2)) & 0x03030303};
            d = __builtin_amdgcn_mfma_i32_32x32x32_i8(st.a[k], w, d, 0, 0, 0);
        }
        return d;
    };
    float acc[TN][16];
#pragma unroll
    for (int t = 0; t < TN; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[t][v] = 0.0f;
    auto rescale = [&](int g, const T2Stage<TN> &st, int t, const v16i d) {
        const v4f *ls = reinterpret_cast<const v4f *>(tsc + g * 32 + 4 * h);
        const v4i *lc = reinterpret_cast<const v4i *>(tco + g * 32 + 4 * h);
        const v4f s0 = ls[0], s1 = ls[2], s2 = ls[4], s3 = ls[6];
        const v4i c0 = lc[0], c1 = lc[2], c2 = lc[4], c3 = lc[6];
        const float sc[16] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w, s2.x, s2.y, s2.z, s2.w, s3.x, s3.y, s3.z, s3.w};
        const int co[16] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w, c2.x, c2.y, c2.z, c2.w, c3.x, c3.y, c3.z, c3.w};
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const float D = float(co[v] + d[v]);
            acc[t][v] = FUSED ? __builtin_fmaf(D, st.ws[t] * sc[v], acc[t][v]) : acc[t][v] + D * (st.ws[t] * sc[v]);
        }
    };

    // group g lives in stage g % kT2GemmDepth; its refill (clamped at the last group, so no
    // branch splits the loads) follows its rescale
    T2Stage<TN> st[kT2GemmDepth];
#pragma unroll
    for (int k = 0; k < kT2GemmDepth; k++) {
        fetch(min(k, G - 1), st[k]);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (int g = 0; g < G; g += kT2GemmDepth) {
#pragma unroll
        for (int k = 0; k < kT2GemmDepth; k++) {
            if (g + k < G) {
#pragma unroll
                for (int t = 0; t < TN; t++) rescale(g + k, st[k], t, product(st[k], t));
            }
            fetch(min(g + k + kT2GemmDepth, G - 1), st[k]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int t = 0; t < TN; t++) {
        const int n = n0 + 32 * t + i;
        if (n >= col_begin + ncol) continue;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int r = m0 + 8 * (v >> 2) + 4 * h + (v & 3);
            if (r >= p.rows) continue;
            float y = acc[t][v];
            if (p.bias && n < p.n_rows) y = y + p.bias[n];
            float *o = p.out + size_t(r) * p.ld_out + (n - col_begin);
            *o = p.accumulate ? *o + y : y;
        }
    }
}

template <int TN, bool FUSED>
int launch_t2_gemm_as(const T2Params &p, hipStream_t s)
{
    const long tiles = long((p.quad_end - p.quad_begin) * 4 + 32 * TN - 1) / (32 * TN) * ((p.rows + 31) / 32);
    t2_gemm_kernel<TN, FUSED><<<unsigned(tiles), 64, size_t(p.G) * 32 * 8, s>>>(p);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

// 32 x 64 tiles while they still give every SIMD two waves, else 32 x 32
template <bool FUSED>
int launch_t2_gemm(const T2Params &p, hipStream_t s)
{
    const long wide = long((p.quad_end - p.quad_begin) * 4 + 63) / 64 * ((p.rows + 31) / 32);
    return wide >= kT2WideTiles ? launch_t2_gemm_as<2, FUSED>(p, s) : launch_t2_gemm_as<1, FUSED>(p, s);
}

// T2b128 products of 5 to 16 rows on the int8 matrix cores: one wave per 16 x 16 output tile, so
// 14336 outputs take 896 waves where 32 x 32 tiles give 448 with half their rows repeated. Per
// group of 128 inputs, four v_mfma_i32_16x16x32_i8 chain the group's int32 dots; the correction
// and the exact rescale follow as in the 32 x 32 kernel above. An integer dot does not depend on
// which step takes which input as long as both operands agree, so each lane reads its row's group
// in two 16-byte pieces, inputs 16·(l/16) + 0..15 and 64 + 16·(l/16) + 0..15 (a row's 128 bytes in
// two loads of 64 bytes per row), and step j takes 8 bytes of piece j/2: inputs
// 64·(j/2) + 16·(l/16) + 8·(j%2) + 0..7, which lie in block 2·(j/2) + (l/16)/2 at offset
// 16·((l/16)%2) + 8·(j%2): from that block's 8 code bytes, bits 2t, t = 2·((l/16)%2) + j%2, of
// every byte of the lo word (inputs + 0..3) and of the hi word (+ 4..7). Lane l feeds row (or
// column) l % 16. Result: lane l holds column l % 16, rows 4·(l/16) + v, v = 0..3. The tile's
// scales and corrections sit in LDS ([G][16] each); operands stream four groups ahead in registers.
constexpr int kT2Gemm16Depth = 4;  // groups in flight
#ifndef FG_T2_MFMA16_ROWS
#define FG_T2_MFMA16_ROWS 5
#endif
constexpr int kT2Gemm16Rows = FG_T2_MFMA16_ROWS;  // fewest rows taken by the 16 x 16 kernel
#ifndef FG_T2_MFMA16_MAX_ROWS
#define FG_T2_MFMA16_MAX_ROWS 16
#endif
// most rows taken by it: for 17-32 rows two row tiles of 16 x 16 measured 24.5 µs against
// 17.4-19.6 for one of 32 x 32
constexpr int kT2Gemm16MaxRows = FG_T2_MFMA16_MAX_ROWS;

typedef long v2l __attribute__((ext_vector_type(2)));
struct T2Stage16 {
    v2l a[2];    // this lane's two 16-byte pieces of its row's group
    int2 w[2];   // its column's 8 code bytes of blocks (l/16)/2 and 2 + (l/16)/2
    float ws;    // the column's scale for the group
};

template <bool FUSED>
__global__ __launch_bounds__(64) void t2_gemm16_kernel(T2Params p)
{
    extern __shared__ __align__(16) float t2_tile16[];  // [G][16] scales, then [G][16] corrections
    const int G = p.G, K = p.K;
    float *tsc = t2_tile16;
    int *tco = reinterpret_cast<int *>(t2_tile16 + G * 16);
    const int lane = threadIdx.x, i = lane & 15, s = lane >> 4;
    const int ncol = (p.quad_end - p.quad_begin) * 4, col_begin = p.quad_begin * 4;
    int tx, ty;
    tile_of(int(blockIdx.x), (ncol + 15) / 16, (p.rows + 15) / 16, tx, ty);
    const int m0 = ty * 16, n0 = col_begin + tx * 16;
    const int row = min(m0 + i, p.rows - 1);  // rows and columns past the edges re-read the last valid one
    const int8_t *arow = p.q + size_t(row) * K + s * 16;
    const int nc = min(n0 + i, col_begin + ncol - 1);
    const uint8_t *wcol = p.codes + size_t(nc >> 2) * p.B * 32 + (nc & 3) * 8;
    const float *wscol = p.wscales + size_t(nc >> 2) * G * 4 + (nc & 3);

    // rows m0 .. m0 + 15's scales and corrections, transposed to [group][row]: lane l takes row
    // l % 16 and the groups congruent to l / 16 mod 4, eight loads (clamped) before their stores
    for (int g0 = s; g0 < G; g0 += 32) {
        float a8[8];
        int c8[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const size_t at = size_t(row) * G + min(g0 + 4 * u, G - 1);
            a8[u] = p.as[at];
            c8[u] = p.corr[at];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int g = g0 + 4 * u;
            if (g < G) {
                tsc[g * 16 + i] = a8[u];
                tco[g * 16 + i] = c8[u];
            }
        }
    }
    __syncthreads();

    auto fetch = [&](int g, T2Stage16 &st) {
        st.a[0] = *reinterpret_cast<const v2l *>(arow + g * 128);
        st.a[1] = *reinterpret_cast<const v2l *>(arow + g * 128 + 64);
        st.w[0] = *reinterpret_cast<const int2 *>(wcol + size_t(4 * g + (s >> 1)) * 32);
        st.w[1] = *reinterpret_cast<const int2 *>(wcol + size_t(4 * g + 2 + (s >> 1)) * 32);
        st.ws = wscol[size_t(g) * 4];
    };
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto step = [&](int g, const T2Stage16 &st) {
        v4i d = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int sh = 4 * (s & 1) + 2 * (j & 1);
            const int2 wd = st.w[j >> 1];
            const int lo = (wd.x >> sh) & 0x03030303, hi = (wd.y >> sh) & 0x03030303;
            d = __builtin_amdgcn_mfma_i32_16x16x32_i8(st.a[j >> 1][j & 1], long(unsigned(lo)) | (long(hi) << 32), d, 0, 0, 0);
        }
        const v4f sc = *reinterpret_cast<const v4f *>(tsc + g * 16 + 4 * s);
        const v4i co = *reinterpret_cast<const v4i *>(tco + g * 16 + 4 * s);
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const float D = float(co[v] + d[v]);
            acc[v] = FUSED ? __builtin_fmaf(D, st.ws * sc[v], acc[v]) : acc[v] + D * (st.ws * sc[v]);
        }
    };

    // group g lives in stage g % kT2Gemm16Depth; its refill (clamped at the last group, so no
    // branch splits the loads) follows its rescale
    T2Stage16 st[kT2Gemm16Depth];
#pragma unroll
    for (int k = 0; k < kT2Gemm16Depth; k++) {
        fetch(min(k, G - 1), st[k]);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (int g = 0; g < G; g += kT2Gemm16Depth) {
#pragma unroll
        for (int k = 0; k < kT2Gemm16Depth; k++) {
            if (g + k < G) step(g + k, st[k]);
            fetch(min(g + k + kT2Gemm16Depth, G - 1), st[k]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    const int n = n0 + i;
    if (n >= col_begin + ncol) return;
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const int r = m0 + 4 * s + v;
        if (r >= p.rows) continue;
        float y = acc[v];
        if (p.bias && n < p.n_rows) y = y + p.bias[n];
        float *o = p.out + size_t(r) * p.ld_out + (n - col_begin);
        *o = p.accumulate ? *o + y : y;
    }
}

template <bool FUSED>
int launch_t2_gemm16(const T2Params &p, hipStream_t s)
{
    const long tiles = long((p.quad_end - p.quad_begin) * 4 + 15) / 16 * ((p.rows + 15) / 16);
    t2_gemm16_kernel<FUSED><<<unsigned(tiles), 64, size_t(p.G) * 16 * 8, s>>>(p);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

template <int R, bool FUSED>
int launch_t2_rows(const T2Params &p, size_t lds, hipStream_t s)
{
    const unsigned gx = unsigned((p.quad_end - p.quad_begin + 3) / 4), gy = unsigned((p.rows + R - 1) / R);
    t2_rows_kernel<R, FUSED><<<dim3(gx, gy), 256, lds, s>>>(p);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

template <int R>
int launch_t2_rows(const T2Params &p, bool fused, hipStream_t s)
{
    const size_t lds = t2_lds_bytes(R, p.K, p.G, fused);
    return fused ? launch_t2_rows<R, true>(p, lds, s) : launch_t2_rows<R, false>(p, lds, s);
}

}  // namespace

// Workspaces come from a stream-ordered pool per device that keeps freed memory for the next
// product: the device's default pool hands it back to the driver at synchronizations, and a new
// allocation then costs more than a large product. The pools live as long as the process.
hipError_t workspace_alloc(void **ptr, size_t bytes, hipStream_t s)
{
    static std::mutex mu;
    static hipMemPool_t pools[64] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipMallocAsync(ptr, bytes, s);
    hipMemPool_t pool = nullptr;
    {
        std::lock_guard<std::mutex> lock(mu);
        if (!pools[dev]) {
            hipMemPoolProps props{};
            props.allocType = hipMemAllocationTypePinned;
            props.location.type = hipMemLocationTypeDevice;
            props.location.id = dev;
            e = hipMemPoolCreate(&pools[dev], &props);
            if (e != hipSuccess) {
                pools[dev] = nullptr;
                return e;
            }
            uint64_t keep = UINT64_MAX;
            (void)hipMemPoolSetAttribute(pools[dev], hipMemPoolAttrReleaseThreshold, &keep);
        }
        pool = pools[dev];
    }
    return hipMallocFromPoolAsync(ptr, bytes, pool, s);
}

// Which kernel a batched product runs, and the scratch it needs: the levels, scales and
// corrections of f32 rows it quantizes first, and the block-major copy of the activation scales
// (as_t [G][Mpad]) when the kernel reads that rather than staging a tile's scales itself. Each
// part starts on a 256-byte boundary.
struct ScratchPlan {
    size_t q_bytes, s_bytes, t_bytes;
    bool lds;    // the register-ring kernels stage the tile's scales in LDS
    int tiles;   // 0: the register-ring kernels; else the LDS-staged kernel, 10·WM + WN
    int Mpad;    // rows of as_t
    size_t total() const { return q_bytes + 2 * s_bytes + t_bytes; }
};

// The kernel of a batched product: 0 for the register-ring kernels, else the LDS-staged kernel's
// tile shape. FG_GEMM_TILE (0, 11 or 21) overrides the choice, for tests and measurements.
static int choose_tiles(const ProductArgs &a)
{
    const fg_table *t = a.t;
    if (a.dots || t->dtype == FG_T2B128 || a.rows <= 16) return 0;
    if (const char *env = getenv("FG_GEMM_TILE")) {
        const int v = atoi(env);
        if (v == 0 || v == 11 || v == 21) return v;
    }
    const long ncols = long(a.quad_end - a.quad_begin) * 4;
    const long narrow = ((ncols + 31) / 32) * ((long(a.rows) + 31) / 32);
    const size_t split_smem = split_lds_bytes(int(t->groups));
    // few 32 x 32 tiles: four waves per tile over alternate groups (gemm_split_kernel), or for the
    // fused scaling one wave per tile (gemm_kernel)
    if (narrow < 2048 && (a.fused || (t->groups % 4 == 0 && split_smem <= 64 * 1024))) return 0;
    // 64 x 64 workgroup tiles: 128 x 64 measured 3-6 % slower on the DiT block's 4096-row
    // products, 15-17 % at 512 x 896 -> 9728 and 8192 x 4608 -> 1152, tied at 16384 x 1152 ->
    // 4608. Over at most four blocks (the int8 attention's scores, 4096 x 96 -> 4096 per head) the
    // 128 x 64 tiles are kept while they still make 1536 workgroups: 0.96 against 1.00 ms per call.
    const long tiles21 = ((ncols + 63) / 64) * ((long(a.rows) + 127) / 128);
    return t->blocks <= 4 && tiles21 >= 1536 ? 21 : 11;
}

ScratchPlan plan_scratch(const ProductArgs &a)
{
    const fg_table *t = a.t;
    const size_t M = a.rows, K = t->cols, G = t->groups;
    ScratchPlan pl{};
    pl.q_bytes = a.x ? (M * K + 255) / 256 * 256 : 0;
    // f32 rows quantized into row-major scales and corrections (quantize_rows), unless they go
    // straight into the block-major copy (then no row-major scales are written)
    const size_t row_scales = a.x ? (M * G * 4 + 255) / 256 * 256 : 0;
    pl.Mpad = int((M + 63) / 64 * 64);
    if (t->dtype == FG_T2B128) {
        pl.lds = true;
        pl.s_bytes = row_scales;
        return pl;
    }
    pl.tiles = choose_tiles(a);
    if (pl.tiles) {
        // the staged kernel reads whole tiles of as_t (rows padded to 128), which f32 rows are
        // quantized straight into; pre-quantized rows' own [M][G] scales it reads as they are
        pl.Mpad = int((M + 127) / 128 * 128);
        pl.t_bytes = a.x ? G * size_t(pl.Mpad) * 4 : 0;
        return pl;
    }
    // The activation scales go to LDS per tile when a tile's fit in 64 KiB and their rows are
    // whole float4s; otherwise the kernel reads a block-major copy.
    const bool dots = a.dots != nullptr;
    pl.lds = !dots && G * 32 * 4 <= 64 * 1024 && G % 4 == 0 && (a.x || (reinterpret_cast<uintptr_t>(a.as) & 15) == 0);
    pl.t_bytes = (pl.lds || dots) ? 0 : G * size_t(pl.Mpad) * 4;
    pl.s_bytes = pl.t_bytes ? 0 : row_scales;
    return pl;
}

// Scratch of a product captured into a graph: allocated once, while the capture is recorded, by a
// plain allocation outside the stream's work (so the graph holds no allocation or free node and a
// replay allocates nothing), and owned by the graph through a user object. The object's
// destructor, which runs when the graph and its instances are gone and may make no HIP call, hands
// the memory back; the library frees it on its next scratch request outside a capture.
static std::mutex g_retired_mu;
static std::vector<void *> g_retired;

static void retire_scratch(void *p)
{
    std::lock_guard<std::mutex> lock(g_retired_mu);
    g_retired.push_back(p);
}

static void free_retired()
{
    std::vector<void *> done;
    {
        std::lock_guard<std::mutex> lock(g_retired_mu);
        done.swap(g_retired);
    }
    for (void *p : done) (void)hipFree(p);
}

// *captured: `s` is capturing, and *ws then holds scratch the capture's graph owns.
static hipError_t captured_scratch(hipStream_t s, size_t bytes, void **ws, bool *captured)
{
    *captured = false;
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamGetCaptureInfo_v2(s, &status, nullptr, &graph, nullptr, nullptr);
    if (e != hipSuccess) return e;
    if (status != hipStreamCaptureStatusActive) return hipSuccess;
    *captured = true;
    if (!graph) return hipErrorStreamCaptureInvalidated;
    // an allocation is not stream work: allowed for this thread whatever mode the capture runs in
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    e = hipThreadExchangeStreamCaptureMode(&mode);
    if (e != hipSuccess) return e;
    void *p = nullptr;
    const hipError_t ea = hipMalloc(&p, bytes);
    (void)hipThreadExchangeStreamCaptureMode(&mode);
    if (ea != hipSuccess) return ea;
    hipUserObject_t obj = nullptr;
    e = hipUserObjectCreate(&obj, p, retire_scratch, 1, hipUserObjectNoDestructorSync);
    if (e != hipSuccess) {
        (void)hipFree(p);
        return e;
    }
    e = hipGraphRetainUserObject(graph, obj, 1, hipGraphUserObjectMove);
    if (e != hipSuccess) {
        (void)hipUserObjectRelease(obj, 1);  // the destructor retires the memory
        return e;
    }
    *ws = p;
    return hipSuccess;
}

// The caller's scratch when it brings one; under graph capture scratch the graph owns; else a pool
// allocation (freed by the caller of this function on the stream once the product is queued).
hipError_t scratch_for(const ProductArgs &a, size_t bytes, hipStream_t s, void **ws, bool *owned)
{
    *ws = nullptr;
    *owned = false;
    if (!bytes) return hipSuccess;
    if (a.workspace) {
        if (bytes > a.workspace_bytes) return hipErrorInvalidValue;  // checked by the entry point first
        *ws = a.workspace;
        return hipSuccess;
    }
    bool captured = false;
    const hipError_t e = captured_scratch(s, bytes, ws, &captured);
    if (e != hipSuccess || captured) return e;
    free_retired();
    *owned = true;
    return workspace_alloc(ws, bytes, s);
}

int launch_t2(const ProductArgs &a, hipStream_t s)
{
    const fg_table *t = a.t;
    const int M = int(a.rows), K = int(t->cols), G = int(t->groups);
    const int col_begin = int(a.quad_begin * 4), ncols = int((a.quad_end - a.quad_begin) * 4);
    int8_t *q = const_cast<int8_t *>(a.q);
    const float *as = a.as;
    const int32_t *corr = a.corr;
    void *ws = nullptr;
    bool owned = false;
    int rc = FG_OK;
    if (a.x) {  // quantize the f32 rows first (groups of 128)
        const ScratchPlan pl = plan_scratch(a);
        const size_t qb = pl.q_bytes, sb = pl.s_bytes;
        FG_HIP(scratch_for(a, pl.total(), s, &ws, &owned));
        q = static_cast<int8_t *>(ws);
        float *sc = reinterpret_cast<float *>(static_cast<char *>(ws) + qb);
        int32_t *co = reinterpret_cast<int32_t *>(static_cast<char *>(ws) + qb + sb);
        rc = launch_quantize_rows(a.x, size_t(M) * K, FG_T2B128, q, sc, co, s);
        as = sc;
        corr = co;
    }
    // the matrix cores for many rows, the streamed kernel for few (the int32 dots stay on the
    // one-thread-per-output kernel)
    const bool fused = a.fused != 0;
    // 5-16 rows take the 16 x 16 tiles over many columns; over few the tiles are too few waves and
    // the streamed kernel's row slices are faster (896 x 4864 at 5-16 rows: 6.1 against 9.4 us;
    // 4096 x 1024: 3.7 against 4.0 at 5-8 rows, 4.4 against 4.3 at 12; 14336 x 4096 at 5 rows:
    // 9.6 against 15.3)
    const int ctiles = (ncols + 15) / 16;
    const bool tiles16 = M >= kT2Gemm16Rows && M <= kT2Gemm16MaxRows && (ctiles >= 300 || (M >= 9 && ctiles >= 256));
    if (rc == FG_OK && !a.dots && (tiles16 || M >= kT2GemmRows) && size_t(G) * 32 * 8 <= 64 * 1024 &&
        (reinterpret_cast<uintptr_t>(q) & 15) == 0) {
        T2Params p{};
        p.codes = reinterpret_cast<const uint8_t *>(t->codes);
        p.wscales = t->scales;
        p.B = int(t->blocks);
        p.G = G;
        p.K = K;
        p.n_rows = int(t->rows);
        p.q = q;
        p.as = as;
        p.corr = corr;
        p.rows = M;
        p.quad_begin = int(a.quad_begin);
        p.quad_end = int(a.quad_end);
        p.col_begin = col_begin;
        p.bias = a.bias;
        p.out = a.out;
        p.ld_out = long(a.ld_out);
        p.accumulate = a.accumulate;
        if (tiles16)
            rc = fused ? launch_t2_gemm16<true>(p, s) : launch_t2_gemm16<false>(p, s);
        else
            rc = fused ? launch_t2_gemm<true>(p, s) : launch_t2_gemm<false>(p, s);
        if (owned) {
            hipError_t e = hipFreeAsync(ws, s);
            if (rc == FG_OK && e != hipSuccess) rc = check_hip(e, "hipFreeAsync");
        }
        return rc;
    }
    // slices of up to four rows (5-16 rows take the 16 x 16 tiles above unless the groups are too
    // many for them, and then the levels of four rows already overflow the LDS)
    int R = M >= 3 ? 4 : M;
    while (R > 1 && t2_lds_bytes(R, K, G, fused) > 64 * 1024) R /= 2;
    if (rc == FG_OK && !a.dots && M > 0 && t2_lds_bytes(R, K, G, fused) <= 64 * 1024 && (reinterpret_cast<uintptr_t>(q) & 15) == 0 &&
        (M + R - 1) / R <= 65535) {
        T2Params p{};
        p.codes = reinterpret_cast<const uint8_t *>(t->codes);
        p.wscales = t->scales;
        p.B = int(t->blocks);
        p.G = G;
        p.K = K;
        p.n_rows = int(t->rows);
        p.q = q;
        p.as = as;
        p.corr = corr;
        p.rows = M;
        p.quad_begin = int(a.quad_begin);
        p.quad_end = int(a.quad_end);
        p.col_begin = col_begin;
        p.bias = a.bias;
        p.out = a.out;
        p.ld_out = long(a.ld_out);
        p.accumulate = a.accumulate;
        rc = R == 4   ? launch_t2_rows<4>(p, fused, s)
             : R == 2 ? launch_t2_rows<2>(p, fused, s)
                      : launch_t2_rows<1>(p, fused, s);
    } else if (rc == FG_OK) {
        const long n = long(M) * ncols;
        t2_product_kernel<<<unsigned((n + 255) / 256), 256, 0, s>>>(reinterpret_cast<const uint8_t *>(t->codes), t->scales, int(t->blocks),
                                                                   G, K, int(t->rows), q, as, corr, M, col_begin, ncols, a.bias,
                                                                   a.out, long(a.ld_out), a.accumulate, a.dots, a.fused);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) rc = check_hip(e, "t2_product_kernel");
    }
    if (owned) {
        hipError_t e = hipFreeAsync(ws, s);
        if (rc == FG_OK && e != hipSuccess) rc = check_hip(e, "hipFreeAsync");
    }
    return rc;
}

template <int WM, int WN>
int launch_batch_as(const GemmParams &p, int items, hipStream_t s)
{
    using T = LdsTile<8, WM, WN>;
    const long groups = long((p.col_end - p.col_begin + T::BN - 1) / T::BN) * ((p.M + T::BM - 1) / T::BM);
    gemm_lds_kernel<8, WM, WN, false><<<dim3(unsigned(groups), unsigned(items)), 256, 2 * size_t(T::STAGE), s>>>(p);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

int launch_gemm_batch(const ProductArgs &a, int items, int per_table, int first, size_t q_stride, size_t as_stride,
                      size_t out_stride, size_t codes_stride, size_t scales_stride, hipStream_t s)
{
    const fg_table *t = a.t;
    if (items < 1 || per_table < 1 || first < 0 || !a.q || !a.as || a.x || a.dots || a.fused || a.accumulate || a.as_t || a.bias ||
        (t->dtype != FG_Q7B32 && t->dtype != FG_Q8B32) || a.rows < 1 || a.quad_end <= a.quad_begin)
        return set_error(FG_ERR_ARG, "a batch of products takes pre-quantized rows and a Q7b32 or Q8b32 table");
    if (items > 65535) return set_error(FG_ERR_SHAPE, "at most 65535 products in a batch");
    GemmParams p{};
    p.codes = t->codes;
    p.wscales = t->scales;
    p.B = int(t->blocks);
    p.G = int(t->groups);
    p.K = int(t->cols);
    p.M = int(a.rows);
    p.Mpad = int((a.rows + 127) / 128 * 128);
    p.col_begin = int(a.quad_begin * 4);
    p.col_end = int(a.quad_end * 4);
    p.n_rows = int(t->rows);
    p.q = a.q;
    p.as = a.as;
    p.out = a.out;
    p.ld_out = long(a.ld_out);
    p.q_batch = long(q_stride);
    p.as_batch = long(as_stride);
    p.out_batch = long(out_stride);
    p.codes_batch = long(codes_stride);
    p.wscales_batch = long(scales_stride);
    p.per_table = per_table;
    p.first = first;
    // workgroup tiles 64 wide, or 128 wide past 64 columns so each row tile's levels are read
    // once (the attention's 72 value channels: 1.043 -> 1.009 ms per call at the DiT shape)
    if (p.col_end - p.col_begin > 64) return launch_batch_as<1, 2>(p, items, s);
    return launch_batch_as<1, 1>(p, items, s);
}

int launch_gemm(const ProductArgs &a, hipStream_t s)
{
    const fg_table *t = a.t;
    if (t->dtype == FG_T2B128) return launch_t2(a, s);
    const int M = int(a.rows), K = int(t->cols), G = int(t->groups);
    const bool dots = a.dots != nullptr;
    // Workspace: levels, scales and corrections (when the input is f32), block-major scales.
    const ScratchPlan pl = plan_scratch(a);
    const int Mpad = pl.Mpad;
    const bool lds = pl.lds;
    const size_t q_bytes = pl.q_bytes, s_bytes = pl.s_bytes, t_bytes = pl.t_bytes;
    void *ws = nullptr;
    bool owned = false;
    FG_HIP(scratch_for(a, pl.total(), s, &ws, &owned));
    int8_t *q = const_cast<int8_t *>(a.q);
    const float *as = a.as;
    char *base = static_cast<char *>(ws);
    int rc = FG_OK;
    float *as_t = reinterpret_cast<float *>(base + q_bytes + 2 * s_bytes);
    // the kernels that read block-major scales read only them: f32 rows are quantized straight
    // into that form, and pre-quantized rows that bring it are not transposed again
    const bool caller_t = !a.x && a.as_t && a.as_t_rows == size_t(Mpad);
    if (a.x) {
        q = reinterpret_cast<int8_t *>(base);
        if (t_bytes) {
            rc = launch_quantize_rows_t(a.x, size_t(M), size_t(K), t->dtype, q, as_t, size_t(Mpad), s);
        } else {
            float *sc = reinterpret_cast<float *>(base + q_bytes);
            int32_t *co = reinterpret_cast<int32_t *>(base + q_bytes + s_bytes);
            rc = launch_quantize_rows(a.x, size_t(M) * K, t->dtype, q, sc, co, s);
            as = sc;
        }
    } else if (t_bytes && !caller_t) {
        const size_t n = size_t(G) * Mpad;
        transpose_scales_kernel<<<unsigned((n + 255) / 256), 256, 0, s>>>(as, M, G, Mpad, as_t);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) rc = check_hip(e, "transpose_scales_kernel");
    }
    const float *as_block = caller_t ? a.as_t : (t_bytes ? as_t : nullptr);
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
        p.as = as;
        p.as_t = as_block;
        p.bias = a.bias;
        p.out = a.out;
        p.ld_out = long(a.ld_out);
        p.accumulate = a.accumulate;
        p.dots = a.dots;
        p.dots_cols = p.col_end - p.col_begin;
        if (pl.tiles)
            rc = t->dtype == FG_Q4B32 ? launch_lds<4>(p, pl.tiles, a.fused != 0, s) : launch_lds<8>(p, pl.tiles, a.fused != 0, s);
        else
            rc = t->dtype == FG_Q4B32 ? launch_tiles<4>(p, dots, lds, a.fused != 0, s) : launch_tiles<8>(p, dots, lds, a.fused != 0, s);
    }
    if (owned) {
        hipError_t e = hipFreeAsync(ws, s);
        if (rc == FG_OK && e != hipSuccess) rc = check_hip(e, "hipFreeAsync");
    }
    return rc;
}

// Rows 1..4 stream the weights once through the matrix-vector kernel; more rows (and the fused
// scaling) go to the matrix cores.
static bool on_matvec(const ProductArgs &a)
{
    // the matrix-vector kernel sums separately rounded terms; the fused scaling runs on the tiles
    return a.t->dtype != FG_T2B128 && a.rows <= 4 && !a.fused;
}

// Two products of the same pre-quantized rows over tables of one shape and format (a layer's gate
// and up): one launch of the split kernel over both when that is the kernel each would take, else
// one launch each.
int launch_product_pair(const ProductArgs &a, const ProductArgs &b, hipStream_t s)
{
    const fg_table *t = a.t, *u = b.t;
    const long ncols = long(a.quad_end - a.quad_begin) * 4;
    const long narrow = ((ncols + 31) / 32) * ((long(a.rows) + 31) / 32);
    const size_t split_smem = split_lds_bytes(int(t->groups));
    const bool split = t->dtype == u->dtype && t->cols == u->cols && t->rows == u->rows && a.rows == b.rows && a.q == b.q &&
                       a.as == b.as && a.q && !a.x && !b.x && !a.dots && !b.dots && !a.fused && !b.fused && !a.bias && !b.bias &&
                       !a.workspace && !b.workspace && a.quad_begin == b.quad_begin && a.quad_end == b.quad_end &&
                       a.accumulate == b.accumulate && a.ld_out == b.ld_out &&
                       (t->dtype == FG_Q7B32 || t->dtype == FG_Q8B32 || t->dtype == FG_Q4B32) && a.rows > 16 &&
                       !on_matvec(a) && choose_tiles(a) == 0 && t->groups % 4 == 0 && t->groups * 32 * 4 <= 64 * 1024 &&
                       (reinterpret_cast<uintptr_t>(a.as) & 15) == 0 && narrow < 2048 && split_smem <= 64 * 1024 &&
                       !(a.rows <= 256 && t->blocks >= 64) && 2 * narrow < (long(1) << 31);
    if (!split) {
        const int rc = launch_product(a, s);
        return rc ? rc : launch_product(b, s);
    }
    GemmParams p{};
    p.codes = t->codes;
    p.wscales = t->scales;
    p.B = int(t->blocks);
    p.G = int(t->groups);
    p.K = int(t->cols);
    p.M = int(a.rows);
    p.Mpad = int((a.rows + 63) / 64 * 64);
    p.col_begin = int(a.quad_begin * 4);
    p.col_end = int(a.quad_end * 4);
    p.n_rows = int(t->rows);
    p.q = a.q;
    p.as = a.as;
    p.out = a.out;
    p.ld_out = long(a.ld_out);
    p.accumulate = a.accumulate;
    p.codes2 = u->codes;
    p.wscales2 = u->scales;
    p.out2 = b.out;
    p.tiles1 = int(narrow);
    if (t->dtype == FG_Q4B32) launch_split<4>(p, unsigned(2 * narrow), s);
    else launch_split<8>(p, unsigned(2 * narrow), s);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

int launch_product(const ProductArgs &a, hipStream_t s)
{
    if (a.rows == 0 || a.quad_end <= a.quad_begin) return FG_OK;
    if (a.t->dtype == FG_T2B128) return launch_t2(a, s);
    if (on_matvec(a)) return launch_matvec(a, s);
    return launch_gemm(a, s);
}

size_t product_scratch_bytes(const ProductArgs &a)
{
    if (a.rows == 0 || a.quad_end <= a.quad_begin || on_matvec(a)) return 0;
    return plan_scratch(a).total();
}

}  // namespace fg
