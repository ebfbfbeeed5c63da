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

#include <algorithm>
#include <cmath>
#include <cstdlib>

namespace fg {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxRowBytes = 64 * 1024;  // one padded score row in LDS: at most 16384 keys
constexpr int kMaxHeadDim = 1024;

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

// keyT[(t · hd + d) · kpad + k] = key[k][d] of table t = image · kv_heads + kh: the keys of every
// (image, key head) with channels as rows, through 64 x 64 tiles in LDS (both sides coalesced).
__global__ __launch_bounds__(256) void key_transpose_kernel(const float *__restrict__ key, size_t stride, size_t offset,
                                                            int kv_heads, int keys, int hd, int kpad,
                                                            float *__restrict__ keyT)
{
    __shared__ float tile[64][65];
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const int k0 = blockIdx.x * 64, d0 = blockIdx.y * 64;
    const size_t t = blockIdx.z, image = t / kv_heads, kh = t % kv_heads;
    const float *src = key + image * size_t(keys) * stride + offset + kh * size_t(hd);
    for (int kk = ty; kk < 64; kk += 4) {
        const int k = k0 + kk, d = d0 + tx;
        if (k < keys && d < hd) tile[kk][tx] = src[size_t(k) * stride + d];
    }
    __syncthreads();
    for (int dd = ty; dd < 64; dd += 4) {
        const int d = d0 + dd, k = k0 + tx;
        if (k < keys && d < hd) keyT[(t * hd + d) * size_t(kpad) + k] = tile[tx][dd];
    }
}

// mean[t · hd + d] = (Σ over the keys in order of key[k][d]) / keys, from the transposed keys:
// one wave per (table, channel) brings the channel's keys into LDS, sixteen coalesced loads of
// 256 keys in flight, then its first lane adds them in key order (the reference's sequential sum).
__global__ __launch_bounds__(64) void key_mean_kernel(const float *__restrict__ keyT, int keys, int kpad,
                                                      float *__restrict__ mean)
{
    extern __shared__ __align__(16) float column[];  // [keys rounded up to 4096]
    const int lane = threadIdx.x;
    const size_t id = blockIdx.x;
    const v4f *src = reinterpret_cast<const v4f *>(keyT + id * size_t(kpad));
    v4f *col4 = reinterpret_cast<v4f *>(column);
    const int n4 = kpad / 4;
    for (int s0 = 0; s0 < n4; s0 += 1024) {
        v4f v[16];
#pragma unroll
        for (int u = 0; u < 16; u++) v[u] = src[min(s0 + 64 * u + lane, n4 - 1)];
#pragma unroll
        for (int u = 0; u < 16; u++) col4[s0 + 64 * u + lane] = v[u];
    }
    __syncthreads();
    if (lane == 0) {
        float s = 0.0f;
        int k = 0;
        for (; k + 16 <= keys; k += 16) {
            v4f x[4];
#pragma unroll
            for (int u = 0; u < 4; u++) x[u] = col4[k / 4 + u];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                s = s + x[u].x;
                s = s + x[u].y;
                s = s + x[u].z;
                s = s + x[u].w;
            }
        }
        for (; k < keys; k++) s = s + column[k];
        mean[id] = s / float(keys);
    }
}

// The cleared row-block of a run-time Q7b32 matrix (QuantizedMatrix::extend's padding rows):
// zero codes (device levels −64) and a zero scale.
__device__ __forceinline__ void clear_block(int8_t *codes32, float *scale)
{
    int4 *dst = reinterpret_cast<int4 *>(codes32);
    const int v = int(0xC0C0C0C0u);
    dst[0] = make_int4(v, v, v, v);
    dst[1] = make_int4(v, v, v, v);
    *scale = 0.0f;
}

// Q7b32 levels of four values at scale d (quant.rs:143-150: rne(x / d) clamped to ±63 through the
// saturating cast), packed as one dword of device levels.
__device__ __forceinline__ int q7_levels4(const float (&x)[4], float d)
{
    int l[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float v = __builtin_rintf(x[j] / d);
        const int level = v != v ? 0 : v >= 127.0f ? 127 : v <= -128.0f ? -128 : int(v);
        l[j] = level < -63 ? -63 : (level > 63 ? 63 : level);
    }
    return pack4(l[0], l[1], l[2], l[3]);
}

// Scratch::quantize's key matrices (attention.rs:100-118) for every (image, key head) at once:
// row k of table t is key[k] − mean over the channels, zeros to the padded width; rows past the
// keys to the quad are cleared. Eight aligned lanes per (table, row, block), four channels each,
// the block's largest magnitude by lane exchanges (q7_block's arithmetic). Indices in 32 bits:
// the host keeps the lane count below 2^31.
__global__ __launch_bounds__(256) void key_table_kernel(const float *__restrict__ key, size_t stride, size_t offset,
                                                        int kv_heads, int keys, int hd, int rows4, int blocks,
                                                        const float *__restrict__ mean, int8_t *__restrict__ codes,
                                                        float *__restrict__ scales, unsigned groups)
{
    const unsigned lid = blockIdx.x * 256u + threadIdx.x, sub = lid & 7u;
    const unsigned g = min(lid >> 3, groups - 1);  // past the end: the last group again, never stored
    const unsigned b = g % unsigned(blocks), rb = g / unsigned(blocks), row = rb % unsigned(rows4),
                   t = rb / unsigned(rows4);
    const size_t tb = (size_t(t) * unsigned(rows4 / 4) + row / 4) * unsigned(blocks) + b;  // quad block of the tables' run
    int *dst = reinterpret_cast<int *>(codes + tb * 128 + (row % 4) * 32);
    float *scale = scales + tb * 4 + row % 4;
    const bool live = int(row) < keys;
    const unsigned image = t / unsigned(kv_heads), kh = t % unsigned(kv_heads);
    const float *src = key + (size_t(image) * unsigned(keys) + min(int(row), keys - 1)) * stride + offset + size_t(kh) * hd;
    const float *mu = mean + size_t(t) * hd;
    float x[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int d = 32 * int(b) + 4 * int(sub) + j;
        x[j] = d < hd ? src[d] - mu[d] : 0.0f;
    }
    float amax = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
    amax = max8(fmaxf(0.0f, amax));
    const float d = group_scale(amax, 63.0f);
    const int packed = q7_levels4(x, d);
    if ((lid >> 3) >= groups) return;
    // rows past the keys: the cleared block (QuantizedMatrix::extend's padding rows), zero codes
    // (device levels −64) and a zero scale
    dst[sub] = live ? packed : int(0xC0C0C0C0u);
    if (sub == 0) *scale = live ? d : 0.0f;
}

// Scratch::quantize's value matrices (Scratch::transpose, attention.rs:119-137) for every
// (image, key head): row d of table t holds value[k][d] over the keys k, zeros to the padded
// width; rows past head_dim to the quad are cleared. One thread per (table, block, row), rows
// fastest so neighbouring threads read neighbouring channels.
__global__ void value_table_kernel(const float *__restrict__ value, size_t stride, size_t offset, int kv_heads,
                                   int keys, int hd, int rows4, int blocks, int8_t *__restrict__ codes,
                                   float *__restrict__ scales, unsigned n)
{
    const unsigned id = blockIdx.x * blockDim.x + threadIdx.x;  // 32-bit: the host keeps n below 2^31
    if (id >= n) return;
    const int row = int(id % unsigned(rows4));
    const unsigned rb = id / unsigned(rows4), b = rb % unsigned(blocks), t = rb / unsigned(blocks);
    const size_t tb = (size_t(t) * unsigned(rows4 / 4) + row / 4) * unsigned(blocks) + b;
    int8_t *dst = codes + tb * 128 + (row % 4) * 32;
    float *scale = scales + tb * 4 + row % 4;
    if (row >= hd) {
        clear_block(dst, scale);
        return;
    }
    const unsigned image = t / unsigned(kv_heads), kh = t % unsigned(kv_heads);
    const float *src = value + size_t(image) * unsigned(keys) * stride + offset + size_t(kh) * hd + row;
    float x[32];
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const int k = 32 * int(b) + i;
        x[i] = k < keys ? src[size_t(k) * stride] : 0.0f;
    }
    *scale = q7_block(x, reinterpret_cast<int *>(dst));
}

// The queries of every (image, head), quantized as the product quantizes its rows (quantize_rows,
// matmul.rs:233-257, for a Q7b32 matrix: zero point 64) over the padded width pd, zeros past
// head_dim: levels [u][r][pd], scales and corrections [u][r][pd / 32], and when `tscales` is set
// the scales block-major as well, [u][pd / 32][queries] (the form the scores' product reads).
// Eight lanes per group of 32.
__global__ __launch_bounds__(256) void query_levels_kernel(const float *__restrict__ query, size_t stride,
                                                           size_t offset, int heads, int queries, int hd, int pd,
                                                           unsigned slots, int8_t *__restrict__ levels,
                                                           float *__restrict__ lscales, int32_t *__restrict__ lcorr,
                                                           float *__restrict__ tscales)
{
    const unsigned id = blockIdx.x * blockDim.x + threadIdx.x;  // 32-bit: the host keeps slots below 2^31
    const unsigned per_row = unsigned(pd / 4);
    const bool active = id < slots;
    const int s4 = int(id % per_row);
    const unsigned rrq = id / per_row;  // u · queries + r
    const size_t rr = rrq;
    const unsigned u = rrq / unsigned(queries), r = rrq % unsigned(queries);
    v4f v{0.0f, 0.0f, 0.0f, 0.0f};
    if (active && 4 * s4 < hd) {
        const unsigned image = u / unsigned(heads), h = u % unsigned(heads);
        const float *src = query + (size_t(image) * unsigned(queries) + r) * stride + offset + size_t(h) * hd + 4 * s4;
        v = v4f{src[0], src[1], src[2], src[3]};
    }
    Group8 gr[1];
    quantize_groups<1>(&v, gr);
    if (active) store_group8(gr[0], 64, s4 / 8, levels + rr * pd, lscales + rr * (pd / 32), lcorr + rr * (pd / 32));
    if (tscales && active && (threadIdx.x & 7) == 0) tscales[(size_t(u) * (pd / 32) + s4 / 8) * unsigned(queries) + r] = gr[0].d;
}

// One workgroup of four waves per query row; thread t holds slots t, t + 256, ... (S of them, four
// scores each) in registers: the row's scores (product · scale below keys4, zeros to pk), their
// maximum over the first `keys`, the exponentials there, and the row quantized straight from
// the registers for the product with the values (quantize_rows over the whole padded width for a
// Q7b32 matrix, zero point 64: eight consecutive slots are eight aligned lanes, and the S groups
// of a thread are independent streams the scheduler interleaves). The exponentials also go to
// LDS, where after one barrier lanes 0..7 of the first wave sum them in the scalar backend's order
// (scalar.rs:117-126, ops.rs:170-175): lane o sums offset o over the whole runs of eight in
// order, lane 0 adds the rest in order, then the eight offset sums in order. Per-element bounds
// are selects, not branches.
template <bool FAST, int S>
__global__ __launch_bounds__(256) void exponentials_kernel(const float *__restrict__ prod, int keys4, float scale,
                                                           int keys, int pk, int8_t *__restrict__ levels,
                                                           float *__restrict__ level_scales, int32_t *__restrict__ level_corr,
                                                           float *__restrict__ sums)
{
    extern __shared__ __align__(16) float row[];  // [pk], then the four waves' maxima
    float *wmax = row + pk;
    v4f *row4 = reinterpret_cast<v4f *>(row);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t r = blockIdx.x;
    const int n4 = pk / 4, k4 = keys4 / 4;
    const v4f *src = reinterpret_cast<const v4f *>(prod + r * keys4);
    v4f v[S];
#pragma unroll
    for (int k = 0; k < S; k++) v[k] = src[min(tid + 256 * k, k4 - 1)];
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < S; k++) {
        const int slot = tid + 256 * k, i = 4 * slot;
        const v4f x = slot < k4 ? v4f{v[k].x * scale, v[k].y * scale, v[k].z * scale, v[k].w * scale}
                                : v4f{0.0f, 0.0f, 0.0f, 0.0f};
        v[k] = x;
        m = fmaxf(m, i < keys ? x.x : -INFINITY);
        m = fmaxf(m, i + 1 < keys ? x.y : -INFINITY);
        m = fmaxf(m, i + 2 < keys ? x.z : -INFINITY);
        m = fmaxf(m, i + 3 < keys ? x.w : -INFINITY);
    }
    m = wave_allmax(m);
    if (lane == 0) wmax[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
#pragma unroll
    for (int k = 0; k < S; k++) {
        const int slot = tid + 256 * k, i = 4 * slot;
        v4f e = v[k];
        const float ex = FAST ? ref_exp_fast(e.x - m) : ref_exp(e.x - m);
        const float ey = FAST ? ref_exp_fast(e.y - m) : ref_exp(e.y - m);
        const float ez = FAST ? ref_exp_fast(e.z - m) : ref_exp(e.z - m);
        const float ew = FAST ? ref_exp_fast(e.w - m) : ref_exp(e.w - m);
        e.x = i < keys ? ex : e.x;
        e.y = i + 1 < keys ? ey : e.y;
        e.z = i + 2 < keys ? ez : e.z;
        e.w = i + 3 < keys ? ew : e.w;
        v[k] = e;
        if (slot < n4) row4[slot] = e;
    }
    Group8 gr[S];
    quantize_groups<S>(v, gr);
#pragma unroll
    for (int k = 0; k < S; k++) {
        const int slot = tid + 256 * k;
        if (slot < n4) store_group8(gr[k], 64, slot / 8, levels + r * pk, level_scales + r * (pk / 32), level_corr + r * (pk / 32));
    }
    __syncthreads();  // the exponentials in LDS
    if (wave == 0) {
        const int whole = keys / 8 * 8;
        float part = 0.0f;
        if (lane < 8) {
            // sixteen reads out before their sixteen additions, in run order
            int i = lane;
            for (; i + 8 * 15 < whole; i += 8 * 16) {
                float x[16];
#pragma unroll
                for (int u = 0; u < 16; u++) x[u] = row[i + 8 * u];
#pragma unroll
                for (int u = 0; u < 16; u++) part = part + x[u];
            }
            for (; i < whole; i += 8) part = part + row[i];
        }
        float total = -0.0f;
        if (lane == 0) {
            for (int i = whole; i < keys; i++) total = total + row[i];
        }
#pragma unroll
        for (int o = 0; o < 8; o++) {
            const float po = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), o));
            if (lane == 0) total = total + po;
        }
        if (lane == 0) sums[r] = total;
    }
}

// out[(image · queries + r) · stride + h · hd + d] = pv[u][r][d] / sums[u][r] for every (image,
// head) u = image · heads + h.
__global__ void divide_kernel(const float *__restrict__ pv, const float *__restrict__ sums, int heads, int queries,
                              int hd, unsigned n, float *__restrict__ out, size_t stride)
{
    const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;  // 32-bit: the host keeps n below 2^31
    if (i >= n) return;
    const unsigned ur = i / unsigned(hd), u = ur / unsigned(queries), r = ur % unsigned(queries);
    const unsigned image = u / unsigned(heads), h = u % unsigned(heads), d = i - ur * unsigned(hd);
    out[(size_t(image) * unsigned(queries) + r) * stride + size_t(h) * hd + d] = pv[i] / sums[ur];
}

unsigned blocks_for(size_t n) { return unsigned((n + kThreads - 1) / kThreads); }

// A query row per workgroup; a row of 16384 keys takes 64 KiB and 16 bytes of LDS, past the
// default limit, which is then raised for the kernel on the current device.
template <bool FAST, int S>
int launch_exponentials_s(const float *prod, int keys4, float scale, int keys, int pk, int8_t *levels, float *level_scales,
                          int32_t *level_corr, float *sums, unsigned queries, hipStream_t st)
{
    const size_t smem = size_t(pk) * 4 + 16;
    if (smem > 64 * 1024)
        FG_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(exponentials_kernel<FAST, S>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
    exponentials_kernel<FAST, S><<<queries, 256, smem, st>>>(prod, keys4, scale, keys, pk, levels, level_scales, level_corr, sums);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

// Slots per thread: the fewest powers of two whose 256 threads cover the row's pk / 4 slots.
template <bool FAST>
int launch_exponentials(const float *prod, int keys4, float scale, int keys, int pk, int8_t *levels, float *level_scales,
                        int32_t *level_corr, float *sums, unsigned queries, hipStream_t st)
{
    const int slots = (pk / 4 + 255) / 256;
    if (slots <= 1) return launch_exponentials_s<FAST, 1>(prod, keys4, scale, keys, pk, levels, level_scales, level_corr, sums, queries, st);
    if (slots <= 2) return launch_exponentials_s<FAST, 2>(prod, keys4, scale, keys, pk, levels, level_scales, level_corr, sums, queries, st);
    if (slots <= 4) return launch_exponentials_s<FAST, 4>(prod, keys4, scale, keys, pk, levels, level_scales, level_corr, sums, queries, st);
    if (slots <= 8) return launch_exponentials_s<FAST, 8>(prod, keys4, scale, keys, pk, levels, level_scales, level_corr, sums, queries, st);
    return launch_exponentials_s<FAST, 16>(prod, keys4, scale, keys, pk, levels, level_scales, level_corr, sums, queries, st);
}

// A run-time Q7b32 matrix (QuantizedMatrix) over caller-provided device storage: `rows` rows of
// `cols` values, codes and scales in the device layout.
fg_table runtime_matrix(int8_t *codes, float *scales, size_t rows, size_t cols)
{
    fg_table t{};
    t.dtype = FG_Q7B32;
    t.rows = rows;
    t.cols = cols;
    t.quads = (rows + 3) / 4;
    t.blocks = t.groups = cols / 32;
    t.code_bytes = t.quads * t.blocks * 128;
    t.codes = codes;
    t.scales = scales;
    t.capacity = rows;
    t.max_cols = cols;
    return t;
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// The call's sizes.
struct Shape {
    size_t hd, keys, queries, pd, pk, keys4, kpad, kquads, vquads, ktables, qtables;
    explicit Shape(const fg_attention *c)
        : hd(c->head_dim), keys(c->keys), queries(c->queries), pd(pad32(hd)), pk(pad32(keys)), keys4((keys + 3) / 4 * 4),
          kpad(keys4), kquads((keys + 3) / 4), vquads((hd + 3) / 4), ktables(c->images * c->kv_heads),
          qtables(c->images * c->heads)
    {
    }
};

// (image, head) units per batch of the weighted values' product: as many as keep their
// exponentials' levels, scales and corrections within 512 MiB, at least one. FG_ATTEND_UNITS
// sets a smaller batch, for tests of the batches' edges.
size_t units_per_batch(const Shape &s)
{
    const size_t per = s.queries * s.pk + 2 * s.queries * (s.pk / 32) * 4;
    size_t n = std::max<size_t>(1, std::min<size_t>(s.qtables, (size_t(512) << 20) / per));
    if (const char *env = getenv("FG_ATTEND_UNITS")) {
        const long v = atol(env);
        if (v >= 1) n = std::min(n, size_t(v));
    }
    return n;
}

// The call's scratch, carved from one allocation of the product's stream-ordered workspace pool:
// no allocation reaches the driver and nothing waits for the stream. The key and value matrices
// of every (image, key head) and the quantized queries of every (image, head) are built up front;
// the scores are per head, their levels per batch of heads, the products' outputs per call.
struct Scratch {
    enum { KEYT, MEAN, KCODES, KSCALES, VCODES, VSCALES, QLEVELS, QSCALES, QCORR, QTSCALES, PROD, ELEVELS, ESCALES, ECORR, SUMS, PV, N };
    size_t size[N];
    void *part[N];
    explicit Scratch(const Shape &s)
    {
        const size_t batch = units_per_batch(s);
        size[KEYT] = s.ktables * s.hd * s.kpad * 4;
        size[MEAN] = s.ktables * s.hd * 4;
        size[KCODES] = s.ktables * s.kquads * (s.pd / 32) * 128;
        size[KSCALES] = s.ktables * s.kquads * (s.pd / 32) * 16;
        size[VCODES] = s.ktables * s.vquads * (s.pk / 32) * 128;
        size[VSCALES] = s.ktables * s.vquads * (s.pk / 32) * 16;
        size[QLEVELS] = s.qtables * s.queries * s.pd;
        size[QSCALES] = size[QCORR] = s.qtables * s.queries * (s.pd / 32) * 4;
        size[QTSCALES] = s.queries % 128 == 0 ? size[QSCALES] : 0;  // block-major, whole tiles of rows only
        size[PROD] = s.queries * s.keys4 * 4;
        size[ELEVELS] = batch * s.queries * s.pk;
        size[ESCALES] = size[ECORR] = batch * s.queries * (s.pk / 32) * 4;
        size[SUMS] = s.qtables * s.queries * 4;
        size[PV] = s.qtables * s.queries * s.hd * 4;
    }
    size_t total() const
    {
        size_t n = 0;
        for (size_t b : size) n += align256(b);
        return n;
    }
    void carve(void *ws)
    {
        char *at = static_cast<char *>(ws);
        for (int i = 0; i < N; i++) {
            part[i] = at;
            at += align256(size[i]);
        }
    }
    template <class T> T *at(int i) const { return static_cast<T *>(part[i]); }
};

int run(const fg_attention *c, float *out, hipStream_t st, const Shape &s, const Scratch &w)
{
    const int hd = int(s.hd), keys = int(s.keys), queries = int(s.queries), pd = int(s.pd), pk = int(s.pk);
    const int keys4 = int(s.keys4), kpad = int(s.kpad);
    const size_t group = c->heads / c->kv_heads, stride = c->heads * c->head_dim;
    const float scale = 1.0f / sqrtf(float(hd));
    // Scratch::quantize (attention.rs:100-137) for every (image, key head): the keys' mean over
    // the keys in order, the keys less their mean and the values transposed as Q7b32 matrices
    const dim3 tiles(unsigned((keys + 63) / 64), unsigned((hd + 63) / 64), unsigned(s.ktables));
    key_transpose_kernel<<<tiles, 256, 0, st>>>(c->key, c->key_stride, c->key_offset, int(c->kv_heads), keys, hd, kpad,
                                                w.at<float>(Scratch::KEYT));
    key_mean_kernel<<<unsigned(s.ktables * s.hd), 64, size_t((kpad + 4095) / 4096 * 4096) * 4, st>>>(
        w.at<float>(Scratch::KEYT), keys, kpad, w.at<float>(Scratch::MEAN));
    const size_t kgroups = s.ktables * s.kquads * 4 * (s.pd / 32), vthreads = s.ktables * s.vquads * 4 * (s.pk / 32);
    key_table_kernel<<<blocks_for(8 * kgroups), kThreads, 0, st>>>(
        c->key, c->key_stride, c->key_offset, int(c->kv_heads), keys, hd, int(s.kquads * 4), pd / 32,
        w.at<float>(Scratch::MEAN), w.at<int8_t>(Scratch::KCODES), w.at<float>(Scratch::KSCALES), unsigned(kgroups));
    value_table_kernel<<<blocks_for(vthreads), kThreads, 0, st>>>(
        c->value, c->value_stride, c->value_offset, int(c->kv_heads), keys, hd, int(s.vquads * 4), pk / 32,
        w.at<int8_t>(Scratch::VCODES), w.at<float>(Scratch::VSCALES), unsigned(vthreads));
    const size_t slots = s.qtables * s.queries * (s.pd / 4);
    query_levels_kernel<<<blocks_for(slots), kThreads, 0, st>>>(
        c->query, c->query_stride, c->query_offset, int(c->heads), queries, hd, pd, unsigned(slots),
        w.at<int8_t>(Scratch::QLEVELS), w.at<float>(Scratch::QSCALES), w.at<int32_t>(Scratch::QCORR),
        s.queries % 128 == 0 ? w.at<float>(Scratch::QTSCALES) : nullptr);
    FG_HIP(hipGetLastError());
    int rc;
    // Scratch::unit (attention.rs:157-214) for every query of an (image, head) unit at once: unit
    // u = image · heads + h reads key head table t = u / group. Per unit the scores' product and
    // the exponentials (into the unit's slice of the batch's levels); per batch of units the
    // weighted values' products in one launch.
    const size_t batch = units_per_batch(s), elev = s.queries * s.pk, escl = s.queries * (s.pk / 32);
    const size_t kcode = s.kquads * (s.pd / 32) * 128, kscl = s.kquads * (s.pd / 32) * 4;
    const size_t vcode = s.vquads * (s.pk / 32) * 128, vscl = s.vquads * (s.pk / 32) * 4;
    for (size_t u0 = 0; u0 < s.qtables; u0 += batch) {
        const size_t u1 = std::min(s.qtables, u0 + batch);
        for (size_t u = u0; u < u1; u++) {
            const size_t t = u / group;
            fg_table ktab = runtime_matrix(w.at<int8_t>(Scratch::KCODES) + t * kcode, w.at<float>(Scratch::KSCALES) + t * kscl,
                                           s.keys, s.pd);
            ProductArgs a{};
            a.t = &ktab;
            a.q = w.at<int8_t>(Scratch::QLEVELS) + u * s.queries * s.pd;
            a.as = w.at<float>(Scratch::QSCALES) + u * s.queries * (s.pd / 32);
            a.corr = w.at<int32_t>(Scratch::QCORR) + u * s.queries * (s.pd / 32);
            if (s.queries % 128 == 0) {
                a.as_t = w.at<float>(Scratch::QTSCALES) + u * s.queries * (s.pd / 32);
                a.as_t_rows = s.queries;
            }
            a.rows = s.queries;
            a.quad_begin = 0;
            a.quad_end = size_t(keys4 / 4);
            a.out = w.at<float>(Scratch::PROD);
            a.ld_out = size_t(keys4);
            if ((rc = launch_product(a, st))) return rc;
            float *sums = w.at<float>(Scratch::SUMS) + u * s.queries;
            int8_t *lev = w.at<int8_t>(Scratch::ELEVELS) + (u - u0) * elev;
            float *lsc = w.at<float>(Scratch::ESCALES) + (u - u0) * escl;
            int32_t *lco = w.at<int32_t>(Scratch::ECORR) + (u - u0) * escl;
            rc = c->exponentials == FG_EXP_FAST
                     ? launch_exponentials<true>(w.at<float>(Scratch::PROD), keys4, scale, keys, pk, lev, lsc, lco, sums,
                                                 unsigned(queries), st)
                     : launch_exponentials<false>(w.at<float>(Scratch::PROD), keys4, scale, keys, pk, lev, lsc, lco, sums,
                                                  unsigned(queries), st);
            if (rc) return rc;
        }
        // the weighted values of every unit of the batch: unit u's levels times value table u / group
        const size_t t0 = u0 / group;
        fg_table vtab = runtime_matrix(w.at<int8_t>(Scratch::VCODES) + t0 * vcode, w.at<float>(Scratch::VSCALES) + t0 * vscl,
                                       s.hd, s.pk);
        ProductArgs b{};
        b.t = &vtab;
        b.q = w.at<int8_t>(Scratch::ELEVELS);
        b.as = w.at<float>(Scratch::ESCALES);
        b.corr = w.at<int32_t>(Scratch::ECORR);
        b.rows = s.queries;
        b.quad_begin = 0;
        b.quad_end = size_t(hd / 4);
        b.out = w.at<float>(Scratch::PV) + u0 * s.queries * s.hd;
        b.ld_out = s.hd;
        if ((rc = launch_gemm_batch(b, int(u1 - u0), int(group), int(u0 % group), elev, escl, s.queries * s.hd, vcode, vscl, st)))
            return rc;
    }
    // each output divided by its row's sum, every head at once
    const size_t n = s.qtables * s.queries * s.hd;
    divide_kernel<<<blocks_for(n), kThreads, 0, st>>>(w.at<float>(Scratch::PV), w.at<float>(Scratch::SUMS), int(c->heads),
                                                      queries, hd, unsigned(n), out, stride);
    FG_HIP(hipGetLastError());
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
    if (c->head_dim % 4 || c->head_dim > size_t(kMaxHeadDim))
        return set_error(FG_ERR_SHAPE, "fg_attend: head_dim must be whole quads, at most 1024");
    if (c->exponentials != FG_EXP_EXACT && c->exponentials != FG_EXP_FAST)
        return set_error(FG_ERR_ARG, "fg_attend: exponentials must be FG_EXP_EXACT or FG_EXP_FAST");
    if (pad32(c->keys) * 4 > size_t(kMaxRowBytes)) return set_error(FG_ERR_SHAPE, "fg_attend: at most 16384 keys");
    // the keys' transpose takes one grid layer per (image, key head); the row kernels a workgroup
    // per query row
    if (c->images * c->kv_heads > 65535 || c->queries > 0x7fffffff)
        return set_error(FG_ERR_SHAPE, "fg_attend: at most 65535 images x key heads and 2^31 - 1 queries");
    // every head of a row lies within the row's stride
    if (c->query_offset + c->heads * c->head_dim > c->query_stride ||
        c->key_offset + c->kv_heads * c->head_dim > c->key_stride ||
        c->value_offset + c->kv_heads * c->head_dim > c->value_stride)
        return set_error(FG_ERR_SHAPE, "fg_attend: an operand's heads run past its row stride");
    const Shape s(c);
    // the preparation and division kernels index their lanes in 32 bits
    const size_t lanes = std::max({8 * s.ktables * s.kquads * 4 * (s.pd / 32), s.ktables * s.vquads * 4 * (s.pk / 32),
                                   s.qtables * s.queries * (s.pd / 4), s.qtables * s.queries * s.hd});
    if (lanes >= (size_t(1) << 31)) return set_error(FG_ERR_SHAPE, "fg_attend: at most 2^31 - 1 values of queries, keys or outputs");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    Scratch w(s);
    void *ws = nullptr;
    FG_HIP(workspace_alloc(&ws, w.total(), st));
    w.carve(ws);
    int rc = run(c, out, st, s, w);
    // the scratch goes back to the pool in stream order, after the call's last kernel
    const hipError_t e = hipFreeAsync(ws, st);
    if (rc == FG_OK && e != hipSuccess) rc = check_hip(e, "hipFreeAsync");
    return rc;
}
