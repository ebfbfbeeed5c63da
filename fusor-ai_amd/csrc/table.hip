// Tables on the device: the reference byte layout in and out (tensor.rs:1-9, quant.rs:89-118),
// Tensor::encode (tensor.rs:97-143, quant.rs:143-177), Matrix::dequantize_row (tensor.rs:247-271)
// and the activation quantizer quantize_rows (matmul.rs:233-257, arch/scalar.rs:48-66).
#include "common.h"

namespace fg {
namespace {

// Where code `input` of row `lane` sits in a reference quad block, and its shift
// (quant.rs:89-95).
__device__ __forceinline__ void code_position(int cpb, int lane, int input, int &byte, int &shift)
{
    int chunk = input >> 2, offset = input & 3;
    int words = 8 / cpb, bits = 8 / cpb;
    byte = (chunk % words) * 16 + lane * 4 + offset;
    shift = bits * (chunk / words);
}

// Reference quad blocks to device quad blocks (and back with `inverse`). In every format the
// code of lane L, input k sits in the reference at byte (c % W)·16 + 4L + k % 4 (c = k / 4, W = 8 /
// codes per byte), and the device's packing puts the codes sharing a reference byte into the same
// device byte: device dword j of lane L is reference dword (j·16 + 4L) / 4 of the quad block, a
// transpose of dwords (quant.rs:89-97). Q7b32 also moves the codes to signed levels, u - 64, byte
// by byte (wrapping, so that any byte round-trips). One thread per device dword, coalesced.
__global__ void relayout_kernel(const uint32_t *__restrict__ src, uint32_t *__restrict__ dst, int dtype, size_t dwords,
                                int inverse)
{
    const size_t id = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= dwords) return;
    const int per_lane = dtype == FG_Q4B32 ? 4 : dtype == FG_T2B128 ? 2 : 8;  // device dwords per lane row
    const size_t quad_block = id / (4 * per_lane);
    const int r = int(id % (4 * per_lane)), lane = r / per_lane, j = r % per_lane;
    const size_t dev = id, ref = quad_block * (4 * per_lane) + size_t(j) * 4 + lane;
    constexpr uint32_t H = 0x80808080u;
    if (!inverse) {
        uint32_t x = src[ref];
        if (dtype == FG_Q7B32) x = ((x | H) - 0x40404040u) ^ ((x ^ 0xBFBFBFBFu) & H);  // bytes u - 64
        dst[dev] = x;
    } else {
        uint32_t x = src[dev];
        if (dtype == FG_Q7B32) x = ((x & 0x7F7F7F7Fu) + 0x40404040u) ^ (x & H);  // bytes level + 64
        dst[ref] = x;
    }
}

// Rust's saturating float casts (NaN to 0).
__device__ __forceinline__ int sat_i8(float v) { return v != v ? 0 : v >= 127.0f ? 127 : v <= -128.0f ? -128 : int(v); }
__device__ __forceinline__ int sat_u8(float v) { return v != v ? 0 : v >= 255.0f ? 255 : v <= 0.0f ? 0 : int(v); }
__device__ __forceinline__ int sat_i32(float v)
{
    return v != v ? 0 : v >= 2147483648.0f ? 2147483647 : v <= -2147483648.0f ? int(0x80000000u) : int(v);
}
// f32::clamp keeps NaN.
__device__ __forceinline__ float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

// One group of a row to codes; returns its scale (quant.rs:143-177, Q8b32 extension).
__device__ float quantize_group(int dtype, const float *x, int n, uint8_t *codes)
{
    if (dtype == FG_Q4B32) {
        float extreme = 0.0f;
        for (int i = 0; i < n; i++)
            if (fabsf(x[i]) > fabsf(extreme)) extreme = x[i];
        float scale = group_scale(extreme, -8.0f);
        for (int i = 0; i < n; i++) codes[i] = uint8_t(sat_u8(clampf(__builtin_rintf(x[i] / scale) + 8.0f, 0.0f, 15.0f)));
        return scale;
    }
    float amax = 0.0f;
    for (int i = 0; i < n; i++) amax = fmaxf(amax, fabsf(x[i]));
    if (dtype == FG_T2B128) {
        float scale = group_scale(amax, 1.0f);
        for (int i = 0; i < n; i++) codes[i] = uint8_t(sat_i32(clampf(__builtin_rintf(x[i] / scale), -1.0f, 1.0f)) + 1);
        return scale;
    }
    float level_max = dtype == FG_Q7B32 ? 63.0f : 127.0f;
    float scale = group_scale(amax, level_max);
    for (int i = 0; i < n; i++) {
        int level = sat_i8(__builtin_rintf(x[i] / scale));
        if (dtype == FG_Q7B32) {
            level = level < -63 ? -63 : (level > 63 ? 63 : level);
            codes[i] = uint8_t(level + 64);
        } else {
            level = level < -127 ? -127 : level;
            codes[i] = uint8_t(int8_t(level));
        }
    }
    return scale;
}

// Tensor::encode: one thread per (quad, group) writes the group's blocks of all four rows and
// their scales, padding rows as zero codes and zero scales (tensor.rs:83-88,124-143).
__global__ void encode_kernel(int dtype, size_t rows, size_t cols, const float *__restrict__ values,
                              uint8_t *__restrict__ bytes, size_t quant_len, size_t quads)
{
    int group = dtype == FG_T2B128 ? 128 : 32;
    size_t groups = cols / group, blocks = cols / 32;
    size_t id = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= quads * groups) return;
    size_t quad = id / groups, g = id % groups;
    int cpb = dtype == FG_Q4B32 ? 2 : dtype == FG_T2B128 ? 4 : 1;
    int qbytes = 128 / cpb;
    float *scales = reinterpret_cast<float *>(bytes + quant_len);
    int bpg = group / 32;
    uint8_t quadblock[4][128];
    for (int b = 0; b < bpg; b++)
        for (int i = 0; i < qbytes; i++) quadblock[b][i] = 0;
    for (int lane = 0; lane < 4; lane++) {
        size_t row = quad * 4 + lane;
        uint8_t codes[128];
        float scale = 0.0f;
        if (row < rows) {
            scale = quantize_group(dtype, values + row * cols + g * group, group, codes);
        } else {
            for (int i = 0; i < group; i++) codes[i] = 0;
        }
        scales[(quad * groups + g) * 4 + lane] = scale;
        for (int b = 0; b < bpg; b++) {
            for (int k = 0; k < 32; k++) {
                int byte, shift;
                code_position(cpb, lane, k, byte, shift);
                quadblock[b][byte] |= uint8_t(codes[b * 32 + k] << shift);
            }
        }
    }
    for (int b = 0; b < bpg; b++) {
        uint8_t *out = bytes + (quad * blocks + g * bpg + b) * qbytes;
        for (int i = 0; i < qbytes; i++) out[i] = quadblock[b][i];
    }
}

// The signed level of code k of a device row-block.
__device__ __forceinline__ int device_level(int dtype, const int8_t *quadblock, int lane, int k)
{
    const uint8_t *u = reinterpret_cast<const uint8_t *>(quadblock);
    switch (dtype) {
    case FG_Q4B32: return int((u[lane * 16 + (k & 15)] >> (4 * (k >> 4))) & 15) - 8;
    case FG_T2B128: return int((u[lane * 8 + (k & 7)] >> (2 * (k >> 3))) & 3) - 1;
    default: return int(quadblock[lane * 32 + k]);
    }
}

// out[k] = scale · (float)level (quant.rs:80-85), one thread per value.
__global__ void dequantize_row_kernel(const int8_t *__restrict__ codes, const float *__restrict__ scales, int dtype,
                                      size_t row, size_t cols, float *__restrict__ out)
{
    size_t k = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (k >= cols) return;
    int group = dtype == FG_T2B128 ? 128 : 32;
    size_t blocks = cols / 32, groups = cols / group;
    size_t quad = row / 4;
    int lane = int(row % 4);
    size_t b = k / 32;
    int qbytes = dtype == FG_Q4B32 ? 64 : dtype == FG_T2B128 ? 32 : 128;
    int level = device_level(dtype, codes + (quad * blocks + b) * qbytes, lane, int(k % 32));
    float scale = scales[(quad * groups + b / (group / 32)) * 4 + lane];
    out[k] = scale * float(level);
}

// quantize_rows: `lanes` threads per group (8 for groups of 32, 32 for groups of 128), four
// values per thread. The group's absmax is a max over its values (order-free, NaN ignored as
// f32::max does); its scale amax/127 by IEEE division; every level rounds ties to even.
template <int LANES>
__global__ void quantize_rows_kernel(const float *__restrict__ x, size_t groups, int zp, int8_t *__restrict__ q,
                                     float *__restrict__ scales, int32_t *__restrict__ corr)
{
    size_t t = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    size_t g = t / LANES;
    int sub = int(t % LANES);
    bool active = g < groups;
    float4 v = active ? reinterpret_cast<const float4 *>(x)[g * LANES + sub] : make_float4(0, 0, 0, 0);
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = max8(fmaxf(0.0f, amax));
    for (int m = 8; m < LANES; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
    int l0, l1, l2, l3;
    const float d = scale_and_levels(amax, v.x, v.y, v.z, v.w, l0, l1, l2, l3);
    int sum = sum8(l0 + l1 + l2 + l3);
    for (int m = 8; m < LANES; m <<= 1) sum += __shfl_xor(sum, m, 64);
    if (!active) return;
    reinterpret_cast<int *>(q)[g * LANES + sub] = pack4(l0, l1, l2, l3);
    if (sub == 0) {
        scales[g] = d;
        corr[g] = -zp * sum;
    }
}

// QuantizedMatrix::extend (matmul.rs:66-72): rows [first, last) to the reference's zero codes
// (u = 0, stored as the level -64) and zero scales. One thread per (row, block).
__global__ void qmatrix_clear_kernel(int8_t *__restrict__ codes, float *__restrict__ scales, size_t first, size_t last,
                                     size_t blocks)
{
    const size_t id = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= (last - first) * blocks) return;
    const size_t row = first + id / blocks, b = id % blocks, quad = row / 4;
    const int lane = int(row % 4);
    int4 *dst = reinterpret_cast<int4 *>(codes + (quad * blocks + b) * 128 + lane * 32);
    const int v = int(0xC0C0C0C0u);
    dst[0] = make_int4(v, v, v, v);
    dst[1] = make_int4(v, v, v, v);
    scales[(quad * blocks + b) * 4 + lane] = 0.0f;
}

// QuantizedMatrix::set_block (matmul.rs:77-90) for blocks [b0, b0 + nb) of rows
// [first, first + count): the block's scale (absmax / 63, 1 for a zero block) and its Q7b32
// levels (round ties to even, clamped to ±63), stored signed. values[r * ld + j * 32 + k] is
// value k of block b0 + j of row first + r. One thread per (row, block).
__global__ void qmatrix_set_kernel(int8_t *__restrict__ codes, float *__restrict__ scales, size_t first, size_t count,
                                   size_t b0, size_t nb, size_t blocks, const float *__restrict__ values, size_t ld)
{
    const size_t id = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= count * nb) return;
    const size_t r = id / nb, j = id % nb;
    const size_t row = first + r, b = b0 + j, quad = row / 4;
    const int lane = int(row % 4);
    float x[32];
    const float4 *src = reinterpret_cast<const float4 *>(values + r * ld + j * 32);
    for (int i = 0; i < 8; i++) {
        const float4 f = src[i];
        x[4 * i] = f.x;
        x[4 * i + 1] = f.y;
        x[4 * i + 2] = f.z;
        x[4 * i + 3] = f.w;
    }
    scales[(quad * blocks + b) * 4 + lane] = q7_block(x, reinterpret_cast<int *>(codes + (quad * blocks + b) * 128 + lane * 32));
}

}  // namespace

int launch_qmatrix_clear(fg_table *t, size_t first, size_t last, hipStream_t s)
{
    const size_t n = (last - first) * t->blocks;
    if (n == 0) return FG_OK;
    qmatrix_clear_kernel<<<unsigned((n + 255) / 256), 256, 0, s>>>(t->codes, t->scales, first, last, t->blocks);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

int launch_qmatrix_set(fg_table *t, size_t first, size_t count, size_t b0, size_t nb, const float *values, size_t ld,
                       hipStream_t s)
{
    const size_t n = count * nb;
    if (n == 0) return FG_OK;
    qmatrix_set_kernel<<<unsigned((n + 127) / 128), 128, 0, s>>>(t->codes, t->scales, first, count, b0, nb, t->blocks,
                                                                values, ld);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

int launch_relayout(const uint8_t *ref_codes, fg_table *t, hipStream_t s)
{
    const size_t n = t->code_bytes / 4;
    if (n == 0) return FG_OK;
    relayout_kernel<<<unsigned((n + 255) / 256), 256, 0, s>>>(reinterpret_cast<const uint32_t *>(ref_codes),
                                                              reinterpret_cast<uint32_t *>(t->codes), t->dtype, n, 0);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

int launch_relayout_range(const uint8_t *ref_codes, uint8_t *dev_codes, int dtype, size_t bytes, hipStream_t s)
{
    // whole quad blocks: the transpose never leaves one, so any run of them relays on its own
    const size_t n = bytes / 4;
    if (n == 0) return FG_OK;
    relayout_kernel<<<unsigned((n + 255) / 256), 256, 0, s>>>(reinterpret_cast<const uint32_t *>(ref_codes),
                                                              reinterpret_cast<uint32_t *>(dev_codes), dtype, n, 0);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

int launch_unrelayout(const fg_table *t, uint8_t *ref_codes, hipStream_t s)
{
    const size_t n = t->code_bytes / 4;
    if (n == 0) return FG_OK;
    relayout_kernel<<<unsigned((n + 255) / 256), 256, 0, s>>>(reinterpret_cast<const uint32_t *>(t->codes),
                                                              reinterpret_cast<uint32_t *>(ref_codes), t->dtype, n, 1);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

int launch_encode(int dtype, size_t rows, size_t cols, const float *values, uint8_t *bytes, hipStream_t s)
{
    size_t quads = (rows + 3) / 4;
    size_t groups = cols / size_t(group_of(dtype));
    size_t quant_len = padded_values(rows, cols) / size_t(codes_per_byte(dtype));
    size_t n = quads * groups;
    if (n == 0) return FG_OK;
    encode_kernel<<<unsigned((n + 127) / 128), 128, 0, s>>>(dtype, rows, cols, values, bytes, quant_len, quads);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

// Lm::embed (lm.rs:97-108): row ids[y] of the table into out[y], one thread per value. An id past
// the table's rows (where the reference's slice index panics) reads nothing and gives a row of NaN.
__global__ void embed_rows_kernel(const int8_t *__restrict__ codes, const float *__restrict__ scales, int dtype,
                                  const int32_t *__restrict__ ids, size_t rows, size_t cols, float *__restrict__ out)
{
    const size_t k = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (k >= cols) return;
    const size_t row = size_t(uint32_t(ids[blockIdx.y]));
    if (row >= rows) {
        out[size_t(blockIdx.y) * cols + k] = __builtin_nanf("");
        return;
    }
    const int group = dtype == FG_T2B128 ? 128 : 32;
    const size_t blocks = cols / 32, groups = cols / group, quad = row / 4, b = k / 32;
    const int lane = int(row % 4);
    const int qbytes = dtype == FG_Q4B32 ? 64 : dtype == FG_T2B128 ? 32 : 128;
    const int level = device_level(dtype, codes + (quad * blocks + b) * qbytes, lane, int(k % 32));
    const float scale = scales[(quad * groups + b / (group / 32)) * 4 + lane];
    out[size_t(blockIdx.y) * cols + k] = scale * float(level);
}

int launch_embed_rows(const fg_table *t, const int32_t *ids, size_t count, float *out, hipStream_t s)
{
    if (t->cols == 0 || count == 0) return FG_OK;
    if (count > 65535) return set_error(FG_ERR_SHAPE, "at most 65535 rows per embedding call");
    embed_rows_kernel<<<dim3(unsigned((t->cols + 255) / 256), unsigned(count)), 256, 0, s>>>(t->codes, t->scales, t->dtype, ids,
                                                                                             t->rows, t->cols, out);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

int launch_dequantize_row(const fg_table *t, size_t row, float *out, hipStream_t s)
{
    if (t->cols == 0) return FG_OK;
    dequantize_row_kernel<<<unsigned((t->cols + 255) / 256), 256, 0, s>>>(t->codes, t->scales, t->dtype, row, t->cols, out);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

namespace {

// quantize_rows_kernel<8>'s arithmetic for groups of 32, the scale of group g of row r stored at
// as_t[g·Mpad + r]; the slots of rows M..Mpad-1 get zero scales. Teams of 8 lanes take the
// (row, group) pairs row first, so a wave's scale stores are one run of a group's column and each
// team reads its row's group as one 128-byte line. Each team takes kQuantPairs pairs, `slice`
// apart, their loads issued together (more bytes in flight per lane).
constexpr int kQuantPairs = 4;

__global__ void quantize_rows_t_kernel(const float *__restrict__ x, unsigned M, unsigned G, unsigned Mpad, unsigned slice,
                                       int8_t *__restrict__ q, float *__restrict__ as_t)
{
    const unsigned t = blockIdx.x * blockDim.x + threadIdx.x;  // 32-bit: the host keeps the lanes below 2^31
    const unsigned team0 = t / 8;
    if (team0 >= slice) return;  // the grid's last threads (a whole team at a time)
    const int sub = int(t % 8);
    float4 v[kQuantPairs];
    unsigned gi[kQuantPairs], r[kQuantPairs];
    bool active[kQuantPairs];
#pragma unroll
    for (int j = 0; j < kQuantPairs; j++) {
        const unsigned team = team0 + unsigned(j) * slice;
        gi[j] = team / Mpad;
        r[j] = team - gi[j] * Mpad;
        active[j] = r[j] < M && gi[j] < G;
        v[j] = active[j] ? reinterpret_cast<const float4 *>(x)[(size_t(r[j]) * G + gi[j]) * 8 + sub] : make_float4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < kQuantPairs; j++) {
        float amax = fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w)));
        amax = max8(fmaxf(0.0f, amax));
        int l0, l1, l2, l3;
        const float d = scale_and_levels(amax, v[j].x, v[j].y, v[j].z, v[j].w, l0, l1, l2, l3);
        if (active[j]) {
            reinterpret_cast<int *>(q)[(size_t(r[j]) * G + gi[j]) * 8 + sub] = pack4(l0, l1, l2, l3);
            if (sub == 0) as_t[size_t(gi[j]) * Mpad + r[j]] = d;
        } else if (gi[j] < G && sub == 0) {
            as_t[size_t(gi[j]) * Mpad + r[j]] = 0.0f;
        }
    }
}

}  // namespace

int launch_quantize_rows_t(const float *x, size_t rows, size_t K, int dtype, int8_t *q, float *as_t, size_t Mpad,
                           hipStream_t s)
{
    if (group_of(dtype) != 32) return set_error(FG_ERR_FORMAT, "block-major scales take groups of 32");
    const size_t G = K / 32, teams = Mpad * G, slice = (teams + kQuantPairs - 1) / kQuantPairs, threads = slice * 8;
    if (teams == 0) return FG_OK;
    if (teams * 8 >= (size_t(1) << 31) || rows > Mpad) return set_error(FG_ERR_SHAPE, "at most 2^31 - 1 quantization lanes in one launch");
    quantize_rows_t_kernel<<<unsigned((threads + 255) / 256), 256, 0, s>>>(x, unsigned(rows), unsigned(G), unsigned(Mpad),
                                                                            unsigned(slice), q, as_t);
    FG_HIP(hipGetLastError());
    return FG_OK;
}

int launch_quantize_rows(const float *x, size_t count, int dtype, int8_t *q, float *scales, int32_t *corr,
                         hipStream_t s)
{
    int group = group_of(dtype);
    size_t groups = count / size_t(group);
    if (groups == 0) return FG_OK;
    int zp = zero_point_of(dtype);
    if (group == 32) {
        size_t threads = groups * 8;
        quantize_rows_kernel<8><<<unsigned((threads + 255) / 256), 256, 0, s>>>(x, groups, zp, q, scales, corr);
    } else {
        size_t threads = groups * 32;
        quantize_rows_kernel<32><<<unsigned((threads + 255) / 256), 256, 0, s>>>(x, groups, zp, q, scales, corr);
    }
    FG_HIP(hipGetLastError());
    return FG_OK;
}

}  // namespace fg
