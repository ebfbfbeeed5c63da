// The extern "C" entry points of include/fusor_gpu.h: argument checks with the reference's
// messages, table ownership, and dispatch to the kernels. No CPU compute path exists: a call the
// GPU kernels do not cover returns an error.
#include <algorithm>
#include <cstdio>
#include <mutex>
#include <string>

#include "common.h"

namespace fg {

// fg_matmul_noalloc's scratch: one array per device, held from the library's load until the
// process ends (each GPU the library runs on keeps its own copy at its own address). Host code
// never uses the array's name as an address: its device address comes from hipGetSymbolAddress,
// once per device, with that device current.
constexpr size_t kNoAllocScratch = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratch];

// The device address of this device's scratch array (looked up on the device's first call).
static int scratch_address(void **out)
{
    static std::mutex mu;
    static void *address[64] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return check_hip(e, "fg_matmul_noalloc: hipGetDevice");
    if (dev < 0 || dev >= 64) return set_error(FG_ERR_ARG, "fg_matmul_noalloc: device index past 63");
    std::lock_guard<std::mutex> lock(mu);
    if (!address[dev]) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return check_hip(e, "fg_matmul_noalloc: hipGetSymbolAddress");
        if (!ptr) return set_error(FG_ERR_HIP, "fg_matmul_noalloc: no device address for the scratch array");
        address[dev] = ptr;
    }
    *out = address[dev];
    return FG_OK;
}

static thread_local std::string g_last_error;

int set_error(int code, const std::string &message)
{
    g_last_error = message;
    return code;
}

int check_hip(hipError_t e, const char *what)
{
    g_last_error = std::string(what) + ": " + hipGetErrorString(e);
    return e == hipErrorOutOfMemory ? FG_ERR_NOMEM : FG_ERR_HIP;
}

static const char *dtype_name(int dtype)
{
    switch (dtype) {
    case FG_F32: return "F32";
    case FG_Q7B32: return "Q7b32";
    case FG_Q4B32: return "Q4b32";
    case FG_T2B128: return "T2b128";
    case FG_Q8B32: return "Q8b32";
    default: return "unknown";
    }
}

// check_quantized (tensor.rs:162-171)
static int check_matrix(int dtype, size_t rows, size_t cols)
{
    if (!is_quantized(dtype)) return set_error(FG_ERR_FORMAT, std::string("a ") + dtype_name(dtype) + " table: a quantized format expected");
    const size_t group = size_t(group_of(dtype));
    if (cols % group != 0)
        return set_error(FG_ERR_FORMAT, std::string("a ") + dtype_name(dtype) + " tensor of shape [" + std::to_string(rows) + ", " +
                                            std::to_string(cols) + "]: a matrix of whole groups of " + std::to_string(group) +
                                            " expected");
    if (rows > (size_t(1) << 31) || cols > (size_t(1) << 20)) return set_error(FG_ERR_SHAPE, "table too large");
    return FG_OK;
}

static size_t byte_len(int dtype, size_t rows, size_t cols)
{
    const size_t padded = padded_values(rows, cols);
    return padded / size_t(codes_per_byte(dtype)) + padded / size_t(group_of(dtype)) * 4;
}

size_t table_byte_len(int dtype, size_t rows, size_t cols) { return byte_len(dtype, rows, cols); }

int table_alloc(int dtype, size_t rows, size_t cols, fg_table **out)
{
    *out = nullptr;
    int rc = check_matrix(dtype, rows, cols);
    if (rc) return rc;
    fg_table *t = new fg_table();
    t->dtype = dtype;
    t->rows = rows;
    t->cols = cols;
    t->quads = (rows + 3) / 4;
    t->blocks = cols / 32;
    t->groups = cols / size_t(group_of(dtype));
    t->code_bytes = t->quads * t->blocks * quad_bytes(dtype);
    t->codes = nullptr;
    t->scales = nullptr;
    const size_t scale_bytes = t->quads * t->groups * 4 * 4;
    hipError_t e = hipMalloc(reinterpret_cast<void **>(&t->codes), std::max<size_t>(t->code_bytes, 16));
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void **>(&t->scales), std::max<size_t>(scale_bytes, 16));
    if (e != hipSuccess) {
        if (t->codes) (void)hipFree(t->codes);
        delete t;
        return check_hip(e, "table storage: hipMalloc");
    }
    *out = t;
    return FG_OK;
}

static int create(const void *bytes, size_t len, int dtype, size_t rows, size_t cols, void *stream, bool device,
                  fg_table **out)
{
    if (!out) return set_error(FG_ERR_ARG, "fg_table_create: a null output handle");
    *out = nullptr;
    int rc = check_matrix(dtype, rows, cols);
    if (rc) return rc;
    const size_t want = byte_len(dtype, rows, cols);
    if (len != want)
        return set_error(FG_ERR_SHAPE, std::to_string(len) + " bytes for a " + dtype_name(dtype) + " table of shape [" +
                                           std::to_string(rows) + ", " + std::to_string(cols) + "] (" + std::to_string(want) +
                                           " expected)");
    if (!bytes && len) return set_error(FG_ERR_ARG, "fg_table_create: null bytes");
    hipStream_t s = as_stream(stream);
    fg_table *t = nullptr;
    if ((rc = table_alloc(dtype, rows, cols, &t))) return rc;
    uint8_t *staging = nullptr;
    const size_t scale_bytes = t->quads * t->groups * 4 * 4;
    hipError_t e = hipSuccess;
    const uint8_t *ref_codes = static_cast<const uint8_t *>(bytes);
    if (!device && t->code_bytes) {
        e = hipMalloc(reinterpret_cast<void **>(&staging), t->code_bytes);
        if (e == hipSuccess) e = hipMemcpyAsync(staging, bytes, t->code_bytes, hipMemcpyHostToDevice, s);
        ref_codes = staging;
    }
    if (e == hipSuccess && scale_bytes)
        e = hipMemcpyAsync(t->scales, static_cast<const uint8_t *>(bytes) + t->code_bytes, scale_bytes,
                           device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, s);
    if (e != hipSuccess) {
        rc = check_hip(e, "fg_table_create");
    } else {
        rc = launch_relayout(ref_codes, t, s);
        if (rc == FG_OK) {
            e = hipStreamSynchronize(s);
            if (e != hipSuccess) rc = check_hip(e, "fg_table_create: upload");
        }
    }
    if (staging) (void)hipFree(staging);
    if (rc) {
        (void)hipFree(t->codes);
        (void)hipFree(t->scales);
        delete t;
        return rc;
    }
    *out = t;
    return FG_OK;
}

static int check_product(const fg_table *t, const fg_input *in, size_t rows, size_t col_begin, size_t col_end, const char *who)
{
    if (!t || !in) return set_error(FG_ERR_ARG, std::string(who) + ": a null table or input");
    if ((in->x == nullptr) == (in->quants == nullptr))
        return set_error(FG_ERR_ARG, std::string(who) + ": exactly one of x and quants is set");
    if (in->quants && (!in->scales || !in->corrections))
        return set_error(FG_ERR_ARG, std::string(who) + ": quantized rows need their scales and corrections");
    // matmul.rs:271-274
    if (col_begin % 4 || col_end % 4 || col_end < col_begin) return set_error(FG_ERR_SHAPE, "columns in whole quads");
    // matmul.rs:531-535
    if (col_end > t->quads * 4) return set_error(FG_ERR_SHAPE, "weights cover the columns");
    if (in->x && (reinterpret_cast<uintptr_t>(in->x) & 15)) return set_error(FG_ERR_ARG, std::string(who) + ": x must be 16-byte aligned");
    if (in->quants && (reinterpret_cast<uintptr_t>(in->quants) & 15))
        return set_error(FG_ERR_ARG, std::string(who) + ": quants must be 16-byte aligned");
    if (rows > (size_t(1) << 24)) return set_error(FG_ERR_SHAPE, "too many rows");
    return FG_OK;
}

static ProductArgs product_args(const fg_table *t, const fg_input *in, size_t rows, size_t col_begin, size_t col_end)
{
    ProductArgs a{};
    a.t = t;
    a.x = in->x;
    a.q = in->quants;
    a.as = in->scales;
    a.corr = in->corrections;
    a.rows = rows;
    a.quad_begin = col_begin / 4;
    a.quad_end = col_end / 4;
    return a;
}

}  // namespace fg

using namespace fg;

extern "C" {

const char *fg_last_error(void) { return g_last_error.c_str(); }

int fg_version(void) { return 1; }

int fg_table_create(const void *bytes, size_t len, int dtype, size_t rows, size_t cols, void *stream, fg_table **out)
{
    return create(bytes, len, dtype, rows, cols, stream, false, out);
}

int fg_table_create_device(const void *bytes, size_t len, int dtype, size_t rows, size_t cols, void *stream, fg_table **out)
{
    return create(bytes, len, dtype, rows, cols, stream, true, out);
}

int fg_table_free(fg_table *t)
{
    if (!t) return FG_OK;
    (void)hipFree(t->codes);
    (void)hipFree(t->scales);
    delete t;
    return FG_OK;
}

int fg_table_shape(const fg_table *t, int *dtype, size_t *rows, size_t *cols)
{
    if (!t) return set_error(FG_ERR_ARG, "fg_table_shape: a null table");
    if (dtype) *dtype = t->dtype;
    if (rows) *rows = t->rows;
    if (cols) *cols = t->cols;
    return FG_OK;
}

size_t fg_table_byte_len(int dtype, size_t rows, size_t cols)
{
    if (!is_quantized(dtype)) return rows * cols * 4;
    return byte_len(dtype, rows, cols);
}

int fg_table_read(const fg_table *t, void *bytes, void *stream)
{
    if (!t || !bytes) return set_error(FG_ERR_ARG, "fg_table_read: a null argument");
    hipStream_t s = as_stream(stream);
    int rc = launch_unrelayout(t, static_cast<uint8_t *>(bytes), s);
    if (rc) return rc;
    FG_HIP(hipMemcpyAsync(static_cast<uint8_t *>(bytes) + t->code_bytes, t->scales, t->quads * t->groups * 16,
                          hipMemcpyDeviceToDevice, s));
    return FG_OK;
}

int fg_encode(int dtype, size_t rows, size_t cols, const float *values, void *bytes, void *stream)
{
    int rc = check_matrix(dtype, rows, cols);
    if (rc) return rc;
    if ((!values && rows * cols) || !bytes) return set_error(FG_ERR_ARG, "fg_encode: a null argument");
    return launch_encode(dtype, rows, cols, values, static_cast<uint8_t *>(bytes), as_stream(stream));
}

int fg_dequantize_row(const fg_table *t, size_t row, float *out, void *stream)
{
    if (!t || !out) return set_error(FG_ERR_ARG, "fg_dequantize_row: a null argument");
    if (row >= t->rows) return set_error(FG_ERR_SHAPE, "row " + std::to_string(row) + " of a table of " + std::to_string(t->rows));
    return launch_dequantize_row(t, row, out, as_stream(stream));
}

int fg_quantize_rows(const float *x, size_t count, int dtype, int8_t *quants, float *scales, int32_t *corrections, void *stream)
{
    if (!is_quantized(dtype)) return set_error(FG_ERR_FORMAT, "quantize_rows: a quantized weight format expected");
    // QuantizedRows::input (matmul.rs:150-160): whole groups
    if (count % size_t(group_of(dtype))) return set_error(FG_ERR_SHAPE, "the input is whole groups of the weights' format");
    if (count == 0) return FG_OK;
    if (!x || !quants || !scales || !corrections) return set_error(FG_ERR_ARG, "fg_quantize_rows: a null argument");
    if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(quants) & 3))
        return set_error(FG_ERR_ARG, "fg_quantize_rows: x must be 16-byte and quants 4-byte aligned");
    return launch_quantize_rows(x, count, dtype, quants, scales, corrections, as_stream(stream));
}

int fg_matmul(const fg_table *t, const fg_input *in, size_t rows, size_t col_begin, size_t col_end, const float *bias, float *out,
              size_t ld_out, int flags, void *stream)
{
    int rc = check_product(t, in, rows, col_begin, col_end, "fg_matmul");
    if (rc) return rc;
    if (!out && rows && col_end > col_begin) return set_error(FG_ERR_ARG, "fg_matmul: a null output");
    if (ld_out < col_end - col_begin) return set_error(FG_ERR_SHAPE, "fg_matmul: ld_out shorter than the columns");
    ProductArgs a = product_args(t, in, rows, col_begin, col_end);
    a.bias = bias;
    a.out = out;
    a.ld_out = ld_out;
    a.accumulate = (flags & FG_ACCUMULATE) != 0;
    a.fused = (flags & FG_FUSED_SCALE) != 0;
    a.parallel = (flags & FG_PARALLEL_SUM) != 0;
    if (flags & ~(FG_ACCUMULATE | FG_FUSED_SCALE | FG_PARALLEL_SUM)) return set_error(FG_ERR_ARG, "fg_matmul: unknown flags");
    if (a.parallel) {
        if (a.fused) return set_error(FG_ERR_ARG, "fg_matmul: FG_PARALLEL_SUM and FG_FUSED_SCALE exclude each other");
        if (t->dtype == FG_T2B128) return set_error(FG_ERR_FORMAT, "fg_matmul: FG_PARALLEL_SUM takes Q7b32, Q8b32 and Q4b32 tables");
        if (rows > 1) return set_error(FG_ERR_SHAPE, "fg_matmul: FG_PARALLEL_SUM takes one row");
    }
    return launch_product(a, as_stream(stream));
}

int fg_matmul_noalloc(const fg_table *t, const fg_input *in, size_t rows, size_t col_begin, size_t col_end, const float *bias,
                      float *out, size_t ld_out, int flags, void *stream)
{
    int rc = check_product(t, in, rows, col_begin, col_end, "fg_matmul_noalloc");
    if (rc) return rc;
    if (!out && rows && col_end > col_begin) return set_error(FG_ERR_ARG, "fg_matmul_noalloc: a null output");
    if (ld_out < col_end - col_begin) return set_error(FG_ERR_SHAPE, "fg_matmul_noalloc: ld_out shorter than the columns");
    if (flags & ~(FG_ACCUMULATE | FG_FUSED_SCALE)) return set_error(FG_ERR_ARG, "fg_matmul_noalloc: unknown flags");
    ProductArgs a = product_args(t, in, rows, col_begin, col_end);
    a.bias = bias;
    a.out = out;
    a.ld_out = ld_out;
    a.accumulate = (flags & FG_ACCUMULATE) != 0;
    a.fused = (flags & FG_FUSED_SCALE) != 0;
    const size_t need = product_scratch_bytes(a);
    if (need > kNoAllocScratch)
        return set_error(FG_ERR_SHAPE, "fg_matmul_noalloc: this product needs " + std::to_string(need) +
                                           " bytes of scratch, more than the " + std::to_string(kNoAllocScratch) +
                                           " the library holds (use fg_matmul)");
    if (need) {
        if ((rc = scratch_address(&a.workspace))) return rc;
        a.workspace_bytes = kNoAllocScratch;
    }
    return launch_product(a, as_stream(stream));
}

int fg_qmatrix_create(size_t capacity, size_t cols, fg_table **out)
{
    if (!out) return set_error(FG_ERR_ARG, "fg_qmatrix_create: a null output handle");
    *out = nullptr;
    // QuantizedMatrix::reset (matmul.rs:47-53)
    if (cols % 32) return set_error(FG_ERR_SHAPE, "rows of whole blocks");
    if (capacity > (size_t(1) << 31) || cols > (size_t(1) << 20)) return set_error(FG_ERR_SHAPE, "matrix too large");
    fg_table *t = new fg_table();
    t->dtype = FG_Q7B32;
    t->capacity = capacity;
    t->max_cols = cols;
    t->rows = 0;
    t->cols = cols;
    t->quads = 0;
    t->blocks = t->groups = cols / 32;
    t->code_bytes = 0;
    const size_t quads = (capacity + 3) / 4;
    hipError_t e = hipMalloc(reinterpret_cast<void **>(&t->codes), std::max<size_t>(quads * t->blocks * 128, 16));
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void **>(&t->scales), std::max<size_t>(quads * t->blocks * 16, 16));
    if (e != hipSuccess) {
        (void)hipFree(t->codes);
        delete t;
        return check_hip(e, "fg_qmatrix_create");
    }
    *out = t;
    return FG_OK;
}

static int check_qmatrix(const fg_table *t, const char *who)
{
    if (!t) return set_error(FG_ERR_ARG, std::string(who) + ": a null matrix");
    if (!t->capacity) return set_error(FG_ERR_FORMAT, std::string(who) + ": a model table, not a run-time matrix");
    return FG_OK;
}

int fg_qmatrix_reset(fg_table *t, size_t cols)
{
    int rc = check_qmatrix(t, "fg_qmatrix_reset");
    if (rc) return rc;
    if (cols % 32) return set_error(FG_ERR_SHAPE, "rows of whole blocks");  // matmul.rs:48
    if (cols > t->max_cols) return set_error(FG_ERR_SHAPE, "fg_qmatrix_reset: wider than the matrix was created for");
    t->rows = 0;
    t->cols = cols;
    t->quads = 0;
    t->blocks = t->groups = cols / 32;
    t->code_bytes = 0;
    return FG_OK;
}

int fg_qmatrix_extend(fg_table *t, size_t rows, void *stream)
{
    int rc = check_qmatrix(t, "fg_qmatrix_extend");
    if (rc) return rc;
    hipStream_t s = as_stream(stream);
    if (rows > (size_t(1) << 31) - t->rows) return set_error(FG_ERR_SHAPE, "matrix too large");
    if (rows > t->capacity - t->rows) {
        // Grow like the reference's Vec: the rows so far are a prefix of the layout (quad-major),
        // so they move with one copy. The old storage is freed once the stream has drained.
        const size_t capacity = std::max(t->capacity * 2, t->rows + rows);
        const size_t quads = (capacity + 3) / 4, used = (t->rows + 3) / 4, blocks = t->max_cols / 32;
        int8_t *codes = nullptr;
        float *scales = nullptr;
        hipError_t e = hipMalloc(reinterpret_cast<void **>(&codes), quads * blocks * 128);
        if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void **>(&scales), quads * blocks * 16);
        if (e == hipSuccess) e = hipMemcpyAsync(codes, t->codes, used * t->blocks * 128, hipMemcpyDeviceToDevice, s);
        if (e == hipSuccess) e = hipMemcpyAsync(scales, t->scales, used * t->blocks * 16, hipMemcpyDeviceToDevice, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) {
            (void)hipFree(codes);
            (void)hipFree(scales);
            return check_hip(e, "fg_qmatrix_extend");
        }
        (void)hipFree(t->codes);
        (void)hipFree(t->scales);
        t->codes = codes;
        t->scales = scales;
        t->capacity = capacity;
    }
    const size_t first = t->rows, last = (t->rows + rows + 3) / 4 * 4;
    rc = launch_qmatrix_clear(t, first, last, s);
    if (rc) return rc;
    t->rows += rows;
    t->quads = (t->rows + 3) / 4;
    t->code_bytes = t->quads * t->blocks * 128;
    return FG_OK;
}

int fg_qmatrix_set_rows(fg_table *t, size_t row, size_t count, const float *values, void *stream)
{
    int rc = check_qmatrix(t, "fg_qmatrix_set_rows");
    if (rc) return rc;
    if (row > t->rows || count > t->rows - row) return set_error(FG_ERR_SHAPE, "fg_qmatrix_set_rows: rows past the matrix");
    if (!values && count) return set_error(FG_ERR_ARG, "fg_qmatrix_set_rows: null values");
    if (reinterpret_cast<uintptr_t>(values) & 15) return set_error(FG_ERR_ARG, "fg_qmatrix_set_rows: values must be 16-byte aligned");
    return launch_qmatrix_set(t, row, count, 0, t->blocks, values, t->cols, as_stream(stream));
}

int fg_qmatrix_set_block(fg_table *t, size_t row, size_t block, const float *values, void *stream)
{
    int rc = check_qmatrix(t, "fg_qmatrix_set_block");
    if (rc) return rc;
    if (row >= t->rows || block >= t->blocks) return set_error(FG_ERR_SHAPE, "fg_qmatrix_set_block: a block past the matrix");
    if (!values) return set_error(FG_ERR_ARG, "fg_qmatrix_set_block: null values");
    if (reinterpret_cast<uintptr_t>(values) & 15) return set_error(FG_ERR_ARG, "fg_qmatrix_set_block: values must be 16-byte aligned");
    return launch_qmatrix_set(t, row, 1, block, 1, values, 32, as_stream(stream));
}

int fg_matmul_dots(const fg_table *t, const fg_input *in, size_t rows, size_t col_begin, size_t col_end, int32_t *dots, void *stream)
{
    int rc = check_product(t, in, rows, col_begin, col_end, "fg_matmul_dots");
    if (rc) return rc;
    if (!dots && rows && col_end > col_begin) return set_error(FG_ERR_ARG, "fg_matmul_dots: a null output");
    ProductArgs a = product_args(t, in, rows, col_begin, col_end);
    a.dots = dots;
    return launch_product(a, as_stream(stream));
}

}  // extern "C"
