// A table's bytes streamed onto the device as a bundle store receives them.
//
// Reference: Store::write (bundle/src/store.rs:90-126) copies each arriving piece of a part into
// the zeroed tensor it belongs to (Tensor::bytes_mut), in order; Store::end_part (:129-146) checks
// that every byte came; Table::load (bundle/src/load.rs:72-84) then wraps the tensor in a Table
// (tensor.rs:200-211), whose device mirror fg_table_create builds from the whole byte array.
//
// Here the pieces go to the device as they arrive. They are gathered in two pinned host buffers
// of kStage bytes; a full buffer goes to the device with one copy on the upload's stream while
// the other buffer fills. A buffer's code bytes land in a device staging buffer and are relaid
// into the table's device layout at once (the quad-block transpose of relayout_kernel never
// leaves a quad block, so every run of whole quad blocks relays on its own): a buffer ends on a
// quad-block boundary and carries a partial quad block over to the next. Scale bytes keep their
// layout and go straight to the table's scales. By the last piece the table is all but done:
// fg_upload_end sends the last buffer and waits for the stream. No full-size host or device copy
// of the table is ever made.
#include <algorithm>
#include <cstring>
#include <string>

#include "common.h"

namespace fg {
namespace {

constexpr size_t kStage = size_t(8) << 20;  // bytes per pinned buffer (a multiple of every quad block)

}  // namespace
}  // namespace fg

struct fg_upload {
    fg_table *table;     // device storage, handed out by fg_upload_end
    size_t total;        // the table's byte length in the reference layout
    size_t received;     // bytes written so far (the offset the next write starts at)
    size_t sent;         // bytes handed to the device (the start of the filling buffer)
    size_t qb;           // bytes per quad block
    hipStream_t stream;
    uint8_t *host[2];    // pinned buffers
    uint8_t *dev[2];     // device staging for their code bytes
    hipEvent_t done[2];  // the last copy out of each buffer and the relayout of its codes
    int cur;             // the buffer filling
    size_t fill;         // bytes in it
};

namespace fg {
namespace {

void release(fg_upload *u)
{
    if (!u) return;
    for (int i = 0; i < 2; i++) {
        if (u->done[i]) (void)hipEventSynchronize(u->done[i]);
        if (u->done[i]) (void)hipEventDestroy(u->done[i]);
        if (u->host[i]) (void)hipHostFree(u->host[i]);
        if (u->dev[i]) (void)hipFree(u->dev[i]);
    }
    if (u->table) {
        (void)hipFree(u->table->codes);
        (void)hipFree(u->table->scales);
        delete u->table;
    }
    delete u;
}

// Sends the filling buffer's first `n` bytes (table bytes [sent, sent + n)) to the device, then
// moves what is left of it to the other buffer (after that buffer's last copy has finished).
int flush(fg_upload *u, size_t n)
{
    fg_table *t = u->table;
    const int b = u->cur;
    const size_t first = u->sent, last = first + n, code_end = t->code_bytes;
    if (first < code_end && n) {
        const size_t codes = std::min(last, code_end) - first;  // whole quad blocks
        FG_HIP(hipMemcpyAsync(u->dev[b], u->host[b], codes, hipMemcpyHostToDevice, u->stream));
        int rc = launch_relayout_range(u->dev[b], reinterpret_cast<uint8_t *>(t->codes) + first, t->dtype, codes, u->stream);
        if (rc) return rc;
    }
    if (last > code_end) {
        const size_t from = std::max(first, code_end);
        FG_HIP(hipMemcpyAsync(reinterpret_cast<uint8_t *>(t->scales) + (from - code_end), u->host[b] + (from - first),
                              last - from, hipMemcpyHostToDevice, u->stream));
    }
    FG_HIP(hipEventRecord(u->done[b], u->stream));
    const int o = 1 - b;
    FG_HIP(hipEventSynchronize(u->done[o]));  // the other buffer's copy (and relayout) is over
    const size_t rest = u->fill - n;
    if (rest) std::memcpy(u->host[o], u->host[b] + n, rest);
    u->sent = last;
    u->cur = o;
    u->fill = rest;
    return FG_OK;
}

// How much of a full buffer can go: up to a quad-block boundary while in the codes.
size_t sendable(const fg_upload *u)
{
    const size_t end = u->sent + u->fill, code_end = u->table->code_bytes;
    if (end >= code_end) return u->fill;  // the codes' tail is whole quad blocks, scales any length
    return end / u->qb * u->qb - u->sent;
}

}  // namespace
}  // namespace fg

using namespace fg;

extern "C" {

int fg_upload_begin(int dtype, size_t rows, size_t cols, void *stream, fg_upload **out)
{
    if (!out) return set_error(FG_ERR_ARG, "fg_upload_begin: a null output handle");
    *out = nullptr;
    fg_upload *u = new fg_upload();
    int rc = table_alloc(dtype, rows, cols, &u->table);
    if (rc) {
        delete u;
        return rc;
    }
    u->total = table_byte_len(dtype, rows, cols);
    u->qb = quad_bytes(dtype);
    u->stream = as_stream(stream);
    hipError_t e = hipSuccess;
    for (int i = 0; i < 2 && e == hipSuccess; i++) {
        e = hipHostMalloc(reinterpret_cast<void **>(&u->host[i]), kStage, hipHostMallocDefault);
        if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void **>(&u->dev[i]), kStage);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&u->done[i], hipEventDisableTiming);
    }
    if (e != hipSuccess) {
        rc = check_hip(e, "fg_upload_begin");
        release(u);
        return rc;
    }
    *out = u;
    return FG_OK;
}

int fg_upload_write(fg_upload *u, size_t offset, const void *bytes, size_t len)
{
    if (!u) return set_error(FG_ERR_ARG, "fg_upload_write: a null upload");
    if (!u->table) return set_error(FG_ERR_ARG, "fg_upload_write: the upload has ended");
    if (!bytes && len) return set_error(FG_ERR_ARG, "fg_upload_write: null bytes");
    // store.rs:95-97: writes arrive in order and stay within the tensor
    if (offset != u->received)
        return set_error(FG_ERR_SHAPE, "table upload: a write at byte " + std::to_string(offset) + ", " +
                                           std::to_string(u->received) + " expected (writes arrive in order)");
    if (len > u->total - u->received) return set_error(FG_ERR_FORMAT, "table upload: write past its end");
    const uint8_t *src = static_cast<const uint8_t *>(bytes);
    while (len) {
        const size_t take = std::min(len, kStage - u->fill);
        std::memcpy(u->host[u->cur] + u->fill, src, take);
        u->fill += take;
        u->received += take;
        src += take;
        len -= take;
        if (u->fill == kStage) {
            int rc = flush(u, sendable(u));
            if (rc) return rc;
        }
    }
    return FG_OK;
}

int fg_upload_end(fg_upload *u, fg_table **out)
{
    if (!u || !out) return set_error(FG_ERR_ARG, "fg_upload_end: a null argument");
    *out = nullptr;
    if (!u->table) return set_error(FG_ERR_ARG, "fg_upload_end: the upload has ended");
    // store.rs:130-137
    if (u->received != u->total)
        return set_error(FG_ERR_FORMAT, "table upload: " + std::to_string(u->received) + " of " + std::to_string(u->total) + " bytes");
    int rc = flush(u, u->fill);
    if (rc) return rc;
    const hipError_t e = hipStreamSynchronize(u->stream);
    if (e != hipSuccess) return check_hip(e, "fg_upload_end");
    *out = u->table;
    u->table = nullptr;
    release(u);
    return FG_OK;
}

int fg_upload_restart(fg_upload *u)
{
    if (!u) return set_error(FG_ERR_ARG, "fg_upload_restart: a null upload");
    if (!u->table) return set_error(FG_ERR_ARG, "fg_upload_restart: the upload has ended");
    // store.rs:148-158: what was written is forgotten; copies still in flight finish first
    for (int i = 0; i < 2; i++) FG_HIP(hipEventSynchronize(u->done[i]));
    u->received = u->sent = u->fill = 0;
    u->cur = 0;
    return FG_OK;
}

int fg_upload_free(fg_upload *u)
{
    release(u);
    return FG_OK;
}

}  // extern "C"
