"""Activation quantization and the quantized product (matmul.rs), on the GPU.

`quantize_rows`, `QuantizedRows.input` and `matmul` keep the reference's names and argument
meaning; activations and outputs are device tensors (torch, float32 / int8 / int32).
"""

import ctypes

from . import _lib
from ._lib import FgInput, ShapeError, check, lib, ptr, stream_handle
from .tensor import BLOCK, QUAD, DType, QuantFormat

ROWS_PER_CALL = 64  # matmul.rs:407


def quantize_rows(x, fmt, quants, scales, corrections):
    """quantize_rows (matmul.rs:233-257): `x` (device f32), whole groups of `fmt`, to int8 levels
    with each group's scale (absmax / 127) and correction (-zero_point * Σq)."""
    fmt = QuantFormat(fmt)
    check(lib().fg_quantize_rows(ptr(x), x.numel(), int(fmt), ptr(quants), ptr(scales), ptr(corrections),
                                 stream_handle()))


class Quantized:
    """matmul.rs:104-112"""

    def __init__(self, fmt, quants, scales, corrections):
        self.format, self.quants, self.scales, self.corrections = QuantFormat(fmt), quants, scales, corrections


class Input:
    """matmul.rs:114-147: f32 rows (quantized inside the product) or rows quantized for a format."""

    def __init__(self, f32=None, quant=None):
        self.f32, self.quant = f32, quant

    def rows(self, width):
        return (self.f32.numel() if self.f32 is not None else self.quant.quants.numel()) // width

    def block(self, width, start, end):
        """Input::block: rows start..end."""
        if self.f32 is not None:
            return Input(f32=self.f32.reshape(-1)[start * width:end * width])
        q = self.quant
        per_row = width // q.format.group()
        return Input(quant=Quantized(q.format, q.quants[start * width:end * width], q.scales[start * per_row:end * per_row],
                                     q.corrections[start * per_row:end * per_row]))

    def ffi(self):
        if self.f32 is not None:
            return FgInput(ptr(self.f32), None, None, None)
        q = self.quant
        return FgInput(None, ptr(q.quants), ptr(q.scales), ptr(q.corrections))


class QuantizedRows:
    """matmul.rs:26-33,149-229: rows of activations quantized for one weight format, on the device."""

    def __init__(self):
        self.quants = self.scales = self.corrections = None

    def input(self, weights, x):
        """Prepares `x` (device f32, whole rows of weights.cols) as the input of `weights`."""
        import torch
        if x.numel() % weights.cols:
            raise ShapeError("the input is whole rows of the weights' width")
        fmt = weights.format
        n = x.numel()
        g = fmt.group()
        self.quants = torch.empty(n, dtype=torch.int8, device=x.device)
        self.scales = torch.empty(n // g, dtype=torch.float32, device=x.device)
        self.corrections = torch.empty(n // g, dtype=torch.int32, device=x.device)
        quantize_rows(x.reshape(-1), fmt, self.quants, self.scales, self.corrections)
        return Input(quant=Quantized(fmt, self.quants, self.scales, self.corrections))


class QuantizedMatrix:
    """QuantizedMatrix (matmul.rs:35-102): a Q7b32 matrix quantized at run time, row by row (an
    attention's keys and values), on the device; `matrix()` multiplies like a model's weights."""

    def __init__(self, capacity=256, max_cols=4096):
        from .tensor import Table
        handle = ctypes.c_void_p()
        check(lib().fg_qmatrix_create(capacity, max_cols, ctypes.byref(handle)))
        self.table = Table.__new__(Table)
        self.table.handle, self.table._dtype = handle, DType.Q7b32
        self.table.rows, self.table.cols = 0, max_cols

    def reset(self, cols):
        """Empties it for rows of `cols` values, a multiple of BLOCK."""
        if cols % BLOCK:
            raise ShapeError("rows of whole blocks")
        check(lib().fg_qmatrix_reset(self.table.handle, cols))
        self.table.rows, self.table.cols = 0, cols

    def extend(self, rows):
        """Appends `rows` rows, every block of which `set_block` then writes once."""
        check(lib().fg_qmatrix_extend(self.table.handle, rows, stream_handle()))
        self.table.rows += rows

    def push(self, row):
        """Appends `row` (a device f32 tensor of cols values)."""
        if row.numel() != self.table.cols:
            raise ShapeError("a row of the matrix's width")
        index = self.table.rows
        self.extend(1)
        self.set_rows(index, row)

    def set_rows(self, first, values):
        """Rows first.. from a device f32 tensor of whole rows (every block of each row)."""
        count = values.numel() // self.table.cols
        check(lib().fg_qmatrix_set_rows(self.table.handle, first, count, ptr(values), stream_handle()))

    def set_block(self, row, block, values):
        """Block `block` of row `row` from 32 device f32 values."""
        if values.numel() != BLOCK:
            raise ShapeError("a block of 32 values")
        check(lib().fg_qmatrix_set_block(self.table.handle, row, block, ptr(values), stream_handle()))

    @property
    def rows(self):
        return self.table.rows

    @property
    def cols(self):
        return self.table.cols

    def matrix(self):
        return self.table.matrix()


def _check_input(weights, x):
    if x.quant is not None and x.quant.format != weights.format:
        raise ShapeError("the input is prepared for the weights' format")  # matmul.rs:301-304


def _check_device_f32(name, t, extent):
    """A caller's float32 device tensor whose storage holds `extent` values from its first one (a
    strided view counts the storage behind it), so that the kernels' reads and writes stay in it."""
    import torch
    if t.dtype != torch.float32 or t.device.type != "cuda":
        raise ShapeError(f"{name} must be a float32 device tensor")
    room = t.untyped_storage().nbytes() // 4 - t.storage_offset()
    if room < extent:
        raise ShapeError(f"{name} holds {room} values from its first, {extent} needed")


def matmul(weights, x, cols, store=None, bias=None, out=None, accumulate=False, fused=False, parallel=False):
    """matmul (matmul.rs:265-276) over output columns `cols` (a range of whole quads).

    Returns the device tensor [rows, len(cols)] of results; with `store`, also calls
    store(row, first_col, [4 floats]) per row and quad, in the reference's order. The results are
    the scalar backend's bits, or with `fused` the NEON backend's (each group's total scaled with
    one fused multiply-add, arch/neon.rs:140-154). `parallel` (one row) sums each output's group
    terms as the decoder's parallel order does: the same terms, reordered additions.
    """
    import torch
    if cols.start % QUAD or cols.stop % QUAD:
        raise ShapeError("columns in whole quads")  # matmul.rs:271-274
    _check_input(weights, x)
    rows = x.rows(weights.cols)
    width = cols.stop - cols.start
    if out is None:
        out = torch.empty((rows, width), dtype=torch.float32, device="cuda")
    if out.dim() == 2:
        if out.shape[1] < width or out.shape[0] < rows or out.stride(1) != 1:
            raise ShapeError(f"out of shape {list(out.shape)} for {rows} rows of {width} columns")
        ld = out.stride(0)
    else:
        if not out.is_contiguous():
            raise ShapeError("out must be contiguous")
        ld = width
    if rows and width:
        _check_device_f32("out", out, (rows - 1) * ld + width)
    if bias is not None:
        _check_device_f32("bias", bias, min(weights.rows, cols.stop))
    inp = x.ffi()
    flags = (_lib.FG_ACCUMULATE if accumulate else 0) | (_lib.FG_FUSED_SCALE if fused else 0) | \
        (_lib.FG_PARALLEL_SUM if parallel else 0)
    check(lib().fg_matmul(weights.table.handle, ctypes.byref(inp), rows, cols.start, cols.stop, ptr(bias), ptr(out),
                          ld, flags, stream_handle()))
    if store is not None:
        host = out.cpu().numpy().reshape(-1)
        for r in range(rows):
            for first in range(0, width, QUAD):
                at = r * ld + first
                store(r, cols.start + first, host[at:at + QUAD].tolist())
    return out


def matmul_dots(weights, x, cols):
    """The int32 group accumulators of the same product: [rows, len(cols), groups]."""
    import torch
    if cols.start % QUAD or cols.stop % QUAD:
        raise ShapeError("columns in whole quads")
    _check_input(weights, x)
    rows = x.rows(weights.cols)
    groups = weights.cols // weights.format.group()
    dots = torch.empty((rows, cols.stop - cols.start, groups), dtype=torch.int32, device="cuda")
    inp = x.ffi()
    check(lib().fg_matmul_dots(weights.table.handle, ctypes.byref(inp), rows, cols.start, cols.stop, ptr(dots),
                               stream_handle()))
    return dots
