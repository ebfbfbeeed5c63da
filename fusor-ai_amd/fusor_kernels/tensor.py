"""Weight tensors and the device views a model reads (tensor.rs, quant.rs).

`Tensor` keeps the reference's bytes on the host (quad-major codes, then f32 scales,
tensor.rs:1-9), so a bundle loader fills it exactly as it fills the reference's. `Table` is the
device mirror a product reads: uploaded once, freed with the object.
"""

import ctypes
import enum

import numpy as np

from . import _lib
from ._lib import FormatError, check, lib, ptr, stream_handle

BLOCK = 32
QUAD = 4
TERNARY_GROUP = 128


class DType(enum.IntEnum):
    """tensor.rs:19-24; Q8b32 is this library's signed 8-bit extension."""
    F32 = 0
    Q7b32 = 1
    Q4b32 = 2
    T2b128 = 3
    Q8b32 = 4

    def quant_format(self):
        return None if self is DType.F32 else QuantFormat(int(self))


class QuantFormat(enum.IntEnum):
    """quant.rs:32-87"""
    Q7b32 = 1
    Q4b32 = 2
    T2b128 = 3
    Q8b32 = 4

    def group(self):
        return TERNARY_GROUP if self is QuantFormat.T2b128 else BLOCK

    def zero_point(self):
        return {QuantFormat.Q7b32: 64, QuantFormat.Q4b32: 8, QuantFormat.T2b128: 1, QuantFormat.Q8b32: 0}[self]

    def codes_per_byte(self):
        return {QuantFormat.Q4b32: 2, QuantFormat.T2b128: 4}.get(self, 1)


def padded_values(rows, cols):
    """tensor.rs:55-57"""
    return (rows + QUAD - 1) // QUAD * QUAD * cols


def byte_len(dtype, shape):
    """tensor.rs:39-51"""
    dtype = DType(dtype)
    count = int(np.prod(shape)) if len(shape) else 1
    fmt = dtype.quant_format()
    if fmt is None:
        return count * 4
    padded = padded_values(*shape) if len(shape) == 2 else count
    return padded // fmt.codes_per_byte() + padded // fmt.group() * 4


def _check_quantized(fmt, shape):
    """tensor.rs:162-171"""
    if len(shape) == 2 and shape[1] % fmt.group() == 0:
        return
    raise FormatError(f"a {fmt.name} tensor of shape {list(shape)}: a matrix of whole groups of "
                      f"{fmt.group()} expected")


class Tensor:
    def __init__(self, dtype, shape, data):
        self._dtype = DType(dtype)
        self._shape = list(shape)
        self._bytes = data

    @classmethod
    def zeroed(cls, dtype, shape):
        return cls(dtype, shape, np.zeros(byte_len(dtype, shape), np.uint8))

    @classmethod
    def encode(cls, dtype, shape, values):
        """Tensor::encode (tensor.rs:97-143): the quantization runs on the GPU."""
        import torch
        dtype = DType(dtype)
        shape = list(shape)
        values = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
        count = int(np.prod(shape))
        if values.size != count:
            raise FormatError(f"{values.size} values for a tensor of shape {shape}")
        fmt = dtype.quant_format()
        if fmt is None:
            return cls(dtype, shape, values.view(np.uint8).copy())
        _check_quantized(fmt, shape)
        rows, cols = shape
        dev_values = torch.from_numpy(values).to("cuda")
        out = torch.empty(byte_len(dtype, shape), dtype=torch.uint8, device="cuda")
        check(lib().fg_encode(int(dtype), rows, cols, ptr(dev_values), ptr(out), stream_handle()))
        return cls(dtype, shape, out.cpu().numpy())

    def dtype(self):
        return self._dtype

    def shape(self):
        return self._shape

    def bytes(self):
        return self._bytes


class Vector:
    """An f32 vector (tensor.rs:173-192), resident on the device as a torch tensor."""

    def __init__(self, tensor):
        if tensor.dtype() != DType.F32 or len(tensor.shape()) != 1:
            raise FormatError(f"a {tensor.dtype().name} tensor of shape {tensor.shape()}: an f32 vector expected")
        import torch
        self._host = tensor.bytes().view(np.float32)
        self.device = torch.from_numpy(self._host.copy()).to("cuda")

    def values(self):
        return self._host


class Table:
    """tensor.rs:194-243: a quantized [rows, cols] matrix, on the device."""

    def __init__(self, tensor, stream=None):
        dtype, shape = tensor.dtype(), tensor.shape()
        fmt = dtype.quant_format()
        if fmt is None:
            raise FormatError(f"a F32 tensor of shape {shape}: the GPU path takes quantized tables")
        _check_quantized(fmt, shape)
        if len(shape) != 2:
            raise FormatError(f"a tensor of shape {shape}: a matrix expected")
        data = np.ascontiguousarray(tensor.bytes(), dtype=np.uint8)
        handle = ctypes.c_void_p()
        check(lib().fg_table_create(data.ctypes.data_as(ctypes.c_void_p), data.size, int(dtype), shape[0], shape[1],
                                    stream_handle(stream), ctypes.byref(handle)))
        self.handle = handle
        self._dtype = dtype
        self.rows, self.cols = shape

    @classmethod
    def from_device_bytes(cls, dtype, rows, cols, data, stream=None):
        """A table from reference bytes already on the device (a torch uint8 tensor)."""
        self = cls.__new__(cls)
        handle = ctypes.c_void_p()
        check(lib().fg_table_create_device(ptr(data), data.numel(), int(dtype), rows, cols, stream_handle(stream),
                                           ctypes.byref(handle)))
        self.handle, self._dtype, self.rows, self.cols = handle, DType(dtype), rows, cols
        return self

    def __del__(self):
        h = getattr(self, "handle", None)
        if h is not None and _lib._lib is not None:
            _lib._lib.fg_table_free(h)
            self.handle = None

    def dtype(self):
        return self._dtype

    def matrix(self):
        return Matrix(self)

    def reference_bytes(self):
        """The bytes back in the reference layout (a host numpy array)."""
        import torch
        out = torch.empty(byte_len(self._dtype, [self.rows, self.cols]), dtype=torch.uint8, device="cuda")
        check(lib().fg_table_read(self.handle, ptr(out), stream_handle()))
        return out.cpu().numpy()

    def dequantize(self):
        """Every row as f32 (tensor.rs:234-242), a device tensor [rows, cols]."""
        import torch
        out = torch.empty((self.rows, self.cols), dtype=torch.float32, device="cuda")
        m = self.matrix()
        for r in range(self.rows):
            m.dequantize_row(r, out[r])
        return out


class TableUpload:
    """A quantized table streamed onto the device piece by piece, as bundle::Store::write receives
    a part's bytes (bundle/src/store.rs:90-126), then handed over as a `Table` once every byte came
    (Store::end_part, store.rs:129-146; Table::load, bundle/src/load.rs:72-84)."""

    def __init__(self, dtype, shape, stream=None):
        dtype = DType(dtype)
        fmt = dtype.quant_format()
        if fmt is None or len(shape) != 2:
            raise FormatError(f"a {dtype.name} tensor of shape {list(shape)}: a quantized matrix expected")
        _check_quantized(fmt, shape)
        handle = ctypes.c_void_p()
        check(lib().fg_upload_begin(int(dtype), shape[0], shape[1], stream_handle(stream), ctypes.byref(handle)))
        self.handle, self._dtype, self._shape = handle, dtype, list(shape)
        self.received = 0
        self.len = byte_len(dtype, shape)

    def write(self, piece):
        """The next bytes (anything exposing the buffer protocol: bytes, a numpy uint8 array...)."""
        view = memoryview(piece).cast("B")
        n = view.nbytes
        if n:
            buf = (ctypes.c_ubyte * n).from_buffer_copy(view) if view.readonly else (ctypes.c_ubyte * n).from_buffer(view)
            check(lib().fg_upload_write(self.handle, self.received, buf, n))
        else:
            check(lib().fg_upload_write(self.handle, self.received, None, 0))
        self.received += n

    def restart(self):
        check(lib().fg_upload_restart(self.handle))
        self.received = 0

    def end(self):
        """The table, once every byte was written."""
        out = ctypes.c_void_p()
        check(lib().fg_upload_end(self.handle, ctypes.byref(out)))
        self.handle = None
        t = Table.__new__(Table)
        t.handle, t._dtype = out, self._dtype
        t.rows, t.cols = self._shape
        return t

    def __del__(self):
        h = getattr(self, "handle", None)
        if h is not None and _lib._lib is not None:
            _lib._lib.fg_upload_free(h)
            self.handle = None


class Matrix:
    """A borrowed [rows, cols] view of a table (tensor.rs:65-81)."""

    def __init__(self, table):
        self.table = table
        self.rows, self.cols = table.rows, table.cols
        self.format = table.dtype().quant_format()

    def dequantize_row(self, row, out):
        """Matrix::dequantize_row (tensor.rs:247-271) into a device f32 tensor of cols values."""
        if out.numel() != self.cols:
            raise _lib.ShapeError("out.len() == cols")
        check(lib().fg_dequantize_row(self.table.handle, row, ptr(out), stream_handle()))
