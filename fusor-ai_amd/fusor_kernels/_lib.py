"""ctypes binding of libfusor_gpu.so (include/fusor_gpu.h).

The library is the only compute path: there is no CPU fallback. Loading fails loudly when the
built library is missing.
"""

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfusor_gpu.so")

FG_OK, FG_ERR_SHAPE, FG_ERR_FORMAT, FG_ERR_HIP, FG_ERR_NOMEM, FG_ERR_ARG = range(6)
FG_ACCUMULATE = 1
FG_FUSED_SCALE = 2
FG_PARALLEL_SUM = 4

_P = ctypes.c_void_p
_S = ctypes.c_size_t
_I = ctypes.c_int
_F = ctypes.c_float


class FgInput(ctypes.Structure):
    _fields_ = [("x", _P), ("quants", _P), ("scales", _P), ("corrections", _P)]


class FgAttention(ctypes.Structure):
    _fields_ = [("heads", _S), ("kv_heads", _S), ("head_dim", _S), ("images", _S), ("queries", _S), ("keys", _S),
                ("query", _P), ("query_stride", _S), ("query_offset", _S),
                ("key", _P), ("key_stride", _S), ("key_offset", _S),
                ("value", _P), ("value_stride", _S), ("value_offset", _S), ("exponentials", _I)]


class FgQwen2Shape(ctypes.Structure):
    _fields_ = [("hidden", _S), ("layers", _S), ("heads", _S), ("kv_heads", _S), ("head_dim", _S),
                ("ffn", _S), ("vocab", _S), ("capacity", _S), ("rope_base", _F), ("eps", _F),
                ("dtype", _I), ("exact", _I)]


class FgQwen2Layer(ctypes.Structure):
    _fields_ = [("norm1", _P), ("norm2", _P), ("qkv_bias", _P), ("qkv", _P), ("o", _P),
                ("gate", _P), ("up", _P), ("down", _P)]


class FgQwen2Probe(ctypes.Structure):
    _fields_ = [("query", _P), ("attention", _P), ("attended", _P), ("inner", _P), ("levels", _P),
                ("scales", _P), ("corrections", _P), ("out", _P)]


# Every symbol include/fusor_gpu.h declares, with its signature.
SIGNATURES = {
    "fg_last_error": (ctypes.c_char_p, []),
    "fg_version": (_I, []),
    "fg_table_create": (_I, [_P, _S, _I, _S, _S, _P, ctypes.POINTER(_P)]),
    "fg_table_create_device": (_I, [_P, _S, _I, _S, _S, _P, ctypes.POINTER(_P)]),
    "fg_table_free": (_I, [_P]),
    "fg_table_shape": (_I, [_P, ctypes.POINTER(_I), ctypes.POINTER(_S), ctypes.POINTER(_S)]),
    "fg_table_byte_len": (_S, [_I, _S, _S]),
    "fg_table_read": (_I, [_P, _P, _P]),
    "fg_upload_begin": (_I, [_I, _S, _S, _P, ctypes.POINTER(_P)]),
    "fg_upload_write": (_I, [_P, _S, _P, _S]),
    "fg_upload_end": (_I, [_P, ctypes.POINTER(_P)]),
    "fg_upload_restart": (_I, [_P]),
    "fg_upload_free": (_I, [_P]),
    "fg_encode": (_I, [_I, _S, _S, _P, _P, _P]),
    "fg_dequantize_row": (_I, [_P, _S, _P, _P]),
    "fg_qmatrix_create": (_I, [_S, _S, ctypes.POINTER(_P)]),
    "fg_qmatrix_reset": (_I, [_P, _S]),
    "fg_qmatrix_extend": (_I, [_P, _S, _P]),
    "fg_qmatrix_set_rows": (_I, [_P, _S, _S, _P, _P]),
    "fg_qmatrix_set_block": (_I, [_P, _S, _S, _P, _P]),
    "fg_attend": (_I, [ctypes.POINTER(FgAttention), _P, _P]),
    "fg_quantize_rows": (_I, [_P, _S, _I, _P, _P, _P, _P]),
    "fg_matmul": (_I, [_P, ctypes.POINTER(FgInput), _S, _S, _S, _P, _P, _S, _I, _P]),
    "fg_matmul_noalloc": (_I, [_P, ctypes.POINTER(FgInput), _S, _S, _S, _P, _P, _S, _I, _P]),
    "fg_matmul_dots": (_I, [_P, ctypes.POINTER(FgInput), _S, _S, _S, _P, _P]),
    "fg_qwen2_create": (_I, [ctypes.POINTER(FgQwen2Shape), _P, _P, _P, _P, _P, ctypes.POINTER(_P)]),
    "fg_qwen2_step": (_I, [_P, _I, _S, _P, _P, _P, _P]),
    "fg_qwen2_layer_forward": (_I, [_P, _S, _S, _P, _P]),
    "fg_qwen2_attention": (_I, [_P, _S, _S, _P, _P, _P, _P]),
    "fg_qwen2_layer_probe": (_I, [_P, _S, _S, _P, ctypes.POINTER(FgQwen2Probe), _P]),
    "fg_qwen2_embed": (_I, [_P, _P, _S, _P, _P]),
    "fg_qwen2_read": (_I, [_P, _P, _S, _S, _S, _P, _P, _P, _P]),
    "fg_qwen2_free": (_I, [_P]),
}

_lib = None


class Error(Exception):
    """kernels::Error (lib.rs:34-38): a tensor whose type or shape does not fit its use."""


class FormatError(Error):
    """Error::Format."""


class ShapeError(AssertionError):
    """A shape or range the reference asserts on (a panic there)."""


class GpuError(RuntimeError):
    """The HIP runtime failed."""


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built: run __graft_entry__.build() (make -C fusor-ai_amd)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(handle, name)
            f.restype = res
            f.argtypes = args
        _lib = handle
    return _lib


def check(rc):
    if rc == FG_OK:
        return
    msg = lib().fg_last_error().decode()
    if rc == FG_ERR_FORMAT:
        raise FormatError(msg)
    if rc == FG_ERR_SHAPE:
        raise ShapeError(msg)
    if rc == FG_ERR_ARG:
        raise ValueError(msg)
    raise GpuError(msg)


def stream_handle(stream=None):
    """The hipStream_t of `stream` (torch's current stream by default)."""
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def ptr(t):
    """Device address of a torch tensor (or None)."""
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())
