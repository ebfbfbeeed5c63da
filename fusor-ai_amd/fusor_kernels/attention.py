"""Int8 attention: attention::attend (blocks/src/attention.rs:24-214) on the GPU.

Keys and values are quantized at run time to Q7b32 rows (QuantizedMatrix), the scores and the
weighted values come from the quantized product, and the f32 steps between them follow the
reference's order (the keys' mean, Exponentials::apply, the division by each row's sum). One
call covers every (image, head); the reference's split of that work over a team's threads
(`ctx.split`, attention.rs:84) does not change a bit of the result, so there is no Ctx here.
"""

import ctypes
import enum
from dataclasses import dataclass

from ._lib import FgAttention, ShapeError, check, lib, ptr, stream_handle


class Exponentials(enum.IntEnum):
    """ops.rs:163-166: `Exact` is exp (within 2 ulp), `Fast` is exp_fast (within 6e-5)."""
    EXACT = 0
    FAST = 1


@dataclass
class Operand:
    """The rows of a query, key or value operand (attention.rs:24-30): head `h` of row `r` is
    the `head_dim` values at `r * stride + offset + h * head_dim` of the device f32 `values`."""
    values: object
    stride: int
    offset: int = 0


@dataclass
class Call:
    """One attention (attention.rs:32-47): `images` images, each of `queries` query rows over
    `keys` key and value rows, in `heads` query heads of `head_dim` over `kv_heads` key and value
    heads, each shared by consecutive query heads."""
    heads: int
    kv_heads: int
    head_dim: int
    images: int
    queries: int
    keys: int
    query: Operand
    key: Operand
    value: Operand
    exponentials: Exponentials = Exponentials.EXACT


def _check_operand(name, op, rows, heads, head_dim):
    import torch
    t = op.values
    if t.dtype != torch.float32 or not t.is_cuda or not t.is_contiguous():
        raise ShapeError(f"{name}: a contiguous float32 device tensor")
    if op.offset + heads * head_dim > op.stride:
        raise ShapeError(f"{name}: its heads run past the row stride")
    if (rows - 1) * op.stride + op.offset + heads * head_dim > t.numel():
        raise ShapeError(f"{name}: {rows} rows of stride {op.stride} do not fit in {t.numel()} values")


def attend(call, out, stream=None):
    """attention::attend (attention.rs:81-95) for the whole call into `out`, rows of
    `heads * head_dim` values (the scores scaled by 1/sqrt(head_dim)). `out` is a float32 device
    tensor of `images * queries` such rows."""
    c = call
    if c.heads <= 0 or c.kv_heads <= 0 or c.heads % c.kv_heads:
        raise ShapeError("the heads must be a positive multiple of the key heads")
    _check_operand("query", c.query, c.images * c.queries, c.heads, c.head_dim)
    _check_operand("key", c.key, c.images * c.keys, c.kv_heads, c.head_dim)
    _check_operand("value", c.value, c.images * c.keys, c.kv_heads, c.head_dim)
    import torch
    if out.dtype != torch.float32:
        raise ShapeError("out must be float32")
    if not out.is_cuda or not out.is_contiguous() or out.numel() < c.images * c.queries * c.heads * c.head_dim:
        raise ShapeError("out: a contiguous device tensor of images * queries rows of heads * head_dim")
    fg = FgAttention(c.heads, c.kv_heads, c.head_dim, c.images, c.queries, c.keys,
                     ptr(c.query.values), c.query.stride, c.query.offset,
                     ptr(c.key.values), c.key.stride, c.key.offset,
                     ptr(c.value.values), c.value.stride, c.value.offset, int(c.exponentials))
    check(lib().fg_attend(ctypes.byref(fg), ptr(out), stream_handle(stream)))
    return out
