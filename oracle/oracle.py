"""ctypes view of the CPU oracle (liboracle.so, built from fusor_oracle.c).

TEST INFRASTRUCTURE ONLY: the parity checker and the CPU baseline. Only tests/,
``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg may import this module; the
product (fusor-ai_amd/) never does.

Every function restates the fusor-ai reference (crates/kernels/src, scalar x86-64 backend);
the C source cites file:line for each.
"""

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, Q7B32, Q4B32, T2B128, Q8B32 = 0, 1, 2, 3, 4
NAMES = {F32: "F32", Q7B32: "Q7b32", Q4B32: "Q4b32", T2B128: "T2b128", Q8B32: "Q8b32"}
BLOCK, QUAD, TERNARY_GROUP = 32, 4, 128

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_S = ctypes.c_size_t
_I = ctypes.c_int
_F = ctypes.c_float


class Qwen2Shape(ctypes.Structure):
    _fields_ = [("hidden", _S), ("layers", _S), ("heads", _S), ("kv_heads", _S),
                ("head_dim", _S), ("ffn", _S), ("vocab", _S), ("capacity", _S),
                ("rope_base", _F), ("eps", _F), ("dtype", _I)]


class Qwen2Layer(ctypes.Structure):
    _fields_ = [("norm1", _P), ("norm2", _P), ("qkv", _P), ("o", _P), ("gate", _P),
                ("up", _P), ("down", _P), ("qkv_bias", _P)]


class Attention(ctypes.Structure):
    """or_attention: one int8 attention call (blocks/src/attention.rs:35-47)."""
    _fields_ = [("heads", _S), ("kv_heads", _S), ("head_dim", _S), ("images", _S), ("queries", _S), ("keys", _S),
                ("query", _P), ("query_stride", _S), ("query_offset", _S),
                ("key", _P), ("key_stride", _S), ("key_offset", _S),
                ("value", _P), ("value_stride", _S), ("value_offset", _S), ("fast", _I)]


def _declare(l):
    sig = {
        "or_group": (_I, [_I]), "or_zero_point": (_I, [_I]), "or_codes_per_byte": (_I, [_I]),
        "or_padded_values": (_S, [_S, _S]), "or_quant_len": (_S, [_I, _S, _S]),
        "or_byte_len": (_S, [_I, _S, _S]),
        "or_pack_lane": (None, [_I, _I, _P, _P]), "or_unpack_lane": (None, [_I, _P, _I, _P]),
        "or_quantize_group": (_F, [_I, _P, _P]),
        "or_encode": (_I, [_I, _S, _S, _P, _P]),
        "or_dequantize_row": (None, [_I, _S, _S, _P, _S, _P]),
        "or_quantize_rows": (None, [_P, _S, _I, _P, _P, _P]),
        "or_matmul": (_I, [_I, _S, _S, _P, _P, _P, _P, _S, _S, _S, _P, _P, _S, _P]),
        "or_matmul_fused": (_I, [_I, _S, _S, _P, _P, _P, _P, _S, _S, _S, _P, _P, _S, _P, _I]),
        "or_matmul_threaded": (_I, [_I, _S, _S, _P, _P, _P, _P, _S, _P, _P, _I]),
        "or_exp": (_F, [_F]), "or_silu": (_F, [_F]),
        "or_exp_fast": (_F, [_F]), "or_exponentials_apply": (_F, [_P, _S, _I]),
        "or_attend": (_I, [_P, _P]),
        "or_dot_f32": (_F, [_P, _P, _S]),
        "or_rms_norm": (None, [_P, _P, _S, _F, _P]),
        "or_rope_inv_freq": (None, [_F, _S, _P]),
        "or_rope_angles": (None, [_P, _S, _S, _P, _P]),
        "or_rope_half": (None, [_P, _S, _P, _P]),
        "or_softmax": (None, [_P, _S]),
        "or_weigh": (None, [_P, _S, _P, _S, _S, _P]),
        "or_rng_new": (None, [_P, ctypes.c_uint64]),
        "or_rng_next_u64": (ctypes.c_uint64, [_P]),
        "or_rng_uniform": (ctypes.c_double, [_P]),
        "or_rng_fill_normal": (None, [_P, _P, _S]),
        "or_qwen2_layer_forward": (_I, [_P, _P, _S, _P, _P, _S, _P, _P, _P, _I]),
        "or_qwen2_step": (_I, [_P, _P, _P, _P, _P, _P, _I, _S, _P, _P, _P, _I]),
        "or_qwen2_embed": (None, [_P, _P, _P, _S, _P]),
        "or_qwen2_read": (_I, [_P, _P, _P, _P, _P, _P, _P, _S, _S, _S, _P, _P, _P, _I]),
        "or_greedy": (_I, [_P, _S]),
    }
    for name, (res, args) in sig.items():
        f = getattr(l, name)
        f.restype = res
        f.argtypes = args


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def group(dtype):
    return lib().or_group(dtype)


def zero_point(dtype):
    return lib().or_zero_point(dtype)


def byte_len(dtype, rows, cols):
    return lib().or_byte_len(dtype, rows, cols)


def quant_len(dtype, rows, cols):
    return lib().or_quant_len(dtype, rows, cols)


def pack_lane(dtype, lane, codes, quad):
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    lib().or_pack_lane(dtype, lane, _ptr(codes), _ptr(quad))


def unpack_lane(dtype, quad, lane):
    out = np.zeros(BLOCK, np.uint8)
    quad = np.ascontiguousarray(quad, dtype=np.uint8)
    lib().or_unpack_lane(dtype, _ptr(quad), lane, _ptr(out))
    return out


def quantize_group(dtype, values):
    values = np.ascontiguousarray(values, dtype=np.float32)
    codes = np.zeros(len(values), np.uint8)
    scale = lib().or_quantize_group(dtype, _ptr(values), _ptr(codes))
    return np.float32(scale), codes


def encode(dtype, rows, cols, values):
    """Tensor::encode: f32 [rows, cols] to the reference's byte layout."""
    values = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    assert values.size == rows * cols
    out = np.zeros(byte_len(dtype, rows, cols), np.uint8)
    if lib().or_encode(dtype, rows, cols, _ptr(values), _ptr(out)) != 0:
        raise ValueError("not whole groups")
    return out


def dequantize_row(dtype, rows, cols, table, row):
    out = np.zeros(cols, np.float32)
    table = np.ascontiguousarray(table, dtype=np.uint8)
    lib().or_dequantize_row(dtype, rows, cols, _ptr(table), row, _ptr(out))
    return out


def dequantize(dtype, rows, cols, table):
    return np.stack([dequantize_row(dtype, rows, cols, table, r) for r in range(rows)])


def quantize_rows(x, dtype):
    """quantize_rows over whole groups: (int8 quants, f32 scales, i32 corrections)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    g = group(dtype)
    q = np.zeros(x.size, np.int8)
    s = np.zeros(x.size // g, np.float32)
    c = np.zeros(x.size // g, np.int32)
    lib().or_quantize_rows(_ptr(x), x.size, dtype, _ptr(q), _ptr(s), _ptr(c))
    return q, s, c


def matmul(dtype, n_rows, cols, table, q, s, c, rows, col_begin=0, col_end=None, bias=None,
           want_dots=False, fused=False):
    """The reference product of `rows` quantized rows over columns [col_begin, col_end); with
    `fused`, the NEON backend's scaling (one fused multiply-add per group)."""
    if col_end is None:
        col_end = (n_rows + 3) // 4 * 4
    width = col_end - col_begin
    out = np.zeros((rows, width), np.float32)
    groups = cols // group(dtype)
    dots = np.zeros((rows, width, groups), np.int32) if want_dots else None
    table = np.ascontiguousarray(table, dtype=np.uint8)
    q = np.ascontiguousarray(q, dtype=np.int8)
    s = np.ascontiguousarray(s, dtype=np.float32)
    c = np.ascontiguousarray(c, dtype=np.int32)
    if bias is not None:
        bias = np.ascontiguousarray(bias, dtype=np.float32)
        if bias.size < col_end:
            bias = np.concatenate([bias, np.zeros(col_end - bias.size, np.float32)])
    rc = lib().or_matmul_fused(dtype, n_rows, cols, _ptr(table), _ptr(q), _ptr(s), _ptr(c), rows,
                               col_begin, col_end, _ptr(bias), _ptr(out), width, _ptr(dots), int(bool(fused)))
    if rc != 0:
        raise ValueError("shape error")
    return (out, dots) if want_dots else out


def matmul_threaded(dtype, n_rows, cols, table, q, s, c, rows, bias=None, threads=1):
    out = np.zeros((rows, n_rows), np.float32)
    lib().or_matmul_threaded(dtype, n_rows, cols, _ptr(table), _ptr(q), _ptr(s), _ptr(c), rows,
                             _ptr(bias), _ptr(out), threads)
    return out


def exp(x):
    return np.float32(lib().or_exp(float(np.float32(x))))


def exp_fast(x):
    return np.float32(lib().or_exp_fast(float(np.float32(x))))


def exponentials_apply(scores, fast):
    """Exponentials::apply (ops.rs:168-191): (the exponentials, their sum)."""
    v = np.ascontiguousarray(scores, dtype=np.float32).copy()
    total = lib().or_exponentials_apply(_ptr(v), v.size, int(bool(fast)))
    return v, np.float32(total)


def attend(heads, kv_heads, head_dim, images, queries, keys, query, key, value, fast=False,
           query_layout=None, key_layout=None, value_layout=None):
    """attention::attend (blocks/src/attention.rs:81-214). Operands are flat f32 arrays with a
    (stride, offset) layout each (default: rows of heads * head_dim, or kv_heads * head_dim);
    returns [images * queries, heads * head_dim]."""
    q = np.ascontiguousarray(query, dtype=np.float32).reshape(-1)
    k = np.ascontiguousarray(key, dtype=np.float32).reshape(-1)
    v = np.ascontiguousarray(value, dtype=np.float32).reshape(-1)
    ql = query_layout or (heads * head_dim, 0)
    kl = key_layout or (kv_heads * head_dim, 0)
    vl = value_layout or (kv_heads * head_dim, 0)
    out = np.zeros((images * queries, heads * head_dim), dtype=np.float32)
    call = Attention(heads, kv_heads, head_dim, images, queries, keys, _ptr(q), ql[0], ql[1], _ptr(k), kl[0], kl[1],
                     _ptr(v), vl[0], vl[1], int(bool(fast)))
    if lib().or_attend(ctypes.byref(call), _ptr(out)):
        raise ValueError("attend: shapes do not fit")
    return out


def silu(x):
    return np.float32(lib().or_silu(float(np.float32(x))))


def rms_norm(x, weight, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    weight = np.ascontiguousarray(weight, dtype=np.float32)
    out = np.zeros_like(x)
    lib().or_rms_norm(_ptr(x), _ptr(weight), x.size, eps, _ptr(out))
    return out


def rope_tables(base, head_dim, positions):
    """cos/sin [positions, head_dim/2] as blocks::rotary computes them."""
    half = head_dim // 2
    inv = np.zeros(half, np.float32)
    lib().or_rope_inv_freq(base, head_dim, _ptr(inv))
    cos = np.zeros((positions, half), np.float32)
    sin = np.zeros((positions, half), np.float32)
    for p in range(positions):
        c = np.zeros(half, np.float32)
        s = np.zeros(half, np.float32)
        lib().or_rope_angles(_ptr(inv), half, p, _ptr(c), _ptr(s))
        cos[p], sin[p] = c, s
    return cos, sin


def rope_half(head, cos, sin):
    """ops::rope by halves (ops.rs:77-85) of one head: a rotated copy."""
    head = np.array(head, dtype=np.float32)
    cos = np.ascontiguousarray(cos, dtype=np.float32)
    sin = np.ascontiguousarray(sin, dtype=np.float32)
    assert cos.size == sin.size == head.size // 2
    lib().or_rope_half(_ptr(head), head.size, _ptr(cos), _ptr(sin))
    return head


def silu_rows(x):
    """silu (ops.rs:272-274) of every value."""
    return np.array([silu(v) for v in np.asarray(x, np.float32).reshape(-1)], np.float32)


def dot_f32(a, b):
    """dot_f32 (arch/scalar.rs:340-342): the products added in index order."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    assert a.size == b.size
    return np.float32(lib().or_dot_f32(_ptr(a), _ptr(b), a.size))


def softmax(x):
    x = np.array(x, dtype=np.float32)
    lib().or_softmax(_ptr(x), x.size)
    return x


def weigh(scores, values):
    """ops::weigh (ops.rs:329-342): the softmax of `scores` (returned) and the sum of the value
    rows [n, dim] weighted by it, in key order."""
    w = np.array(scores, dtype=np.float32)
    v = np.ascontiguousarray(values, dtype=np.float32)
    out = np.zeros(v.shape[1], np.float32)
    lib().or_weigh(_ptr(w), w.size, _ptr(v), v.shape[1], v.shape[1], _ptr(out))
    return w, out


class Rng:
    """rng.rs's Rng: SplitMix64-seeded xoshiro256**."""

    def __init__(self, seed):
        self._state = (ctypes.c_uint64 * 4)()
        lib().or_rng_new(ctypes.cast(self._state, ctypes.c_void_p), seed)

    def next_u64(self):
        return lib().or_rng_next_u64(ctypes.cast(self._state, ctypes.c_void_p))

    def uniform(self):
        return lib().or_rng_uniform(ctypes.cast(self._state, ctypes.c_void_p))

    def normal(self, n):
        out = np.zeros(n, np.float32)
        lib().or_rng_fill_normal(ctypes.cast(self._state, ctypes.c_void_p), _ptr(out), n)
        return out


class Qwen2:
    """The decoder step (blocks::transformer + lm) over numpy weights in reference bytes."""

    def __init__(self, shape, layers, final_norm, table):
        self.shape = shape
        self._keep = []
        arr = (Qwen2Layer * len(layers))()
        for i, ly in enumerate(layers):
            for key in ("norm1", "norm2", "qkv", "o", "gate", "up", "down", "qkv_bias"):
                v = ly.get(key)
                if v is not None:
                    v = np.ascontiguousarray(v)
                    self._keep.append(v)
                setattr(arr[i], key, _ptr(v) if v is not None else None)
        self.layers = arr
        self.final_norm = np.ascontiguousarray(final_norm, dtype=np.float32)
        self.table = np.ascontiguousarray(table, dtype=np.uint8)

    def step(self, kcache, vcache, token, position, threads=1, logits=True):
        sh = self.shape
        hidden = np.zeros(sh.hidden, np.float32)
        out = np.zeros(sh.vocab, np.float32) if logits else None
        nxt = ctypes.c_int(-1)
        rc = lib().or_qwen2_step(ctypes.byref(sh), ctypes.cast(self.layers, ctypes.c_void_p),
                                 _ptr(self.final_norm), _ptr(self.table), _ptr(kcache), _ptr(vcache),
                                 token, position, _ptr(hidden), _ptr(out), ctypes.byref(nxt), threads)
        if rc != 0:
            raise ValueError("position past the cache")
        return hidden, out, nxt.value

    def layer_forward(self, index, kcache, vcache, position, cos, sin, hidden, threads=1):
        hidden = np.array(hidden, dtype=np.float32)
        cos = np.ascontiguousarray(cos, dtype=np.float32)
        sin = np.ascontiguousarray(sin, dtype=np.float32)
        lib().or_qwen2_layer_forward(ctypes.byref(self.shape), ctypes.byref(self.layers[index]), index,
                                     _ptr(kcache), _ptr(vcache), position, _ptr(cos), _ptr(sin),
                                     _ptr(hidden), threads)
        return hidden

    def embed(self, ids):
        """Lm::embed (lm.rs:97-108): the table's rows of `ids`."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.zeros((ids.size, self.shape.hidden), np.float32)
        lib().or_qwen2_embed(ctypes.byref(self.shape), _ptr(self.table), _ptr(ids), ids.size, _ptr(out))
        return out

    def read(self, kcache, vcache, embeddings, first, chunk, threads=1, logits=True):
        """Reader::read (lm.rs:205-228): the rows of `embeddings` from position `first`, `chunk` rows
        per call of the stack; returns the last row's hidden state, logits and greedy token."""
        sh = self.shape
        emb = np.ascontiguousarray(embeddings, dtype=np.float32).reshape(-1, sh.hidden)
        hidden = np.zeros(sh.hidden, np.float32)
        out = np.zeros(sh.vocab, np.float32) if logits else None
        nxt = ctypes.c_int(-1)
        rc = lib().or_qwen2_read(ctypes.byref(sh), ctypes.cast(self.layers, ctypes.c_void_p), _ptr(self.final_norm),
                                 _ptr(self.table), _ptr(kcache), _ptr(vcache), _ptr(emb), emb.shape[0], first, chunk,
                                 _ptr(hidden), _ptr(out), ctypes.byref(nxt), threads)
        if rc != 0:
            raise ValueError("the cache holds every key the span sees")
        return hidden, out, nxt.value
