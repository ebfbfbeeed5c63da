"""The Qwen2 decoder step on the GPU (blocks::transformer + blocks::lm with one row).

Weights are `Table`s (reference bytes uploaded once), norms and biases device f32 tensors, the KV
cache two device tensors [layers, kv_heads, capacity, head_dim]. `step` runs the embedding, every
layer, the final norm, the logits and the greedy token (transformer.rs:294-341, lm.rs:97-179).
"""

import ctypes
from dataclasses import dataclass

from . import _lib
from ._lib import FgQwen2Layer, FgQwen2Probe, FgQwen2Shape, check, lib, ptr, stream_handle


@dataclass
class Shape:
    """transformer::Shape (transformer.rs:54-67) for Qwen2, plus the vocabulary and the cache."""
    hidden: int = 896
    layers: int = 24
    heads: int = 14
    kv_heads: int = 2
    head_dim: int = 64
    ffn: int = 4864
    vocab: int = 151936
    capacity: int = 512
    rope_base: float = 1e6
    eps: float = 1e-6

    def qkv(self):
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    def width(self):
        return self.heads * self.head_dim


class Qwen2:
    def __init__(self, shape, dtype, layers, final_norm, table, kcache, vcache, exact=False):
        """layers: dicts with Tables qkv/o/gate/up/down and device tensors norm1/norm2/qkv_bias."""
        self.shape, self.layers, self.final_norm, self.table = shape, layers, final_norm, table
        self.kcache, self.vcache = kcache, vcache
        arr = (FgQwen2Layer * shape.layers)()
        for i, ly in enumerate(layers):
            arr[i] = FgQwen2Layer(ptr(ly["norm1"]), ptr(ly["norm2"]), ptr(ly.get("qkv_bias")), ly["qkv"].handle,
                                  ly["o"].handle, ly["gate"].handle, ly["up"].handle, ly["down"].handle)
        self._arr = arr
        sh = FgQwen2Shape(shape.hidden, shape.layers, shape.heads, shape.kv_heads, shape.head_dim, shape.ffn,
                          shape.vocab, shape.capacity, shape.rope_base, shape.eps, int(dtype), 1 if exact else 0)
        handle = ctypes.c_void_p()
        check(lib().fg_qwen2_create(ctypes.byref(sh), ctypes.cast(arr, ctypes.c_void_p), ptr(final_norm), table.handle,
                                    ptr(kcache), ptr(vcache), ctypes.byref(handle)))
        self.handle = handle

    def __del__(self):
        h = getattr(self, "handle", None)
        if h is not None and _lib._lib is not None:
            _lib._lib.fg_qwen2_free(h)
            self.handle = None

    def step(self, token, position, hidden=None, logits=None, next_token=None, stream=None):
        check(lib().fg_qwen2_step(self.handle, int(token), int(position), ptr(hidden), ptr(logits), ptr(next_token),
                                  stream_handle(stream)))

    def embed(self, ids, out=None, stream=None):
        """Lm::embed (lm.rs:97-108): the table's rows of the device int32 token ids, [count, hidden]."""
        import torch
        if out is None:
            out = torch.empty((ids.numel(), self.shape.hidden), dtype=torch.float32, device=ids.device)
        check(lib().fg_qwen2_embed(self.handle, ptr(ids), ids.numel(), ptr(out), stream_handle(stream)))
        return out

    def read(self, embeddings, first, chunk, hidden=None, logits=None, next_token=None, stream=None):
        """Reader::read (lm.rs:205-228): the device rows `embeddings` [count, hidden] from position
        `first`, `chunk` rows per call of the stack; the last row's residual row, logits and greedy
        token into the given device tensors."""
        count = embeddings.numel() // self.shape.hidden
        check(lib().fg_qwen2_read(self.handle, ptr(embeddings), count, int(first), int(chunk), ptr(hidden), ptr(logits),
                                  ptr(next_token), stream_handle(stream)))

    def layer_forward(self, layer, position, hidden, stream=None):
        check(lib().fg_qwen2_layer_forward(self.handle, layer, position, ptr(hidden), stream_handle(stream)))

    def attention(self, layer, position, hidden, query, row, stream=None):
        """One layer's attention over `hidden` as the step runs it (an inspection): the rotated
        query heads into `query` and the attention's f32 output row into `row` (device tensors of
        heads * head_dim); the position's key and value are kept in the caches."""
        check(lib().fg_qwen2_attention(self.handle, layer, position, ptr(hidden), ptr(query), ptr(row),
                                       stream_handle(stream)))

    def probe(self, layer, position, hidden, stream=None):
        """One layer over `hidden` as the step runs it, returning what it forms on the way (an
        inspection): the rotated query heads, the attention row before the output projection
        quantizes it, the residual row after that projection, silu(gate)·up, its levels, scales and
        corrections for the down projection, and the layer's output row (device tensors)."""
        import torch
        sh = self.shape
        dev = hidden.device
        f32 = dict(dtype=torch.float32, device=dev)
        out = {"query": torch.empty(sh.width(), **f32), "attention": torch.empty(sh.width(), **f32),
               "attended": torch.empty(sh.hidden, **f32), "inner": torch.empty(sh.ffn, **f32),
               "levels": torch.empty(sh.ffn, dtype=torch.int8, device=dev),
               "scales": torch.empty(sh.ffn // 32, **f32),
               "corrections": torch.empty(sh.ffn // 32, dtype=torch.int32, device=dev),
               "out": torch.empty(sh.hidden, **f32)}
        pr = FgQwen2Probe(*(ptr(out[k]) for k in ("query", "attention", "attended", "inner", "levels", "scales",
                                                  "corrections", "out")))
        check(lib().fg_qwen2_layer_probe(self.handle, layer, position, ptr(hidden), ctypes.byref(pr),
                                         stream_handle(stream)))
        return out
