"""Seeded synthetic inputs shared by the GPU tests."""

import math

import numpy as np

from oracle import oracle as O


def synthetic_table(dtype, rows, cols, seed, scale_lo=1e-3, scale_hi=1e-2):
    """Reference bytes of a [rows, cols] table with i.i.d. codes and scales: Q7b32 levels uniform in
    [-63, 63] (codes 1..127), Q8b32 in [-127, 127], Q4b32 nibbles 0..15, T2b128 bit pairs 0..2;
    scales uniform in [scale_lo, scale_hi]. Codes are i.i.d., so filling the quad layout directly is
    the same draw as packing row by row. Padding rows keep zero codes and zero scales
    (tensor.rs:83-88)."""
    rng = np.random.default_rng(seed)
    quads = (rows + 3) // 4
    blocks = cols // 32
    groups = cols // O.group(dtype)
    qb = 128 // {O.Q4B32: 2, O.T2B128: 4}.get(dtype, 1)
    codes = np.zeros((quads, blocks, qb), np.uint8)
    if dtype == O.Q7B32:
        codes[:] = rng.integers(1, 128, codes.shape, dtype=np.uint8)
    elif dtype == O.Q8B32:
        codes[:] = rng.integers(-127, 128, codes.shape, dtype=np.int16).astype(np.int8).view(np.uint8)
    elif dtype == O.Q4B32:
        codes[:] = rng.integers(0, 256, codes.shape, dtype=np.uint8)
    elif dtype == O.T2B128:
        pairs = rng.integers(0, 3, codes.shape + (4,), dtype=np.uint8)
        codes[:] = pairs[..., 0] | pairs[..., 1] << 2 | pairs[..., 2] << 4 | pairs[..., 3] << 6
    else:
        raise ValueError(dtype)
    scales = rng.uniform(scale_lo, scale_hi, (quads, groups, 4)).astype(np.float32)
    pad = quads * 4 - rows
    if pad:
        # zero the padding lanes' codes in the last quad and their scales
        last = np.zeros((blocks, qb), np.uint8)
        for lane in range(4 - pad):
            for b in range(blocks):
                block_codes = O.unpack_lane(dtype, codes[-1, b], lane)
                O.pack_lane(dtype, lane, block_codes, last[b])
        codes[-1] = last
        scales[-1, :, 4 - pad:] = 0.0
    return np.concatenate([codes.reshape(-1), scales.reshape(-1).view(np.uint8)])


def encoded_table(dtype, rows, cols, seed):
    rng = np.random.default_rng(seed)
    values = rng.standard_normal((rows, cols)).astype(np.float32)
    return O.encode(dtype, rows, cols, values)


def activations(rows, cols, seed, outliers=0.0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    if outliers:
        mask = rng.random((rows, cols)) < outliers
        x[mask] *= 20.0
    return x


def qwen2_model(dtype, hidden, layers, heads, kv_heads, head_dim, ffn, vocab, capacity, seed, synthetic):
    """Reference bytes, norms, biases and N(0,1) caches of a Qwen2 decoder: tables of synthetic codes
    (`synthetic`) or encoded N(0, 1/cols) weights; the oracle's shape record."""
    rng = np.random.default_rng(seed)
    qkv_w = (heads + 2 * kv_heads) * head_dim
    lys = []
    for li in range(layers):
        f = {}
        for j, (name, (r, c)) in enumerate({"qkv": (qkv_w, hidden), "o": (hidden, heads * head_dim), "gate": (ffn, hidden),
                                            "up": (ffn, hidden), "down": (hidden, ffn)}.items()):
            if synthetic:
                f[name] = synthetic_table(dtype, r, c, seed=seed * 1000 + li * 10 + j)
            else:
                f[name] = O.encode(dtype, r, c, (rng.standard_normal((r, c)) / math.sqrt(c)).astype(np.float32))
        f["norm1"] = (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
        f["norm2"] = (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
        f["qkv_bias"] = (0.1 * rng.standard_normal(qkv_w)).astype(np.float32)
        lys.append(f)
    final = (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
    table = synthetic_table(dtype, vocab, hidden, seed=seed + 7) if synthetic else \
        O.encode(dtype, vocab, hidden, rng.standard_normal((vocab, hidden)).astype(np.float32))
    kc = rng.standard_normal((layers, kv_heads, capacity, head_dim)).astype(np.float32)
    vc = rng.standard_normal((layers, kv_heads, capacity, head_dim)).astype(np.float32)
    sh = O.Qwen2Shape(hidden=hidden, layers=layers, heads=heads, kv_heads=kv_heads, head_dim=head_dim, ffn=ffn,
                      vocab=vocab, capacity=capacity, rope_base=1e6, eps=1e-6, dtype=dtype)
    return sh, lys, final, table, kc, vc
