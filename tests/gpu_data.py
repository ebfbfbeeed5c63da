"""Seeded synthetic inputs shared by the GPU tests."""

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
