"""Bounds on what a change of f32 summation order can do to the decoder's rows.

The decoder's parallel order keeps every integer of the reference and every group term
t_g = fl(fl((float)D_g) * fl(ws * as)) of a product; it changes only the order of f32 additions:
a projection's group sums, the RMSNorm's sum of squares, the attention's softmax total and weighted
sums. These helpers give, from the oracle's own quantities, how far two orders can land apart, so a
test can hold the GPU's parallel order to them output by output:

* two orders of the same G terms differ by at most 2 (G - 1) u sum_g |t_g| (u = 2^-24: each
  order is within (G - 1) u sum |t_g| of the exact sum);
* two orders of the sum of H squares (all non-negative) differ by at most 2 (H - 1) u of the
  sum, which moves the RMSNorm's inverse, and with it every normed value and the group scales
  d = amax / 127 of its quantization, by a relative `norm_slack(H)`. The ratio x / d, and so every
  level, moves only by the few roundings that do not cancel: a level can change only where x / d
  lies within `FLIP_MARGIN` of a half-integer, and then by one.
"""

import numpy as np

from oracle import oracle as O

U = 2.0 ** -24
# |x' / d' - x / d| for two normings of one row that differ only in the common inverse: the product
# x * inverse * weight, amax / 127 and x / d each round (under 8 u relative), times the largest
# quotient 127, with a factor of two to spare
FLIP_MARGIN = 2 * 8 * U * 127


def weight_scales(dtype, rows, cols, data):
    """ws[n, g] from the reference bytes: f32 at ((q G + g) 4 + lane) after the codes
    (tensor.rs:1-9)."""
    quads, groups = (rows + 3) // 4, cols // O.group(dtype)
    raw = np.ascontiguousarray(data[O.quant_len(dtype, rows, cols):]).view(np.float32)
    return raw.reshape(quads, groups, 4).transpose(0, 2, 1).reshape(quads * 4, groups)


def group_terms(dtype, rows, cols, data, dots, scales):
    """t[n, g] = fl(fl((float)D) * fl(ws * as)) of one activation row: the terms every order adds."""
    ws = weight_scales(dtype, rows, cols, data)[: dots.shape[0]]
    p = (ws * np.asarray(scales, np.float32)[None, :]).astype(np.float32)
    return (dots.astype(np.float32) * p).astype(np.float32)


def reorder_bound(terms):
    """2 (G - 1) u sum_g |t_g| per output."""
    G = terms.shape[1]
    return 2 * (G - 1) * U * np.abs(terms.astype(np.float64)).sum(axis=1)


def norm_slack(h):
    """Relative change of the RMSNorm's inverse (ops.rs:7-16) between two orders of its H squares:
    half the sum's 2 (H - 1) u, plus the division, the square root and the reciprocal."""
    return (h - 1) * U + 8 * U


def flip_allowance(dtype, rows, cols, data, x, scales):
    """Per output n: sum over the inputs i whose quotient x_i / d lies within FLIP_MARGIN of a
    half-integer of |w[n, i]| * as[g(i)], with w the dequantized weight ws * (u - zp): what one
    level step at each of those inputs can move the output by (1 + 4u to spare)."""
    x = np.asarray(x, np.float32)
    g = O.group(dtype)
    d = np.repeat(np.asarray(scales, np.float32), g)
    t = (x / d).astype(np.float64)
    near = np.abs(np.abs(t - np.floor(t)) - 0.5) <= FLIP_MARGIN
    if not near.any():
        return np.zeros((rows + 3) // 4 * 4)
    cols_near = np.nonzero(near)[0]
    w = np.stack([O.dequantize_row(dtype, rows, cols, data, r)[cols_near] for r in range(rows)])
    allow = (np.abs(w.astype(np.float64)) * d[cols_near].astype(np.float64)[None, :]).sum(axis=1) * (1 + 4 * U)
    return np.concatenate([allow, np.zeros((rows + 3) // 4 * 4 - rows)])


def projection_bound(dtype, rows, cols, data, x, scales, dots, normed):
    """Per output, how far a parallel-order projection of row `x` (quantized to `scales`, with the
    oracle's int32 `dots`) can be from the oracle's group-order one. `normed`: x comes out of an
    RMSNorm whose sum the parallel order also reorders (its inverse then moves by norm_slack, and
    levels near a rounding boundary may step), else the two sides quantize identical rows."""
    terms = group_terms(dtype, rows, cols, data, dots, scales)
    abs_sum = np.abs(terms.astype(np.float64)).sum(axis=1)
    if not normed:
        return reorder_bound(terms)
    slack = norm_slack(cols) + 4 * U
    flips = flip_allowance(dtype, rows, cols, data, x, scales)[:terms.shape[0]]
    moved = abs_sum * slack + flips
    G = terms.shape[1]
    return moved + 2 * (G - 1) * U * (abs_sum + moved)


def rounded(bound, value):
    """A bound on |fl(a') - fl(a)| from |a' - a| <= bound, |a| = |value|: the two roundings."""
    v = np.abs(np.asarray(value, np.float64))
    return bound * (1 + 2 * U) + U * (2 * v + bound)


def added(bound, want):
    """fl(h + y') against fl(h + y) with |y' - y| <= bound and want = fl(h + y)."""
    return rounded(bound, want)


def rotated(bound_x, bound_y, x, y, cos, sin):
    """Bounds on the halves of ops::rope (ops.rs:77-85), x' = x c - y s and y' = y c + x s, from bounds
    on x and y (the oracle's unrotated halves)."""
    c = np.abs(np.asarray(cos, np.float64))
    s = np.abs(np.asarray(sin, np.float64))
    ax, ay = np.abs(np.asarray(x, np.float64)), np.abs(np.asarray(y, np.float64))
    bx = c * bound_x + s * bound_y + 4 * U * (ax * c + ay * s) + 4 * U * (bound_x + bound_y)
    by = c * bound_y + s * bound_x + 4 * U * (ay * c + ax * s) + 4 * U * (bound_x + bound_y)
    return bx, by


def swiglu_bound(gate, up, bound_gate, bound_up):
    """fl(silu(g') * u') against fl(silu(g) * u) (layer.rs:321-341): silu's slope lies in
    [-0.1, 1.1], and its evaluation (ops.rs:272-274, through the exp polynomial) rounds within a few
    ulps, taken as 16 u of |silu(g)| and of its change."""
    g = np.asarray(gate, np.float64)
    u = np.abs(np.asarray(up, np.float64))
    s = np.abs(g / (1 + np.exp(-g)))
    ds = 1.1 * bound_gate + 16 * U * (2 * s + bound_gate)
    return ds * (u + bound_up) + s * bound_up + 2 * U * (s * u + ds * (u + bound_up) + s * bound_up)
