"""Pins the CPU oracle before anything is checked against it.

Each check is independent of the oracle's own code: the reference's known answers and test
tolerances (file:line in fusor-ai's crates/kernels/src), closed forms, invariants and brute force
on small inputs, chosen so that a plausible slip (a wrong scale divisor, truncation for
ties-to-even, a transposed quad lane, a dropped correction, scales of the wrong group) fails one.
"""

import math

import numpy as np
import pytest

from oracle import oracle as O

FORMATS = [O.Q7B32, O.Q4B32, O.T2B128, O.Q8B32]


def pseudo_random(n, seed):
    """matmul.rs:772-780: an LCG over u32, values in [-1, 1)."""
    state = seed & 0xFFFFFFFF
    out = np.empty(n, np.float32)
    for i in range(n):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32(state >> 8) / np.float32(1 << 24) * np.float32(2.0) - np.float32(1.0)
    return out


def ramp(n):
    """tensor.rs:279-283"""
    return np.array([((i * 37 % 101) - 50.0) / 7.0 for i in range(n)], np.float32)


# ---------------------------------------------------------------- layout and weight formats

def test_ternary_rows_keep_their_codes_and_group_scales():
    """tensor.rs:319-330: byte 0 is 0b0001_1000 and ternary weights round-trip exactly."""
    cols = 2 * O.TERNARY_GROUP
    scales = [0.5, 0.25, 2.0, 0.125]
    values = np.array([scales[i // O.TERNARY_GROUP] * ((i * 7 % 3) - 1.0) for i in range(2 * cols)],
                      np.float32)
    table = O.encode(O.T2B128, 2, cols, values)
    assert table[0] == 0b0001_1000
    assert np.array_equal(O.dequantize(O.T2B128, 2, cols, table).reshape(-1), values)


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q4B32])
def test_quantized_rows_dequantize_within_one_step(dtype):
    """tensor.rs:285-317: Q7 within largest/126, Q4 within largest/8 (+1e-5)."""
    values = ramp(4 * 64).reshape(4, 64)
    table = O.encode(dtype, 4, 64, values)
    for row in range(4):
        got = O.dequantize_row(dtype, 4, 64, table, row)
        for b in range(2):
            block = values[row, b * 32:(b + 1) * 32]
            largest = np.max(np.abs(block))
            tol = largest / 126.0 if dtype == O.Q7B32 else largest / 8.0
            assert np.all(np.abs(got[b * 32:(b + 1) * 32] - block) <= tol + 1e-5)


@pytest.mark.parametrize("group,scale,codes", [
    # the first value of largest magnitude, sign kept, over -8 (quant.rs:151-166), worked by hand:
    ([0.5, 8.0, -2.0, 0.0], -1.0, [8, 0, 10, 8]),   # positive extreme; 0.5 / -1 rounds to -0
    ([-8.0, 8.0], 1.0, [0, 15]),                     # the first of equal magnitudes; 16 clamps to 15
    ([8.0, -8.0], -1.0, [0, 15]),
    ([-1.0, 4.0, -3.0], -0.5, [10, 0, 14]),
])
def test_q4_scale_is_the_signed_first_extreme(group, scale, codes):
    """Known answers a scale from |extreme|, or from the last extreme, would fail."""
    values = np.zeros(32, np.float32)
    values[:len(group)] = group
    got_scale, got_codes = O.quantize_group(O.Q4B32, values)
    assert got_scale == np.float32(scale)
    assert got_codes[:len(codes)].tolist() == codes
    assert got_codes[len(codes):].tolist() == [8] * (32 - len(codes))


def test_a_row_of_subnormal_values_keeps_seven_bit_codes():
    """matmul.rs:845-856: one value of bits 94, the rest zero, codes [127, 64]."""
    row = np.zeros(32, np.float32)
    row[0] = np.frombuffer(np.uint32(94).tobytes(), np.float32)[0]
    scale, codes = O.quantize_group(O.Q7B32, row)
    assert list(codes[:2]) == [127, 64]
    assert scale == np.frombuffer(np.uint32(1).tobytes(), np.float32)[0]


def test_encoding_rejects_values_that_are_not_whole_groups():
    """tensor.rs:332-361 (the shape half: a T2 row of 64 is not a group of 128)."""
    with pytest.raises(ValueError):
        O.encode(O.T2B128, 1, 64, np.ones(64, np.float32))


@pytest.mark.parametrize("dtype", FORMATS)
def test_pack_then_unpack_is_identity_and_lanes_are_disjoint(dtype):
    rng = np.random.default_rng(dtype)
    bits = 8 // {O.Q7B32: 1, O.Q4B32: 2, O.T2B128: 4, O.Q8B32: 1}[dtype]
    hi = min(1 << bits, 128 if dtype == O.Q7B32 else 1 << bits)
    quad = np.zeros(128 // (8 // bits), np.uint8)
    codes = [rng.integers(0, hi, 32).astype(np.uint8) for _ in range(4)]
    for lane in range(4):
        O.pack_lane(dtype, lane, codes[lane], quad)
    for lane in range(4):
        assert np.array_equal(O.unpack_lane(dtype, quad, lane), codes[lane])


def test_quad_layout_positions_against_the_documented_rule():
    """quant.rs:10-15: Q7 chunk c of lane L at bytes 16c + 4L; Q4 chunk c < 4 low nibble, c + 4
    high nibble of the same byte."""
    quad = np.zeros(128, np.uint8)
    codes = np.arange(32, dtype=np.uint8) + 1
    O.pack_lane(O.Q7B32, 2, codes, quad)
    for i in range(32):
        c, o = divmod(i, 4)
        assert quad[16 * c + 4 * 2 + o] == codes[i]
    quad = np.zeros(64, np.uint8)
    codes = (np.arange(32) % 16).astype(np.uint8)
    O.pack_lane(O.Q4B32, 1, codes, quad)
    for i in range(32):
        c, o = divmod(i, 4)
        byte = quad[16 * (c % 4) + 4 * 1 + o]
        assert ((byte >> (4 * (c // 4))) & 0xF) == codes[i]


def test_weight_scales_follow_quad_group_lane_order():
    """tensor.rs:3-8: scale of (row n, group g) at ((n/4)·G + g)·4 + n%4."""
    rows, cols = 6, 64
    values = np.zeros((rows, cols), np.float32)
    for r in range(rows):
        for g in range(2):
            values[r, g * 32] = 63.0 * (r + 1) + g  # absmax of the block -> scale = absmax / 63
    table = O.encode(O.Q7B32, rows, cols, values)
    scales = table[O.quant_len(O.Q7B32, rows, cols):].view(np.float32)
    for r in range(rows):
        for g in range(2):
            want = np.float32(63.0 * (r + 1) + g) / np.float32(63.0)
            assert scales[((r // 4) * 2 + g) * 4 + r % 4] == want
    assert np.all(scales[((1 * 2 + 0) * 4 + 2):((1 * 2 + 0) * 4 + 4)] == 0.0)  # padding rows


# ------------------------------------------------------------- activation quantization

def test_activation_quantization_rounds_ties_to_even_and_saturates():
    x = np.zeros(32, np.float32)
    x[0] = 127.0  # d = 1
    x[1:6] = [2.5, 3.5, -2.5, 0.5, -0.5]
    q, s, c = O.quantize_rows(x, O.Q7B32)
    assert s[0] == 1.0
    assert list(q[:6]) == [127, 2, 4, -2, 0, 0]
    assert c[0] == -64 * int(q.astype(np.int64).sum())


def test_activation_quantization_closed_form_and_invariants():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(4 * 256) * 3).astype(np.float32)
    x[5] = 0.0
    x[64:96] = 0.0  # an all-zero block: d = 1, levels 0
    for dtype in FORMATS:
        q, s, c = O.quantize_rows(x, dtype)
        g = O.group(dtype)
        for i in range(x.size // g):
            xs = x[i * g:(i + 1) * g]
            amax = np.float32(np.max(np.abs(xs)))
            d = np.float32(1.0) if amax == 0 else amax / np.float32(127.0)
            assert s[i] == d
            qs = q[i * g:(i + 1) * g].astype(np.int64)
            assert np.all(np.abs(qs) <= 127)
            if amax != 0:
                assert np.max(np.abs(qs)) == 127
            # |x/d - q| <= 1/2 (nearest level) and the sign is kept
            assert np.all(np.abs(xs.astype(np.float64) / float(d) - qs) <= 0.5 + 1e-6)
            assert c[i] == -O.zero_point(dtype) * int(qs.sum())


def test_activation_quantization_keeps_subnormals():
    """No denormal flush: a subnormal group keeps its levels (IEEE division)."""
    x = np.zeros(32, np.float32)
    tiny = np.frombuffer(np.uint32(127 * 3).tobytes(), np.float32)[0]
    x[0] = tiny
    x[1] = np.frombuffer(np.uint32(3).tobytes(), np.float32)[0]
    q, s, _ = O.quantize_rows(x, O.Q7B32)
    assert s[0] == np.frombuffer(np.uint32(3).tobytes(), np.float32)[0]
    assert q[0] == 127 and q[1] == 1


# ------------------------------------------------------------------------ the product

def f64_reference(dtype, rows_w, cols, table, x, rows):
    """matmul.rs:782-807: dequantized weights times int8-round-tripped activations, in f64."""
    w = O.dequantize(dtype, rows_w, cols, table).astype(np.float64)
    g = O.group(dtype)
    out = np.zeros((rows, rows_w))
    for r in range(rows):
        xr = x[r * cols:(r + 1) * cols]
        qx = np.empty(cols)
        for k in range(0, cols, g):
            blk = xr[k:k + g]
            scale = np.max(np.abs(blk)) / np.float32(127.0)
            qx[k:k + g] = (np.rint(blk / scale) * scale).astype(np.float32)
        out[r] = w @ qx
    return out


@pytest.mark.parametrize("dtype", FORMATS)
def test_every_format_matches_the_dequantized_product(dtype):
    """matmul.rs:809-843: 25 outputs x 128 inputs, rows 1/3/8/11, error < 1e-4 (1 + |want|)."""
    outputs, width = 25, 128
    table = O.encode(dtype, outputs, width, pseudo_random(outputs * width, 1))
    for rows in (1, 3, 8, 11):
        x = pseudo_random(rows * width, 7 + rows)
        want = f64_reference(dtype, outputs, width, table, x, rows)
        q, s, c = O.quantize_rows(x, dtype)
        got = O.matmul(dtype, outputs, width, table, q, s, c, rows)[:, :outputs]
        assert np.all(np.abs(got - want) < 1e-4 * (1.0 + np.abs(want))), (dtype, rows)


@pytest.mark.parametrize("dtype", FORMATS)
def test_group_accumulators_are_exact_level_dot_products(dtype):
    """Brute force in int64: D[r, n, g] = corr + Σ u·q = Σ (u − zp)·q over the group."""
    rng = np.random.default_rng(11 + dtype)
    n_rows, cols, rows = 10, 256, 3
    table = O.encode(dtype, n_rows, cols, rng.standard_normal((n_rows, cols)).astype(np.float32))
    x = rng.standard_normal(rows * cols).astype(np.float32)
    q, s, c = O.quantize_rows(x, dtype)
    out, dots = O.matmul(dtype, n_rows, cols, table, q, s, c, rows, want_dots=True)
    w = O.dequantize(dtype, n_rows, cols, table)
    g = O.group(dtype)
    scales = table[O.quant_len(dtype, n_rows, cols):].view(np.float32)
    levels = np.zeros((n_rows, cols), np.int64)
    for n in range(n_rows):
        for gi in range(cols // g):
            ws = scales[((n // 4) * (cols // g) + gi) * 4 + n % 4]
            levels[n, gi * g:(gi + 1) * g] = np.rint(w[n, gi * g:(gi + 1) * g] / ws)
    qq = q.reshape(rows, cols).astype(np.int64)
    for r in range(rows):
        for n in range(n_rows):
            for gi in range(cols // g):
                want = int(np.dot(levels[n, gi * g:(gi + 1) * g], qq[r, gi * g:(gi + 1) * g]))
                assert dots[r, n, gi] == want


def test_f32_sum_is_sequential_over_groups_with_unfused_scaling():
    """Appendix-A order, from quantities the oracle does not compute: s = fl(s + fl(fl(D)·fl(ws·as)))
    in group order; a pairwise or fused sum differs on these inputs."""
    rng = np.random.default_rng(5)
    n_rows, cols, rows = 8, 32 * 40, 2
    table = O.encode(O.Q8B32, n_rows, cols, rng.standard_normal((n_rows, cols)).astype(np.float32))
    x = (rng.standard_normal(rows * cols) * np.exp(rng.standard_normal(rows * cols))).astype(np.float32)
    q, s, c = O.quantize_rows(x, O.Q8B32)
    out, dots = O.matmul(O.Q8B32, n_rows, cols, table, q, s, c, rows, want_dots=True)
    scales = table[O.quant_len(O.Q8B32, n_rows, cols):].view(np.float32)
    G = cols // 32
    mismatched_fma = 0
    for r in range(rows):
        for n in range(n_rows):
            acc = np.float32(0.0)
            fused = np.float32(0.0)
            for g in range(G):
                p = np.float32(scales[((n // 4) * G + g) * 4 + n % 4] * s[r * G + g])
                acc = np.float32(acc + np.float32(np.float32(dots[r, n, g]) * p))
                fused = np.float32(float(fused) + float(np.float32(dots[r, n, g])) * float(p))
            assert out[r, n] == acc
            mismatched_fma += int(fused != acc)
    assert mismatched_fma > 0


def round_f32(value):
    """The f32 nearest a rational (ties to even), by exact comparison of the neighbours."""
    from fractions import Fraction
    if value == 0:
        return np.float32(0.0)
    x = np.float32(float(value))
    best = None
    for c in (np.nextafter(x, np.float32(-np.inf)), x, np.nextafter(x, np.float32(np.inf))):
        key = (abs(Fraction(float(c)) - value), int(np.array(c, np.float32).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return np.float32(best[1])


@pytest.mark.parametrize("dtype", [O.Q8B32, O.Q4B32, O.T2B128])
def test_fused_scaling_rounds_once_per_group(dtype):
    """The NEON backend's scaling (arch/neon.rs:140-154), from exact rationals: per group in order,
    s = round(D·fl(ws·as) + s), one rounding of the exact multiply-add; the separately rounded
    scalar form differs on these inputs."""
    from fractions import Fraction
    rng = np.random.default_rng(17 + dtype)
    n_rows, cols, rows = 8, O.group(dtype) * 12, 2
    table = O.encode(dtype, n_rows, cols, rng.standard_normal((n_rows, cols)).astype(np.float32))
    x = (rng.standard_normal(rows * cols) * np.exp(rng.standard_normal(rows * cols))).astype(np.float32)
    q, s, c = O.quantize_rows(x, dtype)
    out, dots = O.matmul(dtype, n_rows, cols, table, q, s, c, rows, want_dots=True, fused=True)
    plain = O.matmul(dtype, n_rows, cols, table, q, s, c, rows)
    scales = table[O.quant_len(dtype, n_rows, cols):].view(np.float32)
    G = cols // O.group(dtype)
    for r in range(rows):
        for n in range(n_rows):
            acc = np.float32(0.0)
            for g in range(G):
                p = np.float32(scales[((n // 4) * G + g) * 4 + n % 4] * s[r * G + g])
                acc = round_f32(Fraction(int(dots[r, n, g])) * Fraction(float(p)) + Fraction(float(acc)))
            assert out[r, n] == acc, (r, n)
    assert np.any(out[:, :n_rows] != plain[:, :n_rows])


def test_bias_is_added_after_the_sum_and_columns_are_whole_quads():
    rng = np.random.default_rng(9)
    n_rows, cols = 10, 64
    table = O.encode(O.Q7B32, n_rows, cols, rng.standard_normal((n_rows, cols)).astype(np.float32))
    x = rng.standard_normal(cols).astype(np.float32)
    q, s, c = O.quantize_rows(x, O.Q7B32)
    bias = rng.standard_normal(12).astype(np.float32)
    plain = O.matmul(O.Q7B32, n_rows, cols, table, q, s, c, 1)
    biased = O.matmul(O.Q7B32, n_rows, cols, table, q, s, c, 1, bias=bias)
    assert np.array_equal(biased, (plain + bias).astype(np.float32))
    part = O.matmul(O.Q7B32, n_rows, cols, table, q, s, c, 1, col_begin=4, col_end=12)
    assert np.array_equal(part, plain[:, 4:12])
    assert np.all(plain[:, 10:] == 0.0)  # padding lanes: zero codes... times zero scales
    with pytest.raises(ValueError):
        O.matmul(O.Q7B32, n_rows, cols, table, q, s, c, 1, col_begin=2, col_end=8)


def test_threaded_split_equals_the_single_call():
    rng = np.random.default_rng(2)
    for n_rows, rows in ((96, 1), (48, 3), (16, 40)):
        cols = 128
        table = O.encode(O.Q4B32, n_rows, cols, rng.standard_normal((n_rows, cols)).astype(np.float32))
        x = rng.standard_normal(rows * cols).astype(np.float32)
        q, s, c = O.quantize_rows(x, O.Q4B32)
        one = O.matmul(O.Q4B32, n_rows, cols, table, q, s, c, rows)[:, :n_rows]
        for threads in (1, 3, 8):
            assert np.array_equal(O.matmul_threaded(O.Q4B32, n_rows, cols, table, q, s, c, rows,
                                                    threads=threads), one)


# --------------------------------------------------------------------------- f32 ops

def test_exp_and_silu_match_the_f64_reference():
    """ops.rs:352-357: exp within 4e-7 relative over [-20, 20] step 0.01."""
    for i in range(-2000, 2001, 7):
        x = i / 100.0
        want = math.exp(float(np.float32(x)))
        assert abs(float(O.exp(x)) - want) / want < 4e-7
        ws = float(np.float32(x)) / (1.0 + math.exp(-float(np.float32(x))))
        assert abs(float(O.silu(x)) - ws) <= 1e-6 * (1.0 + abs(ws))


def test_rms_norm_and_softmax_against_closed_forms():
    rng = np.random.default_rng(4)
    x = rng.standard_normal(896).astype(np.float32)
    w = rng.standard_normal(896).astype(np.float32)
    got = O.rms_norm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt(np.mean(x64 * x64) + 1e-6) * w
    assert np.max(np.abs(got - want)) < 1e-5 * (1 + np.max(np.abs(want)))
    assert np.array_equal(O.rms_norm(np.full(8, 2.0, np.float32), np.ones(8, np.float32), 0.0),
                          np.ones(8, np.float32))
    s = (rng.standard_normal(512) * 4).astype(np.float32)
    sm = O.softmax(s)
    e = np.exp(s.astype(np.float64) - s.max())
    assert np.max(np.abs(sm - e / e.sum())) < 1e-6
    assert abs(float(sm.astype(np.float64).sum()) - 1.0) < 1e-5


def _fold(values, start=0.0):
    """A left fold in f32 (numpy's float32 additions are IEEE single, one rounding each)."""
    acc = np.float32(start)
    for v in values:
        acc = np.float32(acc + np.float32(v))
    return acc


def test_rms_norm_sums_its_squares_from_the_first_in_index_order():
    """ops.rs:7-16 with dot_f32 (arch/scalar.rs:112-114): the squares added from index 0. One
    square of 2^24 first absorbs every later square of 1 (2^24 + 1 is a tie that rounds to even,
    back to 2^24), so the mean is exactly 4096, the inverse exactly 1/64 and the outputs x / 64;
    summed pairwise, reversed or in blocks the 4095 ones survive (mean 4097) and no output does."""
    n = 4096
    x = np.ones(n, np.float32)
    x[0] = 4096.0
    got = O.rms_norm(x, np.ones(n, np.float32), 0.0)
    want = np.full(n, 1.0 / 64.0, np.float32)
    want[0] = 64.0
    assert np.array_equal(got, want)
    assert _fold(x[::-1] * x[::-1]) != np.float32(2.0 ** 24)  # a reversed sum keeps the ones


def test_rms_norm_scales_the_normalized_value_by_the_weight_last():
    """ops.rs:12: output = (value · inverse) · scale. For these one-value rows (mean = v², eps 0,
    inverse = fl(1/v)) the other association, value · (inverse · scale), rounds differently."""
    cases = 0
    for v in range(3, 40):
        inv = np.float32(np.float32(1.0) / np.float32(np.sqrt(np.float32(v * v))))
        for w in range(3, 40):
            left = np.float32(np.float32(np.float32(v) * inv) * np.float32(w))
            right = np.float32(np.float32(v) * np.float32(inv * np.float32(w)))
            if left == right:
                continue
            got = O.rms_norm(np.array([v], np.float32), np.array([w], np.float32), 0.0)
            assert got[0] == left and got[0] != right, (v, w)
            cases += 1
    assert cases > 20


def test_softmax_totals_every_exponential_in_index_order():
    """ops.rs:302-307: the total is a plain fold over the exponentials (not the sweep's offset
    sums). Score 0 first (exponential exactly 1), then 511 scores of -18, each exponential under
    half an ulp of 1: a fold from index 0 absorbs them all, so the total is exactly 1, the first
    weight exactly 1 and every other weight its exponential unchanged; the eight offset sums of
    Exponentials::apply, a pairwise sum or a reversed one each total about 1 + 7e-6."""
    s = np.full(512, -18.0, np.float32)
    s[0] = 0.0
    w = O.softmax(s)
    tiny = O.exp(np.float32(-18.0))
    assert float(tiny) * 2 < 2.0 ** -24  # under half an ulp of 1
    assert w[0] == np.float32(1.0)
    assert np.all(w[1:] == tiny)
    assert _fold(np.exp(s.astype(np.float32))[::-1]) > np.float32(1.0)  # reversed: not absorbed


def test_weighted_values_add_one_key_at_a_time_in_key_order():
    """ops::weigh (ops.rs:329-342) with the scalar axpy_f32_many (arch/mod.rs:141-147): each
    output adds w_j·v_j from +0 one key at a time. The weights of the scores above (1, then 511
    under half an ulp of 1) on rows of ones: in key order the first term is 1 and absorbs every
    later one, so each output is exactly 1; the terms of a block of DOTS keys summed first, or
    the keys taken last to first, carry them (about 1 + 7e-6). A dropped first key gives about
    8e-6, a key's weight applied to the next key's row leaves the row's own bits wrong."""
    n, dim = 512, 6
    s = np.full(n, -18.0, np.float32)
    s[0] = 0.0
    values = np.ones((n, dim), np.float32)
    w, out = O.weigh(s, values)
    assert w[0] == np.float32(1.0) and np.array_equal(w[1:], np.full(n - 1, O.exp(np.float32(-18.0))))
    assert np.array_equal(out, np.ones(dim, np.float32))
    blocked = _fold([_fold(w[b:b + 4]) for b in range(0, n, 4)])
    assert blocked > np.float32(1.0) and _fold(w[::-1]) > np.float32(1.0)
    # distinct rows: output i is the key-order fold of w_j·v_j[i]
    rng = np.random.default_rng(8)
    s = (rng.standard_normal(37) * 3).astype(np.float32)
    values = rng.standard_normal((37, dim)).astype(np.float32)
    w, out = O.weigh(s, values)
    for i in range(dim):
        assert out[i] == _fold([np.float32(w[j] * values[j, i]) for j in range(37)])


@pytest.mark.parametrize("fast", [False, True])
@pytest.mark.parametrize("tail", [0, 3])
def test_exponentials_sum_the_tail_then_the_eight_offset_sums(fast, tail):
    """Exponentials::apply (ops.rs:168-174) with the scalar sweep (arch/scalar.rs:117-125): sums
    per offset in a run of EXP_RUN = 8 over the whole runs (each from +0 in run order), then a
    fold from -0 of the values past the last whole run followed by the eight sums. With the one
    exponential of 1 at offset 0 and the others under half an ulp of 1, offset 0's sum stays 1
    while offsets 1..7 keep their 64 small terms, so the total exceeds 1 by their seven sums; a
    plain fold from index 0 would absorb every small term and total exactly 1."""
    n = 8 * 64 + tail
    s = np.full(n, -18.0, np.float32)
    s[0] = 0.0
    v, total = O.exponentials_apply(s, fast)
    t = v[1]
    assert np.all(v[1:] == t) and v[0] == np.float32(1.0)
    sums = [_fold(v[k:8 * 64:8]) for k in range(8)]
    assert sums[0] == np.float32(1.0) and sums[1] == _fold([t] * 64)
    want = _fold(list(v[8 * 64:]) + sums, start=-0.0)
    assert total == want
    assert total > np.float32(1.0) and _fold(v) == np.float32(1.0)


def test_rotary_angles_against_f64():
    """rotary.rs tests' 1e-6 bound; frequencies base^(-2i/d)."""
    cos, sin = O.rope_tables(1e6, 64, 600)
    for p in (0, 1, 17, 511, 599):
        for i in range(32):
            f = np.float32(1.0) / np.float32(np.float32(1e6) ** np.float32(2 * i / 64))
            ang = float(np.float32(p) * f)
            assert abs(cos[p, i] - math.cos(ang)) < 1e-6
            assert abs(sin[p, i] - math.sin(ang)) < 1e-6
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)


# ------------------------------------------------------------------------------- rng

def _splitmix_first(seed):
    z = (seed + 0x9E3779B97F4A7C15) & (2**64 - 1)
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & (2**64 - 1)
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & (2**64 - 1)
    return z ^ (z >> 31)


def test_rng_is_splitmix_seeded_xoshiro256starstar():
    """SplitMix64's published first output for seed 0 is 0xE220A8397B1DCDAF; xoshiro256**'s output
    is rotl(s1·5, 7)·9 (Blackman and Vigna)."""
    assert _splitmix_first(0) == 0xE220A8397B1DCDAF
    mask = 2**64 - 1
    state, m = [], 0
    for _ in range(4):
        m = (m + 0x9E3779B97F4A7C15) & mask
        z = m
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
        state.append(z ^ (z >> 31))
    s = state
    rotl = lambda x, k: ((x << k) | (x >> (64 - k))) & mask
    r = O.Rng(0)
    for _ in range(5):
        want = (rotl((s[1] * 5) & mask, 7) * 9) & mask
        t = (s[1] << 17) & mask
        s[2] ^= s[0]; s[3] ^= s[1]; s[1] ^= s[2]; s[0] ^= s[3]; s[2] ^= t; s[3] = rotl(s[3], 45)
        assert r.next_u64() == want
    v = O.Rng(1).normal(20000)
    assert abs(float(v.mean())) < 0.03 and abs(float(v.std()) - 1.0) < 0.03


# ----------------------------------------------------------------- the decoder step

def small_qwen2(dtype, seed=0, layers=2, hidden=64, heads=4, kv_heads=2, head_dim=16, ffn=128,
                vocab=64, capacity=16):
    rng = np.random.default_rng(seed)
    sh = O.Qwen2Shape(hidden=hidden, layers=layers, heads=heads, kv_heads=kv_heads, head_dim=head_dim,
                      ffn=ffn, vocab=vocab, capacity=capacity, rope_base=10000.0, eps=1e-6, dtype=dtype)
    qkv_w = (heads + 2 * kv_heads) * head_dim
    mats, lys = [], []
    for _ in range(layers):
        f = {}
        for name, (r, c) in {"qkv": (qkv_w, hidden), "o": (hidden, heads * head_dim), "gate": (ffn, hidden),
                             "up": (ffn, hidden), "down": (hidden, ffn)}.items():
            w = (rng.standard_normal((r, c)) / math.sqrt(c)).astype(np.float32)
            f[name] = O.encode(dtype, r, c, w)
        f["norm1"] = (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
        f["norm2"] = (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
        f["qkv_bias"] = (0.1 * rng.standard_normal(qkv_w)).astype(np.float32)
        lys.append(f)
    final = (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
    table = O.encode(dtype, vocab, hidden, rng.standard_normal((vocab, hidden)).astype(np.float32))
    return sh, lys, final, table


def f64_qwen2_step(sh, lys, final, table, kc, vc, token, pos):
    """An independent f64 Qwen2 decode step over dequantized weights (the shape of
    blocks/tests/support/mod.rs), activations unquantized."""
    dt, H, D = sh.dtype, sh.hidden, sh.head_dim
    deq = lambda b, r, c: O.dequantize(dt, r, c, b).astype(np.float64)
    rms = lambda x, w: x / np.sqrt(np.mean(x * x) + sh.eps) * w
    h = deq(table, sh.vocab, H)[token].copy()
    inv = 1.0 / (sh.rope_base ** (np.arange(0, D, 2) / D))
    ang = pos * inv
    kc = kc.astype(np.float64).copy()
    vc = vc.astype(np.float64).copy()
    qkv_w = (sh.heads + 2 * sh.kv_heads) * D
    for li, f in enumerate(lys):
        x = rms(h, f["norm1"])
        qkv = deq(f["qkv"], qkv_w, H) @ x + f["qkv_bias"]
        heads = qkv.reshape(-1, D)
        for u in range(sh.heads + sh.kv_heads):
            a, b = heads[u, :D // 2].copy(), heads[u, D // 2:].copy()
            heads[u, :D // 2] = a * np.cos(ang) - b * np.sin(ang)
            heads[u, D // 2:] = b * np.cos(ang) + a * np.sin(ang)
        for k in range(sh.kv_heads):
            kc[li, k, pos] = heads[sh.heads + k]
            vc[li, k, pos] = heads[sh.heads + sh.kv_heads + k]
        att = np.zeros(sh.heads * D)
        for hh in range(sh.heads):
            kv = hh // (sh.heads // sh.kv_heads)
            sc = kc[li, kv, :pos + 1] @ heads[hh] / math.sqrt(D)
            e = np.exp(sc - sc.max())
            att[hh * D:(hh + 1) * D] = (e / e.sum()) @ vc[li, kv, :pos + 1]
        h = h + deq(f["o"], H, sh.heads * D) @ att
        x = rms(h, f["norm2"])
        g = deq(f["gate"], sh.ffn, H) @ x
        u = deq(f["up"], sh.ffn, H) @ x
        h = h + deq(f["down"], H, sh.ffn) @ (g / (1 + np.exp(-g)) * u)
    logits = deq(table, sh.vocab, H) @ rms(h, final)
    return h, logits


def rel_l2(got, want):
    """blocks/tests/support/mod.rs:559-568"""
    return float(np.sqrt(np.sum((got.astype(np.float64) - want) ** 2) / np.sum(want * want)))


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q4B32, O.Q8B32])
def test_qwen2_step_matches_an_f64_reference(dtype):
    """blocks/tests/stacks.rs:51-56: 7-bit weights within 3e-2 (rel-L2) of an f64 reference."""
    sh, lys, final, table = small_qwen2(dtype)
    rng = np.random.default_rng(1)
    pos = 9
    kc = rng.standard_normal((2, 2, 16, 16)).astype(np.float32)
    vc = rng.standard_normal((2, 2, 16, 16)).astype(np.float32)
    model = O.Qwen2(sh, lys, final, table)
    k2, v2 = kc.copy(), vc.copy()
    hidden, logits, tok = model.step(k2, v2, 5, pos)
    want_h, want_l = f64_qwen2_step(sh, lys, final, table, kc, vc, 5, pos)
    tol = 3e-2 if dtype != O.Q4B32 else 1.5e-1
    assert rel_l2(hidden, want_h) < tol
    assert rel_l2(logits, want_l) < tol
    assert tok == int(np.argmax(logits))
    # the step kept this position's keys and values and nothing else
    assert np.array_equal(np.delete(k2, pos, axis=2), np.delete(kc, pos, axis=2))
    assert not np.array_equal(k2[:, :, pos], kc[:, :, pos])
    # threads change nothing
    k3, v3 = kc.copy(), vc.copy()
    h3, l3, _ = model.step(k3, v3, 5, pos, threads=3)
    assert np.array_equal(h3, hidden) and np.array_equal(l3, logits)


def test_greedy_takes_the_first_of_equals():
    l = np.array([1.0, 3.0, 2.0, 3.0], np.float32)
    assert O.lib().or_greedy(l.ctypes.data_as(O.ctypes.c_void_p), 4) == 1
