"""GPU parity of the product path against the CPU oracle: bit-exact bytes, levels, scales,
corrections, int32 group accumulators and f32 outputs, through the C ABI."""

import numpy as np
import pytest

from oracle import oracle as O
from gpu_data import activations, encoded_table, synthetic_table

pytestmark = pytest.mark.gpu

PRODUCT_FORMATS = [O.Q7B32, O.Q8B32, O.Q4B32, O.T2B128]
ALL_FORMATS = [O.Q7B32, O.Q8B32, O.Q4B32, O.T2B128]


@pytest.fixture(scope="module")
def fk(gpu):
    import fusor_kernels
    return fusor_kernels


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def table(fk, dtype, rows, cols, data):
    return fk.Table(fk.Tensor(dtype, [rows, cols], data))


def same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def first_mismatch(a, b):
    a = np.asarray(a, np.float32).reshape(-1)
    b = np.asarray(b, np.float32).reshape(-1)
    bad = np.nonzero(a.view(np.uint32) != b.view(np.uint32))[0]
    return (int(bad[0]), float(a[bad[0]]), float(b[bad[0]]), len(bad)) if len(bad) else None


# ------------------------------------------------------------------------------- tables

@pytest.mark.parametrize("dtype", ALL_FORMATS)
@pytest.mark.parametrize("rows,cols", [(4, 128), (25, 128), (7, 256), (130, 512)])
def test_table_upload_keeps_the_reference_bytes(fk, dtype, rows, cols):
    data = encoded_table(dtype, rows, cols, seed=rows * 7 + dtype)
    t = table(fk, dtype, rows, cols, data)
    assert np.array_equal(t.reference_bytes(), data)


@pytest.mark.parametrize("dtype", ALL_FORMATS)
def test_encode_matches_the_oracle(fk, dtype):
    rng = np.random.default_rng(dtype)
    rows, cols = 9, 256
    values = rng.standard_normal((rows, cols)).astype(np.float32) * 3
    values[0, :32] = 0.0                                   # an all-zero group
    values[1, 5] = np.float32(np.frombuffer(np.uint32(94).tobytes(), np.float32)[0])  # subnormal
    values[1, 32:64] = 0.0
    values[1, 40] = np.frombuffer(np.uint32(94).tobytes(), np.float32)[0]
    values[2, 70] = np.nan
    values[3, 3] = np.inf
    values[4, 130] = -np.inf
    values[5, :128] = np.repeat(np.float32([0.5, -0.5]), 64)  # ties
    got = fk.Tensor.encode(fk.DType(dtype), [rows, cols], values).bytes()
    want = O.encode(dtype, rows, cols, values)
    assert np.array_equal(got, want)


def test_q4_encode_keeps_the_signed_extreme(fk):
    """Q4b32's scale is the first value of largest magnitude over -8 (quant.rs:151-166), sign
    included: known answers worked from that rule, where |extreme| or the last extreme would give
    other codes and scales."""
    rows, cols = 4, 32
    values = np.zeros((rows, cols), np.float32)
    values[0, :4] = [0.5, 8.0, -2.0, 0.0]  # positive extreme: d = -1, 8 -> 0, -2 -> 10, 0.5 -> 8 (-0.5 to even)
    values[1, :2] = [-8.0, 8.0]            # the first of equal magnitudes: d = 1, -8 -> 0, 8 -> 16 clamped to 15
    values[2, :2] = [8.0, -8.0]            # the other way round: d = -1, 8 -> 0, -8 -> 15
    values[3, :3] = [-1.0, 4.0, -3.0]      # d = -0.5: -1 -> 10, 4 -> 0, -3 -> 14
    got = fk.Tensor.encode(fk.DType.Q4b32, [rows, cols], values).bytes()
    assert np.array_equal(got, O.encode(O.Q4B32, rows, cols, values))
    scales = np.ascontiguousarray(got[rows * cols // 2:]).view(np.float32)
    assert scales.tolist() == [-1.0, 1.0, -1.0, -0.5]
    codes = [O.unpack_lane(O.Q4B32, got[:64], lane) for lane in range(4)]
    assert codes[0][:4].tolist() == [8, 0, 10, 8] and codes[0][4:].tolist() == [8] * 28
    assert codes[1][:2].tolist() == [0, 15]
    assert codes[2][:2].tolist() == [0, 15]
    assert codes[3][:3].tolist() == [10, 0, 14]


def test_encode_rejects_partial_groups(fk):
    with pytest.raises(fk.FormatError, match=r"a T2b128 tensor of shape \[1, 64\]: a matrix of whole groups of 128 expected"):
        fk.Tensor.encode(fk.DType.T2b128, [1, 64], np.ones(64, np.float32))
    with pytest.raises(fk.FormatError, match=r"63 values for a tensor of shape \[2, 32\]"):
        fk.Tensor.encode(fk.DType.Q7b32, [2, 32], np.ones(63, np.float32))


@pytest.mark.parametrize("dtype", ALL_FORMATS)
def test_dequantize_row_matches_the_oracle(fk, dtype):
    import torch
    rows, cols = 11, 256
    data = encoded_table(dtype, rows, cols, seed=3 + dtype)
    t = table(fk, dtype, rows, cols, data)
    out = torch.empty(cols, dtype=torch.float32, device="cuda")
    for r in range(rows):
        t.matrix().dequantize_row(r, out)
        assert same_bits(host(out), O.dequantize_row(dtype, rows, cols, data, r)), r
    with pytest.raises(fk.ShapeError):
        t.matrix().dequantize_row(rows, out)


# ----------------------------------------------------------------- activation quantization

@pytest.mark.parametrize("dtype", ALL_FORMATS)
@pytest.mark.parametrize("count", [128, 896, 4864 * 3, 4096 * 16])
def test_quantize_rows_matches_the_oracle(fk, dtype, count):
    import torch
    x = activations(1, count, seed=count + dtype, outliers=0.01).reshape(-1)
    x[:32] = 0.0
    x[40] = np.frombuffer(np.uint32(381).tobytes(), np.float32)[0]
    x[count // 2 + 3] = np.nan
    if count > 1000:
        x[900] = np.inf
    g = O.group(dtype)
    q = torch.empty(count, dtype=torch.int8, device="cuda")
    s = torch.empty(count // g, dtype=torch.float32, device="cuda")
    c = torch.empty(count // g, dtype=torch.int32, device="cuda")
    import fusor_kernels as fk2
    fk2.quantize_rows(dev(x), fk2.QuantFormat(dtype), q, s, c)
    wq, ws, wc = O.quantize_rows(x, dtype)
    assert np.array_equal(host(q), wq)
    assert same_bits(host(s), ws)
    assert np.array_equal(host(c), wc)


def near_ties(groups, seed):
    """Groups whose largest magnitude spans every binade (subnormal to near the largest float) and
    whose other values sit at and within a few ulps of the half-integer multiples of the group's
    scale d = amax / 127, where the rounding of the quotient decides the level."""
    rng = np.random.default_rng(seed)
    exps = rng.integers(-149, 128, groups)
    amax = (rng.uniform(1.0, 2.0, groups) * np.exp2(exps.astype(np.float64))).astype(np.float32)
    amax[amax == 0] = np.float32(1e-45)
    amax[~np.isfinite(amax)] = np.float32(3e38)
    d = amax / np.float32(127.0)
    k = rng.integers(-127, 127, (groups, 32)).astype(np.float32)
    x = ((k + np.float32(0.5)) * d[:, None]).astype(np.float32)
    nudge = rng.integers(-3, 4, (groups, 32)).astype(np.int32)
    mag = np.maximum(np.abs(x).view(np.int32) + nudge, 0).view(np.float32)
    x = np.where(x < 0, -mag, mag).astype(np.float32)
    x = np.clip(x, -amax[:, None], amax[:, None])
    x[:, 0] = amax * np.where(rng.random(groups) < 0.5, 1, -1).astype(np.float32)
    return x.reshape(-1)


@pytest.mark.parametrize("dtype", [O.Q8B32, O.T2B128])
def test_quantize_rows_rounds_quotients_at_every_scale(fk, dtype):
    """Every level is the tie-to-even rounding of the IEEE quotient x / d, for scales from
    subnormal to huge: the shared-reciprocal quotient and the division agree to the bit."""
    import torch
    x = near_ties(8192, seed=dtype)
    count = x.size
    g = O.group(dtype)
    q = torch.empty(count, dtype=torch.int8, device="cuda")
    s = torch.empty(count // g, dtype=torch.float32, device="cuda")
    c = torch.empty(count // g, dtype=torch.int32, device="cuda")
    fk.quantize_rows(dev(x), fk.QuantFormat(dtype), q, s, c)
    wq, ws, wc = O.quantize_rows(x, dtype)
    got = host(q)
    assert np.array_equal(got, wq), np.flatnonzero(got != wq)[:8]
    assert same_bits(host(s), ws)
    assert np.array_equal(host(c), wc)


# ------------------------------------------------------------------------------ products

def gpu_product(fk, t, x, rows, cols=None, fused=True, bias=None, dots=False, fused_scale=False):
    import torch
    m = t.matrix()
    if cols is None:
        cols = range(0, (t.rows + 3) // 4 * 4)
    if fused:
        inp = fk.Input(f32=dev(x.reshape(-1)))
    else:
        inp = fk.QuantizedRows().input(m, dev(x.reshape(-1)))
    if dots:
        return host(fk.matmul_dots(m, inp, cols))
    out = fk.matmul(m, inp, cols, bias=None if bias is None else dev(bias), fused=fused_scale)
    return host(out)


def oracle_product(dtype, rows_w, cols_w, data, x, rows, col_begin=0, col_end=None, bias=None, want_dots=False,
                   fused=False):
    q, s, c = O.quantize_rows(x.reshape(-1), dtype)
    return O.matmul(dtype, rows_w, cols_w, data, q, s, c, rows, col_begin, col_end, bias=bias, want_dots=want_dots,
                    fused=fused)


@pytest.mark.parametrize("dtype", PRODUCT_FORMATS)
@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5, 8, 16, 33, 64, 100])
def test_product_is_bit_exact(fk, dtype, rows):
    n_rows, cols = 37, 256
    data = synthetic_table(dtype, n_rows, cols, seed=rows)
    t = table(fk, dtype, n_rows, cols, data)
    x = activations(rows, cols, seed=100 + rows, outliers=0.02)
    want, want_dots = oracle_product(dtype, n_rows, cols, data, x, rows, want_dots=True)
    got = gpu_product(fk, t, x, rows)
    assert same_bits(got, want), first_mismatch(got, want)
    got_dots = gpu_product(fk, t, x, rows, dots=True)
    assert np.array_equal(got_dots, want_dots)


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q8B32, O.Q4B32])
@pytest.mark.parametrize("rows", [1, 2, 4])
@pytest.mark.parametrize("cols", [32, 96, 160, 1184])
def test_matvec_with_group_counts_not_a_multiple_of_four(fk, dtype, rows, cols):
    """1, 3, 5 and 37 groups per row: the matrix-vector kernel's rows of group terms are padded
    to whole float4s, and the group-order sum must stop at the last real group."""
    n_rows = 37
    data = synthetic_table(dtype, n_rows, cols, seed=cols + rows)
    t = table(fk, dtype, n_rows, cols, data)
    x = activations(rows, cols, seed=3 * cols + rows, outliers=0.02)
    bias = np.random.default_rng(cols).standard_normal(n_rows).astype(np.float32)
    want = oracle_product(dtype, n_rows, cols, data, x, rows, bias=bias)
    got = gpu_product(fk, t, x, rows, bias=bias)
    assert same_bits(got, want), first_mismatch(got, want)
    got_pre = gpu_product(fk, t, x, rows, bias=bias, fused=False)
    assert same_bits(got_pre, want), first_mismatch(got_pre, want)


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q8B32, O.Q4B32])
@pytest.mark.parametrize("cols", [32, 160])
def test_wide_tiles_with_ragged_edges_and_short_rings(fk, dtype, cols):
    """100 rows x 16386 outputs: more than 1024 tiles of 32 x 64, so the product takes the wide
    tiles in their per-XCD order, with a partial last row tile, a partial last column tile and a
    padding row; 1 and 5 blocks per row, fewer than and not a multiple of the four-block ring."""
    rows, n_rows = 100, 16386
    data = synthetic_table(dtype, n_rows, cols, seed=cols)
    t = table(fk, dtype, n_rows, cols, data)
    x = activations(rows, cols, seed=7 + cols, outliers=0.02)
    want, want_dots = oracle_product(dtype, n_rows, cols, data, x, rows, want_dots=True)
    got = gpu_product(fk, t, x, rows)
    assert same_bits(got, want), first_mismatch(got, want)
    assert np.array_equal(gpu_product(fk, t, x, rows, dots=True), want_dots)
    want_f = oracle_product(dtype, n_rows, cols, data, x, rows, fused=True)
    got_f = gpu_product(fk, t, x, rows, fused_scale=True)
    assert same_bits(got_f, want_f), first_mismatch(got_f, want_f)


@pytest.mark.parametrize("dtype", PRODUCT_FORMATS)
@pytest.mark.parametrize("rows", [1, 4, 5, 16, 33, 100])
def test_fused_scale_is_the_neon_backends_bits(fk, dtype, rows):
    """FG_FUSED_SCALE: each group's total scaled with one fused multiply-add in group order (the
    NEON backend, arch/neon.rs:140-154), bit-exact against the oracle's fused product, bias
    included; it differs from the scalar backend's bits somewhere."""
    n_rows, cols = 70, 512
    data = synthetic_table(dtype, n_rows, cols, seed=40 + rows)
    t = table(fk, dtype, n_rows, cols, data)
    x = activations(rows, cols, seed=41 + rows, outliers=0.02)
    bias = np.random.default_rng(rows).standard_normal(n_rows).astype(np.float32)
    want = oracle_product(dtype, n_rows, cols, data, x, rows, bias=bias, fused=True)
    got = gpu_product(fk, t, x, rows, bias=bias, fused_scale=True)
    assert same_bits(got, want), first_mismatch(got, want)
    got_pre = gpu_product(fk, t, x, rows, bias=bias, fused=False, fused_scale=True)
    assert same_bits(got_pre, want)
    plain = oracle_product(dtype, n_rows, cols, data, x, rows, bias=bias)
    assert not same_bits(plain, want)


@pytest.mark.parametrize("dtype", PRODUCT_FORMATS)
@pytest.mark.parametrize("rows", [1, 3, 17])
def test_prequantized_input_equals_in_kernel_quantization(fk, dtype, rows):
    n_rows, cols = 64, 512
    data = synthetic_table(dtype, n_rows, cols, seed=5)
    t = table(fk, dtype, n_rows, cols, data)
    x = activations(rows, cols, seed=6)
    assert same_bits(gpu_product(fk, t, x, rows, fused=True), gpu_product(fk, t, x, rows, fused=False))


@pytest.mark.parametrize("dtype", PRODUCT_FORMATS)
@pytest.mark.parametrize("rows", [1, 6, 40])
def test_column_ranges_bias_and_residual(fk, dtype, rows):
    import torch
    n_rows, cols = 50, 128
    data = synthetic_table(dtype, n_rows, cols, seed=9)
    t = table(fk, dtype, n_rows, cols, data)
    x = activations(rows, cols, seed=10)
    bias = np.random.default_rng(1).standard_normal(n_rows).astype(np.float32)
    want = oracle_product(dtype, n_rows, cols, data, x, rows, 8, 40, bias=bias)
    got = gpu_product(fk, t, x, rows, cols=range(8, 40), bias=bias)
    assert same_bits(got, want)
    # the padding quad past row 50: zero codes and scales, no bias (linear.rs:63-68)
    tail = gpu_product(fk, t, x, rows, cols=range(48, 52), bias=bias)
    wtail = oracle_product(dtype, n_rows, cols, data, x, rows, 48, 52, bias=bias)
    assert same_bits(tail, wtail)
    # project_residual_input: h = fl(h + y) (linear.rs:134-143)
    h0 = np.random.default_rng(2).standard_normal((rows, n_rows)).astype(np.float32)
    h = dev(h0)
    lin = fk.Linear(t, None)
    inp = fk.QuantizedRows().input(t.matrix(), dev(x.reshape(-1)))
    fk.project_residual_input(fk.Ctx(0, 1), lin, inp, h)
    full = oracle_product(dtype, n_rows, cols, data, x, rows)[:, :n_rows]
    upto = n_rows // 16 * 16
    want_h = h0.copy()
    want_h[:, :upto] = (h0[:, :upto] + full[:, :upto]).astype(np.float32)
    assert same_bits(host(h), want_h)
    with pytest.raises(fk.ShapeError, match="columns in whole quads"):
        gpu_product(fk, t, x, rows, cols=range(2, 8))
    with pytest.raises(fk.ShapeError, match="weights cover the columns"):
        gpu_product(fk, t, x, rows, cols=range(0, 56))


def pseudo_random(n, seed):
    """matmul.rs:772-780"""
    state = seed & 0xFFFFFFFF
    out = np.empty(n, np.float32)
    for i in range(n):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32(state >> 8) / np.float32(1 << 24) * np.float32(2.0) - np.float32(1.0)
    return out


@pytest.mark.parametrize("dtype", PRODUCT_FORMATS)
def test_every_format_matches_the_dequantized_product(fk, dtype):
    """matmul.rs:809-843 through the GPU: 25 x 128, rows 1/3/8/11; bit-exact against the oracle
    and within the reference's own f64 tolerance."""
    outputs, width = 25, 128
    data = O.encode(dtype, outputs, width, pseudo_random(outputs * width, 1))
    t = table(fk, dtype, outputs, width, data)
    w = O.dequantize(dtype, outputs, width, data).astype(np.float64)
    for rows in (1, 3, 8, 11):
        x = pseudo_random(rows * width, 7 + rows).reshape(rows, width)
        got = gpu_product(fk, t, x, rows)
        assert same_bits(got, oracle_product(dtype, outputs, width, data, x, rows))
        g = O.group(dtype)
        for r in range(rows):
            qx = np.empty(width)
            for k in range(0, width, g):
                blk = x[r, k:k + g]
                sc = np.max(np.abs(blk)) / np.float32(127.0)
                qx[k:k + g] = (np.rint(blk / sc) * sc).astype(np.float32)
            want = w @ qx
            assert np.all(np.abs(got[r, :outputs] - want) < 1e-4 * (1 + np.abs(want)))


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q8B32])
def test_single_matvec_shape_bit_exact(fk, dtype):
    """4864 x 896, one row ~N(0,1), seed 0: every output and accumulator bit-exact."""
    rows_w, cols = 4864, 896
    data = synthetic_table(dtype, rows_w, cols, seed=0)
    t = table(fk, dtype, rows_w, cols, data)
    x = activations(1, cols, seed=0)
    want, want_dots = oracle_product(dtype, rows_w, cols, data, x, 1, want_dots=True)
    assert same_bits(gpu_product(fk, t, x, 1), want)
    assert same_bits(gpu_product(fk, t, x, 1, fused=False), want)
    assert np.array_equal(gpu_product(fk, t, x, 1, dots=True), want_dots)


@pytest.mark.parametrize("shape", [(512, 896, 9728), (512, 4864, 896), (4096, 1152, 3456), (4096, 1152, 4608),
                                   (4096, 4608, 1152)])
def test_batched_shapes_bit_exact_in_full(fk, shape):
    """The full-size GEMMs (512-row prefill and the 4096-row DiT block's QKV, MLP up and MLP down),
    every output of every row against the oracle's threaded product: every row tile and column tile
    of the per-XCD tile order."""
    rows, k, n = shape
    print(f"batched {rows}x{k}->{n}", flush=True)
    data = synthetic_table(O.Q8B32, n, k, seed=rows + k + n)
    t = table(fk, O.Q8B32, n, k, data)
    x = (activations(rows, k, seed=k + n, outliers=0.01) * np.float32(np.sqrt(2.0))).astype(np.float32)
    got = gpu_product(fk, t, x, rows)
    q, s, c = O.quantize_rows(x.reshape(-1), O.Q8B32)
    want = O.matmul_threaded(O.Q8B32, n, k, data, q, s, c, rows, threads=16)
    assert same_bits(got, want), first_mismatch(got, want)


@pytest.mark.parametrize("rows", [1, 16])
def test_int4_shape_bit_exact(fk, rows):
    n, k = 14336, 4096
    data = synthetic_table(O.Q4B32, n, k, seed=4)
    t = table(fk, O.Q4B32, n, k, data)
    x = activations(rows, k, seed=44)
    got = gpu_product(fk, t, x, rows)
    q, s, c = O.quantize_rows(x.reshape(-1), O.Q4B32)
    want = O.matmul_threaded(O.Q4B32, n, k, data, q, s, c, rows, threads=16)
    assert same_bits(got, want), first_mismatch(got, want)


@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("n_rows,cols", [(70, 384), (37, 1152), (18, 5120), (9, 128), (5, 16384)])
def test_t2_streamed_chunks_rings_and_row_slices(fk, rows, n_rows, cols):
    """T2b128 products of up to 8 rows over few columns, on the streamed kernel (slices of 1, 2 or 4
    rows); 3 groups (one partial 1 KiB chunk), 9 groups (a
    second chunk of one group), 40 groups (five chunks: the four-chunk ring refilled), one group,
    and 128 groups (16384 levels a row: slices of two rows, not four, to fit the workgroup's LDS);
    70 outputs (a last workgroup of two quads); bias and the fused scaling."""
    print(f"t2 {rows} x {cols} -> {n_rows}", flush=True)
    dtype = O.T2B128
    data = synthetic_table(dtype, n_rows, cols, seed=n_rows + cols + rows)
    t = table(fk, dtype, n_rows, cols, data)
    x = activations(rows, cols, seed=cols + 3 * rows, outliers=0.02)
    bias = np.random.default_rng(rows).standard_normal(n_rows).astype(np.float32)
    want = oracle_product(dtype, n_rows, cols, data, x, rows, bias=bias)
    got = gpu_product(fk, t, x, rows, bias=bias)
    assert same_bits(got, want), first_mismatch(got, want)
    got_pre = gpu_product(fk, t, x, rows, bias=bias, fused=False)
    assert same_bits(got_pre, want), first_mismatch(got_pre, want)
    want_f = oracle_product(dtype, n_rows, cols, data, x, rows, fused=True)
    got_f = gpu_product(fk, t, x, rows, fused_scale=True)
    assert same_bits(got_f, want_f), first_mismatch(got_f, want_f)
    lo, hi = 4 * (n_rows // 12), 4 * ((n_rows + 3) // 4)
    want_r = oracle_product(dtype, n_rows, cols, data, x, rows, lo, hi)
    got_r = gpu_product(fk, t, x, rows, cols=range(lo, hi))
    assert same_bits(got_r, want_r), first_mismatch(got_r, want_r)


@pytest.mark.parametrize("rows", [9, 16, 31, 33, 100])
@pytest.mark.parametrize("n_rows,cols", [(70, 384), (37, 1152), (18, 5120), (9, 128)])
def test_t2_on_the_matrix_cores(fk, rows, n_rows, cols):
    """T2b128 products of 9 or more rows (the int8 matrix cores, a group's four blocks chained in
    one accumulator; 16 x 16 tiles up to 16 rows, 32 x 32 or 32 x 64 past them): 3, 9, 40 and 1 groups (odd counts against the two-group ring), partial row
    tiles (9, 31, 33, 100 rows) and column tiles (70 outputs), bias, the fused scaling, a column
    range, pre-quantized rows."""
    print(f"t2 mfma {rows} x {cols} -> {n_rows}", flush=True)
    dtype = O.T2B128
    data = synthetic_table(dtype, n_rows, cols, seed=n_rows + cols + rows + 1)
    t = table(fk, dtype, n_rows, cols, data)
    x = activations(rows, cols, seed=cols + 5 * rows, outliers=0.02)
    bias = np.random.default_rng(rows + 1).standard_normal(n_rows).astype(np.float32)
    want = oracle_product(dtype, n_rows, cols, data, x, rows, bias=bias)
    got = gpu_product(fk, t, x, rows, bias=bias)
    assert same_bits(got, want), first_mismatch(got, want)
    got_pre = gpu_product(fk, t, x, rows, bias=bias, fused=False)
    assert same_bits(got_pre, want), first_mismatch(got_pre, want)
    want_f = oracle_product(dtype, n_rows, cols, data, x, rows, fused=True)
    got_f = gpu_product(fk, t, x, rows, fused_scale=True)
    assert same_bits(got_f, want_f), first_mismatch(got_f, want_f)
    lo, hi = 4 * (n_rows // 12), 4 * ((n_rows + 3) // 4)
    want_r = oracle_product(dtype, n_rows, cols, data, x, rows, lo, hi)
    got_r = gpu_product(fk, t, x, rows, cols=range(lo, hi))
    assert same_bits(got_r, want_r), first_mismatch(got_r, want_r)


@pytest.mark.parametrize("rows", [5, 8, 12, 16])
@pytest.mark.parametrize("n", [4864, 4096])
def test_t2_small_batches_by_width(fk, rows, n):
    """5-16 rows: over 4864 columns (304 tiles of 16) the 16 x 16 matrix-core tiles, over 4096 (256
    tiles) the streamed row slices up to 8 rows and the tiles from 9; every output, bias, a column
    range, the fused scaling."""
    print(f"t2 small batch {rows} x 512 -> {n}", flush=True)
    dtype, k = O.T2B128, 512
    data = synthetic_table(dtype, n, k, seed=n + rows)
    t = table(fk, dtype, n, k, data)
    x = activations(rows, k, seed=rows + 7, outliers=0.02)
    bias = np.random.default_rng(rows).standard_normal(n).astype(np.float32)
    want = oracle_product(dtype, n, k, data, x, rows, bias=bias)
    got = gpu_product(fk, t, x, rows, bias=bias)
    assert same_bits(got, want), first_mismatch(got, want)
    want_r = oracle_product(dtype, n, k, data, x, rows, 64, n - 4)
    got_r = gpu_product(fk, t, x, rows, cols=range(64, n - 4))
    assert same_bits(got_r, want_r), first_mismatch(got_r, want_r)
    want_f = oracle_product(dtype, n, k, data, x, rows, fused=True)
    got_f = gpu_product(fk, t, x, rows, fused_scale=True)
    assert same_bits(got_f, want_f), first_mismatch(got_f, want_f)


def test_t2_many_tiles_bit_exact(fk):
    """128 rows x 4096 -> 2048 T2b128 (256 tiles in the per-XCD order), every output against the
    oracle's threaded product."""
    rows, n, k = 128, 2048, 4096
    data = synthetic_table(O.T2B128, n, k, seed=12)
    t = table(fk, O.T2B128, n, k, data)
    x = activations(rows, k, seed=13, outliers=0.01)
    got = gpu_product(fk, t, x, rows)
    q, s, c = O.quantize_rows(x.reshape(-1), O.T2B128)
    want = O.matmul_threaded(O.T2B128, n, k, data, q, s, c, rows, threads=16)
    assert same_bits(got, want), first_mismatch(got, want)


def test_t2_wide_tiles_bit_exact(fk):
    """512 rows x 128 -> 8196 T2b128: 2064 tiles of 32 x 64 (two MFMA chains per wave sharing the
    rows' operands), the last holding 4 columns; every output, with the fused scaling too."""
    rows, n, k = 512, 8196, 128
    data = synthetic_table(O.T2B128, n, k, seed=14)
    t = table(fk, O.T2B128, n, k, data)
    x = activations(rows, k, seed=15, outliers=0.01)
    q, s, c = O.quantize_rows(x.reshape(-1), O.T2B128)
    got = gpu_product(fk, t, x, rows)
    want = O.matmul_threaded(O.T2B128, n, k, data, q, s, c, rows, threads=16)
    assert same_bits(got, want), first_mismatch(got, want)
    got_f = gpu_product(fk, t, x, rows, fused_scale=True)
    want_f = oracle_product(O.T2B128, n, k, data, x, rows, fused=True)
    assert same_bits(got_f, want_f), first_mismatch(got_f, want_f)


@pytest.mark.parametrize("rows", [1, 16])
def test_t2_large_shape_bit_exact(fk, rows):
    """14336 x 4096 T2b128, every output against the oracle's threaded product."""
    n, k = 14336, 4096
    data = synthetic_table(O.T2B128, n, k, seed=2)
    t = table(fk, O.T2B128, n, k, data)
    x = activations(rows, k, seed=22)
    got = gpu_product(fk, t, x, rows)
    q, s, c = O.quantize_rows(x.reshape(-1), O.T2B128)
    want = O.matmul_threaded(O.T2B128, n, k, data, q, s, c, rows, threads=16)
    assert same_bits(got, want), first_mismatch(got, want)


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q4B32])
@pytest.mark.parametrize("rows,k", [(5, 32 * 8), (16, 32 * 8), (9, 32 * 17), (12, 32 * 28), (7, 32 * 3)])
def test_small_batch_streamed_with_one_or_two_stages(fk, dtype, rows, k):
    """The streamed small-batch product with fewer blocks than one stage of 16 (8 or 3 blocks),
    and one whole stage and 1 or 12 blocks of a second (17, 28 blocks: a tile's two waves split
    each stage's blocks 8 and 8, so the last stage's terms come from the first wave alone or from
    both); 5-16 rows, 8228 columns."""
    n = 8228
    data = synthetic_table(dtype, n, k, seed=rows + k)
    t = table(fk, dtype, n, k, data)
    x = activations(rows, k, seed=rows * 7 + k, outliers=0.02)
    got = gpu_product(fk, t, x, rows)
    want = oracle_product(dtype, n, k, data, x, rows)
    assert same_bits(got, want), first_mismatch(got, want)


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q8B32, O.Q4B32])
@pytest.mark.parametrize("rows", [5, 16])
def test_small_batch_streamed_over_many_columns(fk, dtype, rows):
    """5-16 rows over 515 tiles of 16 columns (the last workgroup's columns partly past the
    table): the operands streamed through LDS in stages of 16 blocks, four whole stages and a
    partial one of 8; then a column range starting inside the table, with bias."""
    n, k = 8228, 32 * 72
    data = synthetic_table(dtype, n, k, seed=rows + 17)
    t = table(fk, dtype, n, k, data)
    x = activations(rows, k, seed=rows + 71, outliers=0.02)
    bias = np.random.default_rng(6).standard_normal(n).astype(np.float32)
    got = gpu_product(fk, t, x, rows, bias=bias)
    want = oracle_product(dtype, n, k, data, x, rows, bias=bias)
    assert same_bits(got, want), first_mismatch(got, want)
    got = gpu_product(fk, t, x, rows, cols=range(36, n), bias=bias)
    assert same_bits(got, oracle_product(dtype, n, k, data, x, rows, 36, n, bias=bias))


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q4B32])
def test_small_batch_streamed_scale_products_below_the_normal_range(fk, dtype):
    """The streamed small-batch product forms fl(ws * as) with an f32 MFMA outer product: weight
    scales near 1e-8 and activations near 1e-30 make every such product subnormal, while the
    terms fl(D * p) are normal; the MFMA must round them as the VALU multiply does."""
    n, k, rows = 8228, 32 * 40, 16
    data = synthetic_table(dtype, n, k, seed=dtype + 40, scale_lo=1e-9, scale_hi=1e-8)
    t = table(fk, dtype, n, k, data)
    x = (activations(rows, k, seed=41) * np.float32(1e-30)).astype(np.float32)
    got = gpu_product(fk, t, x, rows)
    want = oracle_product(dtype, n, k, data, x, rows)
    assert same_bits(got, want), first_mismatch(got, want)
    assert np.all(np.isfinite(want)) and np.any(want != 0)


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q4B32])
@pytest.mark.parametrize("rows", [16, 40])
def test_split_rounds_with_whole_batches_and_a_tail(fk, dtype, rows):
    """Few tiles, long rows: four waves per tile take turns over the groups (11 rounds of four
    groups: two whole batches of four rounds and a tail of three), every sum in group order."""
    n, k = 96, 32 * 44
    data = synthetic_table(dtype, n, k, seed=rows + 7)
    t = table(fk, dtype, n, k, data)
    x = activations(rows, k, seed=rows + 70, outliers=0.02)
    bias = np.random.default_rng(4).standard_normal(n).astype(np.float32)
    got = gpu_product(fk, t, x, rows, bias=bias)
    want = oracle_product(dtype, n, k, data, x, rows, bias=bias)
    assert same_bits(got, want), first_mismatch(got, want)


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q8B32, O.Q4B32])
@pytest.mark.parametrize("rows", [5, 11, 16])
def test_small_batch_over_whole_tiles_bit_exact(fk, dtype, rows):
    """5-16 rows with whole tiles of 16 groups (the LDS-staged small-batch kernel): every row and
    column, a column range with bias, and the residual form."""
    import torch
    n, k = 100, 512
    data = synthetic_table(dtype, n, k, seed=rows + 3 * dtype)
    t = table(fk, dtype, n, k, data)
    x = activations(rows, k, seed=rows, outliers=0.02)
    assert same_bits(gpu_product(fk, t, x, rows), oracle_product(dtype, n, k, data, x, rows))
    bias = np.random.default_rng(2).standard_normal(n).astype(np.float32)
    got = gpu_product(fk, t, x, rows, cols=range(16, 100), bias=bias)
    assert same_bits(got, oracle_product(dtype, n, k, data, x, rows, 16, 100, bias=bias))
    h0 = np.random.default_rng(3).standard_normal((rows, n)).astype(np.float32)
    h = dev(h0)
    lin = fk.Linear(t, None)
    inp = fk.QuantizedRows().input(t.matrix(), dev(x.reshape(-1)))
    fk.project_residual_input(fk.Ctx(0, 1), lin, inp, h)
    full = oracle_product(dtype, n, k, data, x, rows)[:, :n]
    want_h = h0.copy()
    want_h[:, :96] = (h0[:, :96] + full[:, :96]).astype(np.float32)
    assert same_bits(host(h), want_h)


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q8B32, O.Q4B32])
def test_batched_product_with_subnormal_scale_products(fk, dtype):
    """Weight scales near 1e-8 and activations near 1e-30: every fl(ws·as) is subnormal (about
    1e-41) while the terms fl(D·p) are normal; the batched path keeps the reference's bits."""
    n, k, rows = 70, 256, 40
    data = synthetic_table(dtype, n, k, seed=dtype, scale_lo=1e-9, scale_hi=1e-8)
    t = table(fk, dtype, n, k, data)
    x = (activations(rows, k, seed=3) * np.float32(1e-30)).astype(np.float32)
    want = oracle_product(dtype, n, k, data, x, rows)
    assert same_bits(gpu_product(fk, t, x, rows), want), first_mismatch(gpu_product(fk, t, x, rows), want)
    assert np.all(np.isfinite(want)) and np.any(want != 0)


def test_batched_rows_equal_row_by_row_products(fk):
    """A size-independent property: the matrix-core path and the matrix-vector path are the same
    function of each row."""
    n, k, rows = 1152, 896, 24
    data = synthetic_table(O.Q7B32, n, k, seed=8)
    t = table(fk, O.Q7B32, n, k, data)
    x = activations(rows, k, seed=8)
    batched = gpu_product(fk, t, x, rows)
    for r in range(0, rows, 5):
        assert same_bits(batched[r:r + 1], gpu_product(fk, t, x[r:r + 1], 1))


def test_zero_rows_and_empty_ranges(fk):
    data = synthetic_table(O.Q7B32, 8, 64, seed=1)
    t = table(fk, O.Q7B32, 8, 64, data)
    x = activations(2, 64, seed=1)
    assert gpu_product(fk, t, x, 2, cols=range(4, 4)).shape == (2, 0)


# ------------------------------------------------------------------------ golden vectors

def _golden(name):
    import os
    with np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", name)) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name,dtype", [("Q7b32", O.Q7B32), ("Q4b32", O.Q4B32), ("T2b128", O.T2B128),
                                        ("Q8b32", O.Q8B32)])
def test_golden_lcg_vectors_on_the_gpu(fk, name, dtype):
    """tests/golden/lcg_25x128.npz: levels, scales, corrections, group accumulators and f32
    outputs of the reference test's inputs (matmul.rs:809-843), bit for bit."""
    import torch
    g = _golden("lcg_25x128.npz")
    t = table(fk, dtype, 25, 128, g[f"{name}/table"])
    assert np.array_equal(t.reference_bytes(), g[f"{name}/table"])
    for rows in (1, 3, 8, 11):
        p = f"{name}/rows{rows}/"
        x = g[p + "x"]
        n, grp = x.size, O.group(dtype)
        q = torch.empty(n, dtype=torch.int8, device="cuda")
        s = torch.empty(n // grp, dtype=torch.float32, device="cuda")
        c = torch.empty(n // grp, dtype=torch.int32, device="cuda")
        fk.quantize_rows(dev(x), fk.QuantFormat(dtype), q, s, c)
        assert np.array_equal(host(q), g[p + "q"])
        assert same_bits(host(s), g[p + "scales"])
        assert np.array_equal(host(c), g[p + "corrections"])
        assert same_bits(gpu_product(fk, t, x, rows), g[p + "out"])
        assert np.array_equal(gpu_product(fk, t, x, rows, dots=True), g[p + "dots"])


@pytest.mark.parametrize("name,dtype", [("Q7b32", O.Q7B32), ("Q8b32", O.Q8B32)])
def test_golden_single_matvec_digest_on_the_gpu(fk, name, dtype):
    """tests/golden/matvec_4864x896_seed0.npz: the 4864 x 896 seed-0 matvec's outputs and
    accumulators by digest."""
    import hashlib
    g = _golden("matvec_4864x896_seed0.npz")
    data = synthetic_table(dtype, 4864, 896, seed=0)
    t = table(fk, dtype, 4864, 896, data)
    x = activations(1, 896, seed=0)
    out = np.ascontiguousarray(gpu_product(fk, t, x, 1), np.float32)
    assert hashlib.sha256(out.tobytes()).digest() == g[f"{name}/out_sha256"].tobytes()
    dots = np.ascontiguousarray(gpu_product(fk, t, x, 1, dots=True), np.int32)
    assert hashlib.sha256(dots.tobytes()).digest() == g[f"{name}/dots_sha256"].tobytes()
