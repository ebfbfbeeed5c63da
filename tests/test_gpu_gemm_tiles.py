"""The batched matrix-core products at each of their kernel choices, against the oracle.

The product picks its kernel by shape; FG_GEMM_TILE forces one (0: the register-ring kernels, which
over few 32 x 32 tiles and a multiple of four blocks are the four-wave split kernel; 11: the
LDS-staged kernel's 64 x 64 workgroup tiles, 21: its 128 x 64), so every choice meets the edge
cases here: rows and columns that end inside a tile, an odd number of blocks (the last two-block
stage half empty) or of rounds of four blocks (the split kernel's last pair of rounds half
empty), activation scales staged in LDS (more than 64 blocks) or read with the operands, a column
range that starts inside the table, bias and the residual form, f32 and pre-quantized rows, the
NEON backend's fused scaling, and scale products fl(ws * as) that are subnormal (both kernels form
them with an f32 MFMA outer product, which must round them as the VALU does).
"""

import numpy as np
import pytest

from oracle import oracle as O
from gpu_data import activations, synthetic_table

pytestmark = pytest.mark.gpu

TILES = ["0", "11", "21"]


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


def same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def first_mismatch(a, b):
    a = np.asarray(a, np.float32).reshape(-1)
    b = np.asarray(b, np.float32).reshape(-1)
    bad = np.nonzero(a.view(np.uint32) != b.view(np.uint32))[0]
    return (int(bad[0]), float(a[bad[0]]), float(b[bad[0]]), len(bad)) if len(bad) else None


def oracle(dtype, n, k, data, x, rows, col_begin=0, col_end=None, bias=None, fused=False):
    q, s, c = O.quantize_rows(x.reshape(-1), dtype)
    return O.matmul(dtype, n, k, data, q, s, c, rows, col_begin, col_end, bias=bias, fused=fused)


@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q8B32, O.Q4B32])
@pytest.mark.parametrize("rows,n,k", [(17, 36, 32), (100, 200, 160), (257, 516, 1152), (130, 2050, 96), (300, 260, 2176)])
def test_tile_shapes_bit_exact(fk, monkeypatch, tile, dtype, rows, n, k):
    monkeypatch.setenv("FG_GEMM_TILE", tile)
    print(f"tile {tile} dtype {dtype} {rows}x{k}->{n}", flush=True)
    data = synthetic_table(dtype, n, k, seed=rows + n + k)
    t = fk.Table(fk.Tensor(dtype, [n, k], data))
    m = t.matrix()
    x = activations(rows, k, seed=rows * 3 + k, outliers=0.01)
    width = (n + 3) // 4 * 4
    want = oracle(dtype, n, k, data, x, rows)
    got = host(fk.matmul(m, fk.Input(f32=dev(x.reshape(-1))), range(0, width)))
    assert same_bits(got, want), first_mismatch(got, want)
    inp = fk.QuantizedRows().input(m, dev(x.reshape(-1)))
    got = host(fk.matmul(m, inp, range(0, width)))
    assert same_bits(got, want), first_mismatch(got, want)
    # a column range starting inside the table, with bias, added to a residual
    bias = np.random.default_rng(n).standard_normal(n).astype(np.float32)
    lo, hi = 8, width - 4 if width > 12 else width
    h0 = np.random.default_rng(k).standard_normal((rows, hi - lo)).astype(np.float32)
    h = dev(h0)
    fk.matmul(m, inp, range(lo, hi), bias=dev(bias), out=h, accumulate=True)
    want_b = oracle(dtype, n, k, data, x, rows, lo, hi, bias=bias)
    assert same_bits(host(h), (h0 + want_b).astype(np.float32))
    # the NEON backend's scaling
    got_f = host(fk.matmul(m, inp, range(0, width), fused=True))
    want_f = oracle(dtype, n, k, data, x, rows, fused=True)
    assert same_bits(got_f, want_f), first_mismatch(got_f, want_f)


@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q8B32, O.Q4B32])
def test_tile_scale_products_below_the_normal_range(fk, monkeypatch, tile, dtype):
    """Weight scales near 1e-8 and activations near 1e-30: every fl(ws·as) is subnormal while the
    terms fl(D·p) are normal."""
    monkeypatch.setenv("FG_GEMM_TILE", tile)
    n, k, rows = 70, 256, 40
    data = synthetic_table(dtype, n, k, seed=dtype, scale_lo=1e-9, scale_hi=1e-8)
    t = fk.Table(fk.Tensor(dtype, [n, k], data))
    x = (activations(rows, k, seed=3) * np.float32(1e-30)).astype(np.float32)
    want = oracle(dtype, n, k, data, x, rows)
    got = host(fk.matmul(t.matrix(), fk.Input(f32=dev(x.reshape(-1))), range(0, 72)))
    assert same_bits(got, want), first_mismatch(got, want)
    assert np.all(np.isfinite(want)) and np.any(want != 0)


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q8B32, O.Q4B32])
@pytest.mark.parametrize("rows,n,k", [(17, 96, 2048), (64, 260, 4864), (158, 896, 2048), (256, 132, 3072)])
def test_row_bands_over_a_long_k(fk, dtype, rows, n, k):
    """17 to 256 rows over 64 or more blocks take the paired 16-row tiles in bands of 16 rows: a last
    band that ends inside its tile, a last column tile of two quads, f32 and pre-quantized rows, a
    column range starting inside the table with bias, added to a residual."""
    print(f"row bands dtype {dtype} {rows}x{k}->{n}", flush=True)
    data = synthetic_table(dtype, n, k, seed=rows + n + k + 1)
    t = fk.Table(fk.Tensor(dtype, [n, k], data))
    m = t.matrix()
    x = activations(rows, k, seed=rows + k, outliers=0.01)
    width = (n + 3) // 4 * 4
    want = oracle(dtype, n, k, data, x, rows)
    got = host(fk.matmul(m, fk.Input(f32=dev(x.reshape(-1))), range(0, width)))
    assert same_bits(got, want), first_mismatch(got, want)
    inp = fk.QuantizedRows().input(m, dev(x.reshape(-1)))
    got = host(fk.matmul(m, inp, range(0, width)))
    assert same_bits(got, want), first_mismatch(got, want)
    bias = np.random.default_rng(n).standard_normal(n).astype(np.float32)
    lo, hi = 4, width
    h0 = np.random.default_rng(k).standard_normal((rows, hi - lo)).astype(np.float32)
    h = dev(h0)
    fk.matmul(m, inp, range(lo, hi), bias=dev(bias), out=h, accumulate=True)
    want_b = oracle(dtype, n, k, data, x, rows, lo, hi, bias=bias)
    assert same_bits(host(h), (h0 + want_b).astype(np.float32))


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q8B32, O.Q4B32])
@pytest.mark.parametrize("rows,n,k", [(17, 36, 256), (40, 260, 4864), (158, 1152, 896), (512, 896, 4864)])
def test_fused_scaling_over_few_tiles(fk, dtype, rows, n, k):
    """The NEON backend's scaling over few 32 x 32 tiles (four waves per tile on its 16 x 16 quarters):
    a last row and column tile that end inside the tile, an odd number of stages, bias and the
    residual form, against the oracle's fused product."""
    print(f"fused few tiles dtype {dtype} {rows}x{k}->{n}", flush=True)
    data = synthetic_table(dtype, n, k, seed=rows + n + k + 2)
    t = fk.Table(fk.Tensor(dtype, [n, k], data))
    m = t.matrix()
    x = activations(rows, k, seed=rows + 2 * k, outliers=0.01)
    width = (n + 3) // 4 * 4
    want = oracle(dtype, n, k, data, x, rows, fused=True)
    got = host(fk.matmul(m, fk.Input(f32=dev(x.reshape(-1))), range(0, width), fused=True))
    assert same_bits(got, want), first_mismatch(got, want)
    inp = fk.QuantizedRows().input(m, dev(x.reshape(-1)))
    bias = np.random.default_rng(n).standard_normal(n).astype(np.float32)
    h0 = np.random.default_rng(k).standard_normal((rows, width - 4)).astype(np.float32)
    h = dev(h0)
    fk.matmul(m, inp, range(4, width), bias=dev(bias), out=h, accumulate=True, fused=True)
    want_b = oracle(dtype, n, k, data, x, rows, 4, width, bias=bias, fused=True)
    assert same_bits(host(h), (h0 + want_b).astype(np.float32))
