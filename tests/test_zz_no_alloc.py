"""fg_matmul_noalloc: the product with no device allocation, its scratch a fixed array per device.

Through the C ABI, against fg_matmul on the same inputs (bit for bit: both run the same kernels),
two calls in a row where the second is smaller (the array keeps the first call's contents), the
formats and row paths that use the scratch (f32 rows on the matrix cores, T2b128), a path that
needs none, and the error for a product past the array's size.
"""

import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from gpu_data import activations, synthetic_table

pytestmark = pytest.mark.gpu

SCRATCH = 32 << 20


@pytest.fixture(scope="module")
def fk(gpu):
    import fusor_kernels
    return fusor_kernels


def noalloc(fk, table, x, rows, width, bias=None, out=None, flags=0):
    import torch
    from fusor_kernels import _lib
    if out is None:
        out = torch.full((rows, width), float("nan"), dtype=torch.float32, device="cuda")
    inp = _lib.FgInput(_lib.ptr(x), None, None, None)
    _lib.check(_lib.lib().fg_matmul_noalloc(table.handle, ctypes.byref(inp), rows, 0, width, _lib.ptr(bias),
                                            _lib.ptr(out), out.stride(0), flags, _lib.stream_handle()))
    return out


def same_bits(a, b):
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q8B32, O.Q4B32, O.T2B128])
def test_noalloc_equals_the_allocating_product_twice_in_a_row(fk, dtype):
    import torch
    print(f"noalloc dtype {dtype}", flush=True)
    cases = [(512, 896, 1152), (37, 640, 260)] if dtype != O.T2B128 else [(64, 512, 96), (9, 256, 40)]
    for rows, k, n in cases:  # the second call smaller than the first
        data = synthetic_table(dtype, n, k, seed=rows + n)
        t = fk.Table(fk.Tensor(dtype, [n, k], data))
        width = (n + 3) // 4 * 4
        xh = activations(rows, k, seed=rows + k, outliers=0.01)
        x = torch.from_numpy(xh.reshape(-1)).cuda()
        bias = torch.from_numpy(np.random.default_rng(n).standard_normal(n).astype(np.float32)).cuda()
        want = fk.matmul(t.matrix(), fk.Input(f32=x), range(0, width), bias=bias)
        got = noalloc(fk, t, x, rows, width, bias=bias)
        torch.cuda.synchronize()
        assert same_bits(got.cpu().numpy(), want.cpu().numpy()), (rows, k, n)
        q, s, c = O.quantize_rows(xh.reshape(-1), dtype)
        oracle = O.matmul(dtype, n, k, data, q, s, c, rows, bias=bias.cpu().numpy())
        assert same_bits(got.cpu().numpy(), oracle), (rows, k, n)


def test_noalloc_on_the_staged_kernel(fk):
    """Products on the LDS-staged kernel, whose f32 rows are quantized straight into block-major
    scales (no row-major scales or corrections in the scratch): 6144 x 4096 -> 4096 needs 24 MiB of
    levels and 3 MiB of scales, then a smaller call. Bit for bit against fg_matmul on every row and
    against the oracle on the first rows (rows are independent)."""
    import torch
    dtype = O.Q8B32
    for rows, k, n in [(6144, 4096, 4096), (512, 4096, 4096)]:
        print(f"noalloc staged {rows} x {k} -> {n}", flush=True)
        data = synthetic_table(dtype, n, k, seed=rows + 1)
        t = fk.Table(fk.Tensor(dtype, [n, k], data))
        xh = activations(rows, k, seed=rows + 2, outliers=0.01)
        x = torch.from_numpy(xh.reshape(-1)).cuda()
        want = fk.matmul(t.matrix(), fk.Input(f32=x), range(0, n))
        got = noalloc(fk, t, x, rows, n)
        torch.cuda.synchronize()
        got_h = got.cpu().numpy()
        assert same_bits(got_h, want.cpu().numpy()), (rows, k, n)
        head = 16
        q, s, c = O.quantize_rows(xh[:head].reshape(-1), dtype)
        assert same_bits(got_h[:head], O.matmul(dtype, n, k, data, q, s, c, head)), (rows, k, n)


def test_noalloc_accumulates_and_takes_the_fused_scale(fk):
    import torch
    from fusor_kernels import _lib
    rows, k, n = 24, 512, 200
    data = synthetic_table(O.Q8B32, n, k, seed=3)
    t = fk.Table(fk.Tensor(O.Q8B32, [n, k], data))
    x = torch.from_numpy(activations(rows, k, seed=4).reshape(-1)).cuda()
    h0 = torch.from_numpy(np.random.default_rng(5).standard_normal((rows, n)).astype(np.float32)).cuda()
    want = h0.clone()
    fk.matmul(t.matrix(), fk.Input(f32=x), range(0, n), out=want, accumulate=True, fused=True)
    got = noalloc(fk, t, x, rows, n, out=h0.clone(), flags=_lib.FG_ACCUMULATE | _lib.FG_FUSED_SCALE)
    torch.cuda.synchronize()
    assert same_bits(got.cpu().numpy(), want.cpu().numpy())


def test_noalloc_without_scratch_and_past_its_size(fk):
    import torch
    # one row runs on the matrix-vector kernel, which quantizes in the kernel: no scratch at all
    data = synthetic_table(O.Q7B32, 4864, 896, seed=0)
    t = fk.Table(fk.Tensor(O.Q7B32, [4864, 896], data))
    x = torch.from_numpy(activations(1, 896, seed=0).reshape(-1)).cuda()
    want = fk.matmul(t.matrix(), fk.Input(f32=x), range(0, 4864))
    got = noalloc(fk, t, x, 1, 4864)
    torch.cuda.synchronize()
    assert same_bits(got.cpu().numpy(), want.cpu().numpy())
    # 8192 rows of 4096 f32 values need 32 MiB of levels plus their scales and corrections
    big = torch.zeros(8192 * 4096, dtype=torch.float32, device="cuda")
    t2 = fk.Table(fk.Tensor(O.Q8B32, [16, 4096], synthetic_table(O.Q8B32, 16, 4096, seed=1)))
    with pytest.raises(fk.ShapeError, match="bytes of scratch"):
        noalloc(fk, t2, big, 8192, 16)
