"""GPU parity of the run-time Q7b32 matrix (QuantizedMatrix), the team-split projections
(project, project_residual) and the row products (conv::project_rows) against the oracle,
bit for bit, through the C ABI."""

import numpy as np
import pytest

from oracle import oracle as O
from gpu_data import activations, synthetic_table

pytestmark = pytest.mark.gpu


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


def oracle_product(dtype, rows_w, cols_w, data, x, rows, col_begin=0, col_end=None, bias=None):
    q, s, c = O.quantize_rows(np.ascontiguousarray(x, np.float32).reshape(-1), dtype)
    return O.matmul(dtype, rows_w, cols_w, data, q, s, c, rows, col_begin, col_end, bias=bias)


# ---------------------------------------------------------------------- QuantizedMatrix

def test_quantized_matrix_rows_are_the_encoded_rows(fk):
    """push / set_block write what Tensor::encode writes for those rows (quantize_q7 and
    set_block agree: quant.rs:143-149, matmul.rs:77-90); extended rows stay zero codes and zero
    scales (matmul.rs:66-72), as the padding of a table is (tensor.rs:83-88)."""
    rng = np.random.default_rng(11)
    cols = 128
    values = (rng.standard_normal((5, cols)) * 2).astype(np.float32)
    values[1, :32] = 0.0                       # a zero block: scale 1
    values[3, 40] = np.float32(1e-40)          # a subnormal in a block of zeros
    values[3, 32:40] = 0.0
    values[3, 41:64] = 0.0
    values[4, 100] = np.nan
    m = fk.QuantizedMatrix(capacity=3, max_cols=256)   # grows twice
    m.reset(cols)
    for r in range(5):
        m.push(dev(values[r]))
    assert m.rows == 5
    assert np.array_equal(m.table.reference_bytes(), O.encode(O.Q7B32, 5, cols, values))
    # set_block over a block of row 2
    block = (rng.standard_normal(32) * 5).astype(np.float32)
    m.set_block(2, 1, dev(block))
    values[2, 32:64] = block
    assert np.array_equal(m.table.reference_bytes(), O.encode(O.Q7B32, 5, cols, values))
    # three more rows, unset: zero codes and scales (the padding rows of a 5-row table)
    m.extend(3)
    assert m.rows == 8
    assert np.array_equal(m.table.reference_bytes(), O.encode(O.Q7B32, 5, cols, values))
    # rows set in bulk
    more = rng.standard_normal((3, cols)).astype(np.float32)
    m.set_rows(5, dev(more))
    full = np.concatenate([values, more])
    want = O.encode(O.Q7B32, 8, cols, full)
    assert np.array_equal(m.table.reference_bytes(), want)
    # dequantize_row of the run-time matrix
    import torch
    out = torch.empty(cols, dtype=torch.float32, device="cuda")
    for r in range(8):
        m.matrix().dequantize_row(r, out)
        assert same_bits(host(out), O.dequantize_row(O.Q7B32, 8, cols, want, r))


def test_quantized_matrix_multiplies_like_weights(fk):
    """The attention use (attention.rs:81-214): keys as the weights of a product."""
    rng = np.random.default_rng(12)
    cols, n = 64, 37
    keys = rng.standard_normal((n, cols)).astype(np.float32)
    m = fk.QuantizedMatrix(capacity=64, max_cols=cols)
    m.reset(cols)
    m.extend(n)
    m.set_rows(0, dev(keys))
    data = O.encode(O.Q7B32, n, cols, keys)
    for rows in (1, 3, 9):
        x = activations(rows, cols, seed=rows)
        got = host(fk.matmul(m.matrix(), fk.Input(f32=dev(x.reshape(-1))), range(0, 40)))
        assert same_bits(got, oracle_product(O.Q7B32, n, cols, data, x, rows))


def test_quantized_matrix_reset_and_errors(fk):
    rng = np.random.default_rng(13)
    m = fk.QuantizedMatrix(capacity=8, max_cols=128)
    m.reset(128)
    m.push(dev(rng.standard_normal(128).astype(np.float32)))
    m.reset(64)                              # narrower rows, no rows
    assert m.rows == 0
    vals = rng.standard_normal((2, 64)).astype(np.float32)
    m.push(dev(vals[0]))
    m.push(dev(vals[1]))
    assert np.array_equal(m.table.reference_bytes(), O.encode(O.Q7B32, 2, 64, vals))
    with pytest.raises(fk.ShapeError, match="rows of whole blocks"):
        m.reset(40)
    with pytest.raises(fk.ShapeError, match="wider than"):
        m.reset(256)
    with pytest.raises(fk.ShapeError, match="rows past the matrix"):
        m.set_rows(1, dev(vals))
    with pytest.raises(fk.ShapeError, match="a block past the matrix"):
        m.set_block(0, 2, dev(vals[0, :32]))
    with pytest.raises(fk.ShapeError, match="a row of the matrix's width"):
        m.push(dev(np.zeros(32, np.float32)))


# ------------------------------------------------------------------ team-split projections

@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q4B32, O.T2B128])
@pytest.mark.parametrize("rows", [1, 5])
def test_project_and_project_residual_over_a_team(fk, dtype, rows):
    """linear.rs:100-143: every thread's share of the columns, together, is the whole product
    plus bias; the residual form adds it in place."""
    n, k = 96, 256
    data = synthetic_table(dtype, n, k, seed=rows + 20 * dtype)
    t = fk.Table(fk.Tensor(dtype, [n, k], data))
    bias = np.random.default_rng(3).standard_normal(n).astype(np.float32)
    lin = fk.Linear(t, fk.Vector(fk.Tensor(fk.DType.F32, [n], bias.view(np.uint8))))
    x = activations(rows, k, seed=4)
    buf = dev(np.concatenate([x.reshape(-1), np.full(k, 7.0, np.float32)]))  # one row past `rows`
    want = oracle_product(dtype, n, k, data, x, rows, bias=bias)[:, :n]
    import torch
    out = torch.full((rows, n), np.nan, dtype=torch.float32, device="cuda")
    for i in range(3):
        fk.project(fk.Ctx(i, 3), lin, fk.SharedRows(buf, rows), fk.QuantizedRows(), out)
    assert same_bits(host(out), want)
    h0 = np.random.default_rng(5).standard_normal((rows, n)).astype(np.float32)
    h = dev(h0)
    for i in range(2):
        fk.project_residual(fk.Ctx(i, 2), lin, fk.SharedRows(buf, rows), h, fk.QuantizedRows())
    assert same_bits(host(h), (h0 + want).astype(np.float32))


@pytest.mark.parametrize("rows,n,threads", [(100, 48, 3), (20, 160, 2), (7, 40, 2)])
def test_project_rows_splits_by_rows_or_columns(fk, rows, n, threads):
    """conv.rs:563-606: by rows when rows >= outputs or outputs are not whole 16-column units,
    else by columns; each thread's share is the reference's bits."""
    import torch
    k = 128
    data = synthetic_table(O.Q8B32, n, k, seed=rows)
    t = fk.Table(fk.Tensor(fk.DType.Q8b32, [n, k], data))
    bias = np.random.default_rng(6).standard_normal(n).astype(np.float32)
    lin = fk.Linear(t, fk.Vector(fk.Tensor(fk.DType.F32, [n], bias.view(np.uint8))))
    x = activations(rows, k, seed=7, outliers=0.02)
    out = torch.full((rows, n), np.nan, dtype=torch.float32, device="cuda")
    for i in range(threads):
        fk.project_rows(fk.Ctx(i, threads), lin, (dev(x), rows), fk.Patches(), out)
    want = oracle_product(O.Q8B32, n, k, data, x, rows, bias=bias)[:, :n]
    assert same_bits(host(out), want)
