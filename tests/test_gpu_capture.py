"""fg_matmul captured in a HIP graph: the scratch of f32 rows is the graph's, not an allocation node.

Products that quantize f32 rows first (the matrix cores from five rows, T2b128) need scratch for the
levels and scales. Under capture it is allocated once, outside the stream's work, and owned by the
graph; each replay rewrites it before reading it. Every replay is checked against the eager product
bit for bit, with the program's own eager products and synchronizations between replays and new
input values before some of them (a replay reads the input tensor it was captured with); after the
graph is gone, the next product (which frees the graph's scratch) is checked too.
"""

import numpy as np
import pytest

from oracle import oracle as O
from gpu_data import activations, synthetic_table

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fk(gpu):
    import fusor_kernels
    return fusor_kernels


def same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


CASES = [(O.Q8B32, 5, 896, 1152), (O.Q7B32, 40, 4864, 896), (O.Q8B32, 512, 896, 4096), (O.Q4B32, 64, 4096, 1024),
         (O.T2B128, 64, 512, 200)]


@pytest.mark.parametrize("dtype,rows,k,n", CASES)
def test_captured_product_replays_match_the_eager_product(fk, dtype, rows, k, n):
    import torch
    print(f"captured product dtype {dtype} {rows}x{k}->{n}", flush=True)
    data = synthetic_table(dtype, n, k, seed=rows + n)
    t = fk.Table(fk.Tensor(dtype, [n, k], data))
    m = t.matrix()
    width = (n + 3) // 4 * 4
    xs = [activations(rows, k, seed=rows + i, outliers=0.01) for i in range(3)]
    x = torch.from_numpy(xs[0].reshape(-1)).cuda()
    out = torch.full((rows, width), float("nan"), dtype=torch.float32, device="cuda")
    inp = fk.Input(f32=x)
    fk.matmul(m, inp, range(0, width), out=out)  # eager once (kernels loaded, pools warm)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fk.matmul(m, inp, range(0, width), out=out)
    other = fk.Table(fk.Tensor(dtype, [n, k], synthetic_table(dtype, n, k, seed=rows + n + 1)))
    for replay, xi in enumerate([0, 0, 1, 2, 1]):
        x.copy_(torch.from_numpy(xs[xi].reshape(-1)))
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        want = fk.matmul(m, fk.Input(f32=x), range(0, width)).cpu().numpy()
        assert same_bits(got, want), (replay, xi)
        # the program's own eager work between replays, on a product of the same shape
        fk.matmul(other.matrix(), fk.Input(f32=x), range(0, width))
        torch.cuda.synchronize()
    q, s, c = O.quantize_rows(xs[1].reshape(-1), dtype)
    head = min(rows, 16)
    assert same_bits(got[:head], O.matmul(dtype, n, k, data, q[:head * k], s[:head * k // O.group(dtype)],
                                          c[:head * k // O.group(dtype)], head))
    del graph
    torch.cuda.synchronize()
    after = fk.matmul(m, fk.Input(f32=x), range(0, width))
    torch.cuda.synchronize()
    assert same_bits(after.cpu().numpy(), got)
