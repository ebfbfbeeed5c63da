"""The boundary's thread-safety contract: every thread of a team calls the product at once.

The reference calls the projection from each team thread on its own `Ctx::split(N, 16)` column
range (linear.rs:113-143, team/src/team.rs:46-68); the C ABI promises that concurrent calls on
disjoint outputs are independent. Eight host threads call fg_quantize_rows and fg_matmul together
(ctypes releases the interpreter lock for the call), once on one shared stream and once on a
stream each; their shares must equal one full-range call to the bit. The batched case quantizes
its f32 rows inside each call, so the calls also share the product's workspace pool.
"""

import threading

import numpy as np
import pytest

from oracle import oracle as O
from gpu_data import activations, synthetic_table

pytestmark = pytest.mark.gpu

THREADS = 8


@pytest.fixture(scope="module")
def fk(gpu):
    import fusor_kernels
    return fusor_kernels


def run_team(fn):
    """fn(i) on THREADS threads started together; re-raises the first failure."""
    barrier = threading.Barrier(THREADS)
    errors = []

    def body(i):
        try:
            barrier.wait()
            fn(i)
        except BaseException as e:  # noqa: BLE001 - reported below
            errors.append(e)

    threads = [threading.Thread(target=body, args=(i,)) for i in range(THREADS)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    if errors:
        raise errors[0]


@pytest.mark.parametrize("per_thread_streams", [False, True])
@pytest.mark.parametrize("dtype,rows,n,k", [(O.Q7B32, 1, 4864, 896), (O.Q4B32, 1, 14336, 1024),
                                            (O.Q8B32, 40, 1152, 896), (O.Q7B32, 16, 2048, 512)])
def test_team_threads_share_one_product(fk, per_thread_streams, dtype, rows, n, k):
    import torch
    print(f"team of {THREADS}: dtype {dtype} {rows}x{k}->{n} per-thread streams {per_thread_streams}", flush=True)
    data = synthetic_table(dtype, n, k, seed=n + rows)
    t = fk.Table(fk.Tensor(dtype, [n, k], data))
    m = t.matrix()
    x = torch.from_numpy(activations(rows, k, seed=rows + k, outliers=0.01).reshape(-1)).cuda()
    bias = torch.from_numpy(np.random.default_rng(n).standard_normal(n).astype(np.float32)).cuda()
    full = fk.matmul(m, fk.Input(f32=x), range(0, n), bias=bias)
    torch.cuda.synchronize()
    want = full.cpu().numpy()
    q, s, c = O.quantize_rows(activations(rows, k, seed=rows + k, outliers=0.01).reshape(-1), dtype)
    assert np.array_equal(want.view(np.uint32), O.matmul(dtype, n, k, data, q, s, c, rows, bias=bias.cpu().numpy())
                          .view(np.uint32))

    out = torch.full((rows, n), float("nan"), dtype=torch.float32, device="cuda")
    g = O.group(dtype)
    levels = torch.zeros(rows * k, dtype=torch.int8, device="cuda")
    scales = torch.zeros(rows * k // g, dtype=torch.float32, device="cuda")
    corrs = torch.zeros(rows * k // g, dtype=torch.int32, device="cuda")
    shared = torch.cuda.Stream()
    torch.cuda.synchronize()

    def share(i):
        stream = torch.cuda.Stream() if per_thread_streams else shared
        with torch.cuda.stream(stream):
            cols = fk.Ctx(i, THREADS).split(n, fk.COLUMN_ALIGN)
            if len(cols):
                fk.matmul(m, fk.Input(f32=x), cols, bias=bias, out=out[:, cols.start:cols.stop])
            # and this thread's rows-share of the activation quantization (whole groups)
            groups = rows * k // g
            lo, hi = groups * i // THREADS, groups * (i + 1) // THREADS
            if hi > lo:
                fk.quantize_rows(x[lo * g:hi * g], fk.QuantFormat(dtype), levels[lo * g:hi * g], scales[lo:hi],
                                 corrs[lo:hi])
        stream.synchronize()

    run_team(share)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(levels.cpu().numpy(), q)
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), s.view(np.uint32))
    assert np.array_equal(corrs.cpu().numpy(), c)
