"""fg_attend (attention::attend, blocks/src/attention.rs:81-214) on the GPU against the oracle.

Every step is deterministic and the f32 steps follow the reference's order, so the outputs are
bit-identical to the oracle's for both exponentials, across the product's row paths (1-4 rows
on the matrix-vector kernel, 5-16 and 17+ on the matrix cores), grouped heads, several images,
padded head and key counts, and operands read by stride and offset from one fused row."""
import numpy as np
import pytest

from oracle import oracle as O

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


def gpu_attend(fk, H, KV, D, I, Q, K, q, k, v, fast, layouts=None):
    import torch
    ql, kl, vl = layouts or ((H * D, 0), (KV * D, 0), (KV * D, 0))
    qd, kd, vd = dev(q.reshape(-1)), dev(k.reshape(-1)), dev(v.reshape(-1))
    if layouts:
        kd = vd = qd
    out = torch.full((I * Q, H * D), float("nan"), dtype=torch.float32, device="cuda")
    call = fk.Call(H, KV, D, I, Q, K, fk.Operand(qd, *ql), fk.Operand(kd, *kl), fk.Operand(vd, *vl),
                   fk.Exponentials.FAST if fast else fk.Exponentials.EXACT)
    fk.attend(call, out)
    return host(out)


def same_bits(a, b):
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


CASES = [  # heads, kv_heads, head_dim, images, queries, keys, fast
    (2, 2, 64, 1, 3, 200, True),      # 3 query rows: the scores on the matrix-vector kernel
    (6, 1, 32, 3, 5, 9, True),        # 5 rows: the scores on the 16-row matrix-core kernel
    (4, 2, 40, 2, 37, 53, False),     # 37 rows, padded head_dim (40 -> 64) and keys (53 -> 64)
    (4, 2, 40, 2, 37, 53, True),
    (3, 3, 16, 1, 1, 1, False),       # one key, one query
    (8, 2, 128, 1, 64, 1000, False),  # a long row of keys; 128 value channels: 128-wide tiles
    (2, 1, 72, 1, 70, 300, True),     # the DiT block's head size: 72 channels in one 128-wide tile
    (1, 1, 64, 1, 4, 4096, True),     # the DiT block's 4096 keys, the scores on the matrix-vector kernel
    (2, 1, 64, 1, 5, 16384, False),   # the largest row of keys: 64 KiB of scores per row in LDS
    (1, 1, 32, 1, 2, 16384, True),
]


@pytest.mark.parametrize("case", CASES)
def test_attend_is_the_oracles_bits(fk, case):
    H, KV, D, I, Q, K, fast = case
    print("attend", case, flush=True)
    rng = np.random.default_rng(sum(case))
    q = rng.standard_normal((I * Q, H * D)).astype(np.float32)
    k = rng.standard_normal((I * K, KV * D)).astype(np.float32)
    v = rng.standard_normal((I * K, KV * D)).astype(np.float32)
    want = O.attend(H, KV, D, I, Q, K, q, k, v, fast=fast)
    got = gpu_attend(fk, H, KV, D, I, Q, K, q, k, v, fast)
    assert same_bits(got, want), np.max(np.abs(got - want))


@pytest.mark.parametrize("units", [1, 4, 5])
def test_attend_in_batches_of_heads(fk, monkeypatch, units):
    """The weighted values' product runs per batch of (image, head) units, each unit reading key
    head table unit / group; batches of 1, 4 and 5 units over 2 images of 6 heads in 2 key heads
    start at every offset into a key head's group."""
    H, KV, D, I, Q, K = 6, 2, 72, 2, 37, 53
    monkeypatch.setenv("FG_ATTEND_UNITS", str(units))
    rng = np.random.default_rng(units)
    q = rng.standard_normal((I * Q, H * D)).astype(np.float32)
    k = rng.standard_normal((I * K, KV * D)).astype(np.float32)
    v = rng.standard_normal((I * K, KV * D)).astype(np.float32)
    want = O.attend(H, KV, D, I, Q, K, q, k, v, fast=True)
    got = gpu_attend(fk, H, KV, D, I, Q, K, q, k, v, True)
    assert same_bits(got, want), np.max(np.abs(got - want))


def test_attend_reads_a_fused_qkv_row(fk):
    H, KV, D, I, Q = 4, 2, 32, 2, 21
    rng = np.random.default_rng(3)
    row = (H + 2 * KV) * D
    qkv = rng.standard_normal((I * Q, row)).astype(np.float32)
    layouts = ((row, 0), (row, H * D), (row, (H + KV) * D))
    want = O.attend(H, KV, D, I, Q, Q, qkv, qkv, qkv, query_layout=layouts[0], key_layout=layouts[1],
                    value_layout=layouts[2])
    got = gpu_attend(fk, H, KV, D, I, Q, Q, qkv, qkv, qkv, False, layouts)
    assert same_bits(got, want)


def test_attend_twice_in_a_row_gives_the_same_bits(fk):
    H, KV, D, I, Q, K = 2, 1, 32, 1, 9, 40
    rng = np.random.default_rng(8)
    q = rng.standard_normal((I * Q, H * D)).astype(np.float32)
    k = rng.standard_normal((I * K, KV * D)).astype(np.float32)
    v = rng.standard_normal((I * K, KV * D)).astype(np.float32)
    a = gpu_attend(fk, H, KV, D, I, Q, K, q, k, v, True)
    b = gpu_attend(fk, H, KV, D, I, Q, K, q, k, v, True)
    assert same_bits(a, b) and same_bits(a, O.attend(H, KV, D, I, Q, K, q, k, v, fast=True))


def test_attend_rejects_shapes_it_does_not_take(fk):
    import torch
    z = torch.zeros(4096, dtype=torch.float32, device="cuda")
    out = torch.zeros(4096, dtype=torch.float32, device="cuda")
    def call(H, KV, D, I=1, Q=1, K=1, qs=None):
        return fk.Call(H, KV, D, I, Q, K, fk.Operand(z, qs or H * D), fk.Operand(z, KV * D), fk.Operand(z, KV * D))
    with pytest.raises(fk.ShapeError):
        fk.attend(call(3, 2, 16), out)          # heads not a multiple of the key heads
    with pytest.raises(fk.ShapeError):
        fk.attend(call(2, 1, 18), out)          # head_dim not whole quads
    with pytest.raises(fk.ShapeError):
        fk.attend(call(2, 1, 16, qs=16), out)   # the heads run past the row stride
    with pytest.raises(fk.ShapeError):
        fk.attend(call(2, 1, 16, Q=1000), out)  # the rows run past the tensor
    big = torch.zeros(16416 * 16, dtype=torch.float32, device="cuda")
    with pytest.raises(fk.ShapeError):
        fk.attend(fk.Call(1, 1, 16, 1, 1, 16416, fk.Operand(big, 16), fk.Operand(big, 16), fk.Operand(big, 16)), out)
