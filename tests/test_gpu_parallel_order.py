"""The decoder's parallel-order kernels against the oracle on identical inputs.

The decode step's fast mode keeps every integer and every group term of the reference and changes
only the order of f32 additions: the team sums of a projection's group terms, and the attention as
flash decoding (chunks of keys merged by the output projection). These tests hold each of them,
kernel by kernel, to the bound such a reordering allows and to 1e-5 relative:

* a projection summed in parallel (fg_matmul with FG_PARALLEL_SUM, the decoder's team sums) against
  the oracle's group-order product at the decode step's shapes: every output within
  2 (G - 1) 2^-24 sum_g |t_g| of it (two orders of the same G terms t_g), and 1e-5 relative in norm;
* one layer's attention row (fg_qwen2_attention) against softmax (or_softmax over or_dot_f32 scores)
  and the weighted sum of the values, on the query, keys and values the kernels themselves used:
  every output within 1e-5 of sum_j w_j |v_j| and 1e-5 relative in norm.
"""

import numpy as np
import pytest

from oracle import oracle as O
from gpu_data import activations, synthetic_table

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


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


def weight_scales(dtype, rows, cols, data):
    """ws[n, g] from the reference bytes: f32 at ((q G + g) 4 + lane) after the codes
    (tensor.rs:1-9)."""
    quads, groups = (rows + 3) // 4, cols // O.group(dtype)
    raw = np.ascontiguousarray(data[O.quant_len(dtype, rows, cols):]).view(np.float32)
    return raw.reshape(quads, groups, 4).transpose(0, 2, 1).reshape(quads * 4, groups)


def group_terms(dtype, rows, cols, data, dots, scales):
    """t[n, g] = fl(fl((float)D) * fl(ws * as)) of one activation row: the terms both orders add."""
    ws = weight_scales(dtype, rows, cols, data)[: dots.shape[0]]
    p = (ws * scales[None, :].astype(np.float32)).astype(np.float32)
    return (dots.astype(np.float32) * p).astype(np.float32)


DECODE_SHAPES = [(1152, 896), (896, 896), (4864, 896), (896, 4864), (151936, 896)]


@pytest.mark.parametrize("n,k", DECODE_SHAPES)
@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q4B32])
def test_parallel_sum_projection_within_the_reordering_bound(fk, n, k, dtype):
    print(f"parallel-order projection {n}x{k} dtype {dtype}", flush=True)
    data = synthetic_table(dtype, n, k, seed=n + k + dtype)
    t = fk.Table(fk.Tensor(dtype, [n, k], data))
    m = t.matrix()
    x = activations(1, k, seed=k + 1, outliers=0.01)
    q, s, c = O.quantize_rows(x.reshape(-1), dtype)
    want, dots = O.matmul(dtype, n, k, data, q, s, c, 1, want_dots=True)
    want, dots = want[0, :n], dots[0, :n]
    width = (n + 3) // 4 * 4
    got_f32 = host(fk.matmul(m, fk.Input(f32=dev(x.reshape(-1))), range(0, width), parallel=True))[0, :n]
    inp = fk.QuantizedRows().input(m, dev(x.reshape(-1)))
    got_pre = host(fk.matmul(m, inp, range(0, width), parallel=True))[0, :n]
    terms = group_terms(dtype, n, k, data, dots, s)
    G = terms.shape[1]
    # the oracle's group-order sum is the sequential sum of these terms (pins the helper itself)
    seq = np.zeros(n, np.float32)
    for g in range(G):
        seq = (seq + terms[:, g]).astype(np.float32)
    assert np.array_equal(seq.view(np.uint32), want.view(np.uint32))
    bound = 2 * (G - 1) * U * np.abs(terms.astype(np.float64)).sum(axis=1)
    for got in (got_f32, got_pre):
        err = np.abs(got.astype(np.float64) - want.astype(np.float64))
        assert np.all(err <= bound), (int(np.argmax(err - bound)), float(np.max(err - bound)))
        rel = np.linalg.norm(got.astype(np.float64) - want) / np.linalg.norm(want.astype(np.float64))
        assert rel <= 1e-5, rel
    assert np.array_equal(got_f32.view(np.uint32), got_pre.view(np.uint32))
    if n >= 4864:
        # the flag reaches the tree sums: over this many outputs some additions round differently
        assert not np.array_equal(got_f32.view(np.uint32), want.view(np.uint32))


def test_parallel_sum_rejects_what_it_does_not_cover(fk):
    data = synthetic_table(O.Q7B32, 64, 128, seed=1)
    t = fk.Table(fk.Tensor(O.Q7B32, [64, 128], data))
    x = dev(activations(2, 128, seed=2).reshape(-1))
    with pytest.raises(fk.ShapeError, match="one row"):
        fk.matmul(t.matrix(), fk.Input(f32=x), range(0, 64), parallel=True)
    with pytest.raises(ValueError, match="exclude"):
        fk.matmul(t.matrix(), fk.Input(f32=x[:128]), range(0, 64), parallel=True, fused=True)


# ------------------------------------------------------------------- the attention row

def build_layer(heads, kv_heads, head_dim, hidden, capacity, seed):
    rng = np.random.default_rng(seed)
    qkv_w = (heads + 2 * kv_heads) * head_dim
    dims = {"qkv": (qkv_w, hidden), "o": (hidden, heads * head_dim), "gate": (64, hidden), "up": (64, hidden),
            "down": (hidden, 64)}
    f = {name: O.encode(O.Q7B32, r, c, (rng.standard_normal((r, c)) / np.sqrt(c)).astype(np.float32))
         for name, (r, c) in dims.items()}
    f["norm1"] = (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
    f["norm2"] = (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
    f["qkv_bias"] = (0.1 * rng.standard_normal(qkv_w)).astype(np.float32)
    kc = rng.standard_normal((1, kv_heads, capacity, head_dim)).astype(np.float32)
    vc = rng.standard_normal((1, kv_heads, capacity, head_dim)).astype(np.float32)
    return dims, f, kc, vc


def attention_model(fk, heads, kv_heads, head_dim, hidden, capacity, exact, seed):
    dims, f, kc, vc = build_layer(heads, kv_heads, head_dim, hidden, capacity, seed)
    shape = fk.Shape(hidden=hidden, layers=1, heads=heads, kv_heads=kv_heads, head_dim=head_dim, ffn=64, vocab=64,
                     capacity=capacity)
    layer = {k: fk.Table(fk.Tensor(O.Q7B32, list(dims[k]), f[k])) for k in dims}
    layer["norm1"], layer["norm2"], layer["qkv_bias"] = dev(f["norm1"]), dev(f["norm2"]), dev(f["qkv_bias"])
    table = fk.Table(fk.Tensor(O.Q7B32, [64, hidden], O.encode(O.Q7B32, 64, hidden,
                                                              np.ones((64, hidden), np.float32))))
    kd, vd = dev(kc), dev(vc)
    model = fk.Qwen2(shape, O.Q7B32, [layer], dev(f["norm1"]), table, kd, vd, exact=exact)
    model._keep = (layer, table)
    return model, kd, vd


def softmax_row(query, kcache, vcache, heads, kv_heads, head_dim, position):
    """The attention of each head over keys 0..position (ops.rs:301-342): scores dot_f32(q, k_j) /
    sqrt(D) in f32, or_softmax, then sum_j w_j v_j in f64; also sum_j w_j |v_j| (the bound's scale)."""
    group = heads // kv_heads
    scale = np.float32(1.0) / np.sqrt(np.float32(head_dim))
    out = np.zeros((heads, head_dim))
    mag = np.zeros((heads, head_dim))
    for h in range(heads):
        kv = h // group
        q = query[h * head_dim:(h + 1) * head_dim]
        scores = np.array([O.dot_f32(q, kcache[0, kv, j]) * scale for j in range(position + 1)], np.float32)
        w = O.softmax(scores).astype(np.float64)
        v = vcache[0, kv, :position + 1].astype(np.float64)
        out[h] = w @ v
        mag[h] = w @ np.abs(v)
    return out.reshape(-1), mag.reshape(-1)


@pytest.mark.parametrize("exact", [False, True])
@pytest.mark.parametrize("heads,kv_heads,head_dim,hidden,capacity", [(14, 2, 64, 896, 512), (4, 1, 32, 128, 300),
                                                                     (8, 2, 128, 256, 640), (12, 2, 128, 256, 300)])
def test_attention_row_equals_softmax_on_identical_inputs(fk, exact, heads, kv_heads, head_dim, hidden, capacity):
    """Flash decoding (parallel order: chunks of 64-key tiles, four waves per chunk, merged by the
    output projection's prologue with the position's own key; rows of heads up to 1024 wide), the
    sliced weighted sums of wider rows, and the exact-order kernels, each against softmax and the
    weighted sum over the query, keys and values the kernels used."""
    import torch
    model, kd, vd = attention_model(fk, heads, kv_heads, head_dim, hidden, capacity, exact, seed=head_dim + heads)
    x = np.random.default_rng(heads).standard_normal(hidden).astype(np.float32)
    width = heads * head_dim
    for position in (0, 1, 63, 64, 200, capacity - 1):
        print(f"attention row heads {heads}/{kv_heads} D {head_dim} exact {exact} position {position}", flush=True)
        query = torch.empty(width, dtype=torch.float32, device="cuda")
        row = torch.full((width,), float("nan"), dtype=torch.float32, device="cuda")
        model.attention(0, position, dev(x), query, row)
        got, q, kc, vc = host(row), host(query), host(kd), host(vd)
        want, mag = softmax_row(q, kc, vc, heads, kv_heads, head_dim, position)
        err = np.abs(got.astype(np.float64) - want)
        assert np.all(err <= 1e-5 * mag), (position, int(np.argmax(err / np.maximum(mag, 1e-30))))
        assert np.linalg.norm(got - want) <= 1e-5 * np.linalg.norm(want), position
