"""The decoder's prefill (fg_qwen2_read: Reader::read, lm.rs:205-228) against the oracle's read.

Rows go through the stack a chunk at a time, each layer over every row of the chunk with its
products on the matrix cores, each row attending to the keys up to its own position. In the exact
order the caches, the last row's residual row, its logits and its greedy token are bit-identical to
the oracle's read (itself pinned to one decode step per token, tests/test_oracle_read.py), for every
chunk size; in the parallel order they stay within the reference's stack tolerance.
"""

import numpy as np
import pytest

from oracle import oracle as O
from gpu_data import qwen2_model

pytestmark = pytest.mark.gpu

FAST_TOLERANCE = 2e-2


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
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.sqrt(np.sum((got - want) ** 2) / np.sum(want * want)))


def gpu_model(fk, dtype, params, exact):
    sh, lys, final, table, kc, vc = params
    shape = fk.Shape(hidden=sh.hidden, layers=sh.layers, heads=sh.heads, kv_heads=sh.kv_heads, head_dim=sh.head_dim,
                     ffn=sh.ffn, vocab=sh.vocab, capacity=sh.capacity, rope_base=sh.rope_base, eps=sh.eps)
    dims = {"qkv": (shape.qkv(), sh.hidden), "o": (sh.hidden, shape.width()), "gate": (sh.ffn, sh.hidden),
            "up": (sh.ffn, sh.hidden), "down": (sh.hidden, sh.ffn)}
    layers = []
    for f in lys:
        d = {k: fk.Table(fk.Tensor(dtype, list(dims[k]), f[k])) for k in dims}
        d["norm1"], d["norm2"], d["qkv_bias"] = dev(f["norm1"]), dev(f["norm2"]), dev(f["qkv_bias"])
        layers.append(d)
    head = fk.Table(fk.Tensor(dtype, [sh.vocab, sh.hidden], table))
    kd, vd = dev(kc), dev(vc)
    model = fk.Qwen2(shape, dtype, layers, dev(final), head, kd, vd, exact=exact)
    model._keep = (layers, head)
    return model, kd, vd


def read_gpu(fk, dtype, params, ids, first, chunk, exact):
    """The GPU's read, embedding on the device too: hidden, logits, token, caches, embeddings."""
    import torch
    sh = params[0]
    model, kd, vd = gpu_model(fk, dtype, params, exact)
    emb = model.embed(dev(np.asarray(ids, np.int32)))
    hidden = torch.empty(sh.hidden, dtype=torch.float32, device="cuda")
    logits = torch.empty(sh.vocab, dtype=torch.float32, device="cuda")
    nxt = torch.empty(1, dtype=torch.int32, device="cuda")
    model.read(emb, first, chunk, hidden, logits, nxt)
    return host(hidden), host(logits), int(host(nxt)[0]), host(kd), host(vd), host(emb)


def read_both(fk, dtype, params, ids, first, chunk, exact, threads=8):
    """The GPU's read and the oracle's, from the same caches."""
    sh, lys, final, table, kc, vc = params
    got = read_gpu(fk, dtype, params, ids, first, chunk, exact)
    oracle = O.Qwen2(sh, lys, final, table)
    want_emb = oracle.embed(ids)
    k2, v2 = kc.copy(), vc.copy()
    want = oracle.read(k2, v2, want_emb, first, chunk, threads=threads)
    return got, want + (k2, v2, want_emb)


SMALL = dict(hidden=128, layers=2, heads=4, kv_heads=2, head_dim=32, ffn=256, vocab=96, capacity=80)


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q8B32, O.Q4B32])
@pytest.mark.parametrize("chunk", [1, 4, 5, 16, 17, 64])
def test_exact_read_is_bit_identical_for_every_chunk(fk, dtype, chunk):
    """Chunks of 1 and 4 rows take the matrix-vector kernel, 5 to 16 the 16-row tiles, 17 and more
    the 32 x 32 tiles; 37 rows from position 6 leave a partial last chunk."""
    print(f"prefill dtype {dtype} chunk {chunk}", flush=True)
    params = qwen2_model(dtype, seed=31, synthetic=False, **SMALL)
    ids = np.random.default_rng(chunk + dtype).integers(0, SMALL["vocab"], 37).astype(np.int32)
    got, want = read_both(fk, dtype, params, ids, 6, chunk, exact=True)
    assert same_bits(got[5], want[5]), "embeddings"
    assert same_bits(got[0], want[0]), "hidden"
    assert same_bits(got[1], want[1]), "logits"
    assert got[2] == want[2]
    assert same_bits(got[3], want[3]) and same_bits(got[4], want[4]), "caches"


@pytest.mark.parametrize("head_dim,heads,kv_heads", [(64, 4, 1), (128, 2, 2), (32, 6, 3), (128, 12, 2)])
def test_read_head_sizes(fk, head_dim, heads, kv_heads):
    """Every head size, and rows of heads wider than 1024; 70 rows from position 0 in chunks of 32
    (keys and values staged in passes of 4096 / D rows: rows that see one to three passes)."""
    print(f"prefill heads {heads}/{kv_heads} D {head_dim}", flush=True)
    shape = dict(hidden=256, layers=2, heads=heads, kv_heads=kv_heads, head_dim=head_dim, ffn=512, vocab=64,
                 capacity=128)
    params = qwen2_model(O.Q7B32, seed=head_dim + heads, synthetic=False, **shape)
    ids = np.random.default_rng(head_dim).integers(0, 64, 70).astype(np.int32)
    got, want = read_both(fk, O.Q7B32, params, ids, 0, 32, exact=True)
    assert same_bits(got[0], want[0]) and same_bits(got[1], want[1]) and got[2] == want[2]
    assert same_bits(got[3], want[3]) and same_bits(got[4], want[4])
    got, want = read_both(fk, O.Q7B32, params, ids, 0, 32, exact=False)
    assert rel_l2(got[0], want[0]) < FAST_TOLERANCE and rel_l2(got[1], want[1]) < FAST_TOLERANCE


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q8B32, O.Q4B32])
def test_qwen2_half_billion_shape_prefill_of_158_rows(fk, dtype):
    """The Qwen2-0.5B shape: 158 rows from position 100 (a cache of N(0,1) rows before it) in chunks
    of 64, the reference's prefill length (models/ming/baseline.json:52-55): bit-identical."""
    print(f"prefill Qwen2-0.5B shape dtype {dtype}", flush=True)
    params = qwen2_model(dtype, hidden=896, layers=24, heads=14, kv_heads=2, head_dim=64, ffn=4864, vocab=151936,
                         capacity=512, seed=13, synthetic=True)
    ids = np.random.default_rng(dtype).integers(0, 151936, 158).astype(np.int32)
    got, want = read_both(fk, dtype, params, ids, 100, 64, exact=True, threads=16)
    assert same_bits(got[0], want[0]) and same_bits(got[1], want[1]) and got[2] == want[2]
    assert same_bits(got[3], want[3]) and same_bits(got[4], want[4])
    # parallel order (the attention on the matrix cores) against the same oracle read, in one
    # chunk of 158 rows as the bench reads: 24 random-weight layers amplify any level flip, so the
    # decode step's bound at this shape (0.1) applies
    fast = read_gpu(fk, dtype, params, ids, 100, 158, exact=False)
    e_h, e_l = rel_l2(fast[0], want[0]), rel_l2(fast[1], want[1])
    print(f"parallel order rel-L2: hidden {e_h:.3e} logits {e_l:.3e}", flush=True)
    assert e_h < 0.1 and e_l < 0.1


@pytest.mark.parametrize("first", [1400, 1500])
def test_read_over_long_caches(fk, first):
    """Rows that see over a thousand keys: from position 1400 the per-block attention stages its keys
    and values in a dozen passes; from 1500 the rows' scores no longer fit its LDS and the chunk
    takes the scores and weighted-sum kernels over its rows instead. Bit-identical in exact order,
    within the stack tolerance in parallel order."""
    print(f"prefill from position {first}", flush=True)
    shape = dict(hidden=128, layers=1, heads=4, kv_heads=2, head_dim=32, ffn=256, vocab=64, capacity=1600)
    params = qwen2_model(O.Q7B32, seed=first, synthetic=False, **shape)
    ids = np.random.default_rng(first).integers(0, 64, 40).astype(np.int32)
    got, want = read_both(fk, O.Q7B32, params, ids, first, 40, exact=True)
    assert same_bits(got[0], want[0]) and same_bits(got[1], want[1]) and got[2] == want[2]
    assert same_bits(got[3], want[3]) and same_bits(got[4], want[4])
    got, want = read_both(fk, O.Q7B32, params, ids, first, 40, exact=False)
    assert rel_l2(got[0], want[0]) < FAST_TOLERANCE and rel_l2(got[1], want[1]) < FAST_TOLERANCE


def test_read_then_decode_continues_the_sequence(fk):
    """A read followed by decode steps at the next positions equals one step per token (exact)."""
    import torch
    dtype = O.Q7B32
    params = qwen2_model(dtype, seed=41, synthetic=False, **SMALL)
    sh, lys, final, table, kc, vc = params
    model, kd, vd = gpu_model(fk, dtype, params, exact=True)
    ids = np.random.default_rng(3).integers(0, sh.vocab, 20).astype(np.int32)
    nxt = torch.empty(1, dtype=torch.int32, device="cuda")
    model.read(model.embed(dev(ids[:12])), 0, 5, next_token=nxt)
    logits = torch.empty(sh.vocab, dtype=torch.float32, device="cuda")
    for i in range(12, 20):
        model.step(int(ids[i]), i, logits=logits, next_token=nxt)
    oracle = O.Qwen2(sh, lys, final, table)
    k2, v2 = kc.copy(), vc.copy()
    for i in range(20):
        _, want_l, want_t = oracle.step(k2, v2, int(ids[i]), i)
    assert same_bits(host(logits), want_l) and int(host(nxt)[0]) == want_t
    assert same_bits(host(kd), k2) and same_bits(host(vd), v2)


def test_read_refuses_rows_past_the_cache(fk):
    params = qwen2_model(O.Q7B32, seed=5, synthetic=False, **SMALL)
    model, _, _ = gpu_model(fk, O.Q7B32, params, exact=True)
    emb = model.embed(dev(np.arange(10, dtype=np.int32)))
    with pytest.raises(fk.ShapeError, match="holds every key"):
        model.read(emb, SMALL["capacity"] - 9, 4)
