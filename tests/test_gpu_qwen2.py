"""The Qwen2 decoder step on the GPU against the oracle's step (blocks::transformer + lm).

Exact mode keeps every reduction in the reference's order: hidden state, logits, greedy token and
the kept keys and values are bit-identical. Fast mode (parallel reductions) is held to a relative
L2 error of 2e-2 (the reference's own bound for 7-bit stacks, blocks/tests/stacks.rs:51-56) and
the same greedy token.
"""

import math

import numpy as np
import pytest

from oracle import oracle as O
from gpu_data import qwen2_model as build

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


def rel_l2(got, want):
    got = got.astype(np.float64)
    want = want.astype(np.float64)
    return float(np.sqrt(np.sum((got - want) ** 2) / np.sum(want * want)))


def gpu_model(fk, dtype, sh, lys, final, table, kc, vc, exact):
    shape = fk.Shape(hidden=sh.hidden, layers=sh.layers, heads=sh.heads, kv_heads=sh.kv_heads, head_dim=sh.head_dim,
                     ffn=sh.ffn, vocab=sh.vocab, capacity=sh.capacity, rope_base=sh.rope_base, eps=sh.eps)
    qkv_w = shape.qkv()
    dims = {"qkv": (qkv_w, sh.hidden), "o": (sh.hidden, shape.width()), "gate": (sh.ffn, sh.hidden),
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


def run_both(fk, dtype, params, token, position, exact):
    import torch
    sh, lys, final, table, kc, vc = params
    model, kd, vd = gpu_model(fk, dtype, sh, lys, final, table, kc, vc, exact)
    hidden = torch.empty(sh.hidden, dtype=torch.float32, device="cuda")
    logits = torch.empty(sh.vocab, dtype=torch.float32, device="cuda")
    nxt = torch.empty(1, dtype=torch.int32, device="cuda")
    model.step(token, position, hidden, logits, nxt)
    k2, v2 = kc.copy(), vc.copy()
    want_h, want_l, want_t = O.Qwen2(sh, lys, final, table).step(k2, v2, token, position, threads=8)
    return (host(hidden), host(logits), int(host(nxt)[0]), host(kd), host(vd)), (want_h, want_l, want_t, k2, v2)


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


SMALL = dict(hidden=128, layers=2, heads=4, kv_heads=2, head_dim=32, ffn=256, vocab=96, capacity=32)


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q8B32, O.Q4B32])
def test_small_decoder_exact_mode_is_bit_identical(fk, dtype):
    params = build(dtype, seed=3, synthetic=False, **SMALL)
    for position in (0, 5, 31):
        got, want = run_both(fk, dtype, params, token=17, position=position, exact=True)
        assert same_bits(got[0], want[0]), ("hidden", position)
        assert same_bits(got[1], want[1]), ("logits", position)
        assert got[2] == want[2]
        assert same_bits(got[3], want[3]) and same_bits(got[4], want[4])


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q4B32])
def test_small_decoder_fast_mode_within_tolerance(fk, dtype):
    params = build(dtype, seed=4, synthetic=False, **SMALL)
    got, want = run_both(fk, dtype, params, token=3, position=20, exact=False)
    assert rel_l2(got[0], want[0]) < FAST_TOLERANCE
    assert rel_l2(got[1], want[1]) < FAST_TOLERANCE


@pytest.mark.parametrize("head_dim,heads,kv_heads", [(64, 4, 1), (128, 2, 2), (32, 6, 3)])
def test_decoder_head_sizes_and_many_key_chunks(fk, head_dim, heads, kv_heads):
    """Every head size the decoder takes, and positions past several 64-key chunks of the
    parallel-order attention: exact mode bit-identical, parallel order within tolerance."""
    shape = dict(hidden=256, layers=2, heads=heads, kv_heads=kv_heads, head_dim=head_dim, ffn=512, vocab=64,
                 capacity=300)
    params = build(O.Q7B32, seed=head_dim, synthetic=False, **shape)
    for position in (63, 64, 200, 299):
        got, want = run_both(fk, O.Q7B32, params, token=9, position=position, exact=True)
        assert same_bits(got[0], want[0]), ("hidden", position)
        assert same_bits(got[1], want[1]), ("logits", position)
        assert same_bits(got[3], want[3]) and same_bits(got[4], want[4])
        got, want = run_both(fk, O.Q7B32, params, token=9, position=position, exact=False)
        assert rel_l2(got[0], want[0]) < FAST_TOLERANCE, ("fast hidden", position)
        assert rel_l2(got[1], want[1]) < FAST_TOLERANCE, ("fast logits", position)


@pytest.mark.parametrize("head_dim,heads,kv_heads", [(64, 4, 2), (128, 2, 1)])
def test_exact_attention_with_few_keys_and_a_ragged_capacity(fk, head_dim, heads, kv_heads):
    """The one-launch exact-order attention (head sizes 64 and 128) with 1, 2, 16, 17 and 37 keys in
    a cache of 37 positions (its LDS rows are laid out past a capacity that is not whole runs of
    16): bit-identical to the oracle's step."""
    shape = dict(hidden=128, layers=2, heads=heads, kv_heads=kv_heads, head_dim=head_dim, ffn=256, vocab=64,
                 capacity=37)
    params = build(O.Q7B32, seed=head_dim + 1, synthetic=False, **shape)
    for position in (0, 1, 15, 16, 36):
        got, want = run_both(fk, O.Q7B32, params, token=5, position=position, exact=True)
        assert same_bits(got[0], want[0]), ("hidden", position)
        assert same_bits(got[1], want[1]), ("logits", position)
        assert got[2] == want[2]
        assert same_bits(got[3], want[3]) and same_bits(got[4], want[4])


def test_decoder_with_rows_of_heads_wider_than_1024(fk):
    """12 query heads of 128 over 2 key heads: the attention row (1536) is past what the
    flash-decoding merge takes, so parallel order runs the scores and weighted-sum kernels with
    eight slices of partial sums and a block-reduced total; positions on both sides of one
    256-key chunk of values. Exact mode bit-identical, parallel order within tolerance."""
    shape = dict(hidden=256, layers=2, heads=12, kv_heads=2, head_dim=128, ffn=512, vocab=64, capacity=300)
    params = build(O.Q7B32, seed=12, synthetic=False, **shape)
    for position in (200, 255, 256, 299):
        got, want = run_both(fk, O.Q7B32, params, token=7, position=position, exact=True)
        assert same_bits(got[0], want[0]), ("hidden", position)
        assert same_bits(got[1], want[1]), ("logits", position)
        assert same_bits(got[3], want[3]) and same_bits(got[4], want[4])
        got, want = run_both(fk, O.Q7B32, params, token=7, position=position, exact=False)
        assert rel_l2(got[0], want[0]) < FAST_TOLERANCE, ("fast hidden", position)
        assert rel_l2(got[1], want[1]) < FAST_TOLERANCE, ("fast logits", position)


def test_layer_forward_equals_the_oracle_layer(fk):
    import torch
    dtype = O.Q7B32
    sh, lys, final, table, kc, vc = build(dtype, seed=5, synthetic=False, **SMALL)
    model, kd, vd = gpu_model(fk, dtype, sh, lys, final, table, kc, vc, exact=True)
    x = np.random.default_rng(0).standard_normal(sh.hidden).astype(np.float32)
    h = dev(x)
    model.layer_forward(1, 7, h)
    cos, sin = O.rope_tables(sh.rope_base, sh.head_dim, sh.capacity)
    k2, v2 = kc.copy(), vc.copy()
    want = O.Qwen2(sh, lys, final, table).layer_forward(1, k2, v2, 7, cos[7], sin[7], x)
    assert same_bits(host(h), want)


@pytest.mark.parametrize("exact", [True, False])
def test_consecutive_steps_feed_back_the_greedy_token(fk, exact):
    """Several steps on one model, each fed the previous step's greedy token (the head's
    workgroups leave one candidate each, a last launch picks among them). Exact mode matches the
    oracle's tokens and cache rows step by step; parallel order repeats its own first step."""
    import torch
    dtype = O.Q7B32
    shape = dict(SMALL, vocab=600)  # 150 quads: 10 workgroups of candidates
    sh, lys, final, table, kc, vc = build(dtype, seed=8, synthetic=False, **shape)
    model, kd, vd = gpu_model(fk, dtype, sh, lys, final, table, kc, vc, exact)
    oracle = O.Qwen2(sh, lys, final, table)
    k2, v2 = kc.copy(), vc.copy()
    nxt = torch.empty(1, dtype=torch.int32, device="cuda")
    token = 5
    firsts = []
    for position in range(4, 9):
        model.step(token, position, next_token=nxt)
        got = int(host(nxt)[0])
        _, _, want = oracle.step(k2, v2, token, position, threads=8)
        if exact:
            assert got == want, position
        firsts.append(got)
        token = want
    if exact:
        assert same_bits(host(kd), k2) and same_bits(host(vd), v2)
    else:
        again, _, _ = gpu_model(fk, dtype, sh, lys, final, table, kc, vc, exact)
        again.step(5, 4, next_token=nxt)
        assert int(host(nxt)[0]) == firsts[0]


def first_largest(logits):
    """Prediction::greedy (lm.rs:169-179): the first index of the largest logit, NaNs never win,
    and a NaN first logit keeps index 0."""
    best, idx = logits[0], 0
    for i in range(1, len(logits)):
        if logits[i] > best:
            best, idx = logits[i], i
    return idx


@pytest.mark.parametrize("exact", [True, False])
@pytest.mark.parametrize("start", [5, 300])
def test_greedy_pick_takes_the_first_of_equal_logits_and_never_a_nan(fk, exact, start):
    """The greedy token with ties and NaNs placed in the head's table (64 rows per workgroup of
    candidates): the largest row a copied to row a // 2 (the same workgroup for a small a, another
    for a large one), a NaN scale on row a // 2 instead, and a NaN scale on row 0. Exact mode
    matches the oracle's token; both modes pick the reference's token from their own logits."""
    import torch
    dtype = O.Q7B32
    shape = dict(SMALL, vocab=700)  # 175 quads: 11 workgroups of candidates
    sh, lys, final, table, kc, vc = build(dtype, seed=12, synthetic=False, **shape)
    rng = np.random.default_rng(12)
    rows = rng.standard_normal((sh.vocab, sh.hidden)).astype(np.float32)
    base = O.encode(dtype, sh.vocab, sh.hidden, rows)
    # a token whose own (embedding) row none of the changes touches (the tied table makes a token's
    # own row its largest logit, as here)
    for token in range(start, start + 40):
        _, _, a = O.Qwen2(sh, lys, final, base).step(kc.copy(), vc.copy(), token, 9, threads=8)
        if a > 1 and token != a // 2:
            break
    else:
        pytest.fail("no token leaves its own row unchanged")
    b = a // 2
    tied = rows.copy()
    tied[b] = rows[a]
    quant_len = (sh.vocab + 3) // 4 * 4 * sh.hidden  # Q7b32: a byte per code; the scales follow
    groups = sh.hidden // 32

    def nan_scale(t, row):
        t = t.copy()
        at = quant_len + ((row // 4 * groups) * 4 + row % 4) * 4  # the row's first group
        t[at:at + 4] = np.frombuffer(np.float32(np.nan).tobytes(), np.uint8)
        return t

    cases = {"tie": (O.encode(dtype, sh.vocab, sh.hidden, tied), b), "nan_earlier": (nan_scale(base, b), a),
             "nan_first": (nan_scale(base, 0), 0)}
    for name, (t, expect) in cases.items():
        model, _, _ = gpu_model(fk, dtype, sh, lys, final, t, kc, vc, exact)
        logits = torch.empty(sh.vocab, dtype=torch.float32, device="cuda")
        nxt = torch.empty(1, dtype=torch.int32, device="cuda")
        model.step(token, 9, logits=logits, next_token=nxt)
        got, got_l = int(host(nxt)[0]), host(logits)
        assert got == first_largest(got_l), name
        if name == "tie":
            assert same_bits(got_l[a], got_l[b]) and got != a, name
        elif name == "nan_earlier":
            assert np.isnan(got_l[b]) and got != b, name
        else:
            assert np.isnan(got_l[0]) and got == 0, name
        if exact:
            _, _, want = O.Qwen2(sh, lys, final, t).step(kc.copy(), vc.copy(), token, 9, threads=8)
            assert got == want == expect, name


def test_decoder_rejects_positions_past_the_cache(fk):
    import torch
    dtype = O.Q7B32
    sh, lys, final, table, kc, vc = build(dtype, seed=6, synthetic=False, **SMALL)
    model, _, _ = gpu_model(fk, dtype, sh, lys, final, table, kc, vc, exact=False)
    with pytest.raises(fk.ShapeError):
        model.step(1, sh.capacity)


@pytest.mark.parametrize("exact", [True, False])
@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q8B32, O.Q4B32])
def test_qwen2_half_billion_shape_at_position_511(fk, exact, dtype):
    """The Qwen2-0.5B-shaped step (hidden 896, 24 layers, 14/2 heads of 64, FFN 4864, vocabulary
    151936) at position 511 over a cache of N(0,1) keys and values, with 7-bit, full-range 8-bit
    and 4-bit tables (the reference's LM layers run Q4b32: models/ming/compile/src/lib.rs:49-56)."""
    print(f"Qwen2-0.5B shape dtype {dtype} exact {exact}", flush=True)
    params = build(dtype, hidden=896, layers=24, heads=14, kv_heads=2, head_dim=64, ffn=4864, vocab=151936,
                   capacity=512, seed=11, synthetic=True)
    got, want = run_both(fk, dtype, params, token=1234, position=511, exact=exact)
    if exact:
        assert same_bits(got[0], want[0])
        assert same_bits(got[1], want[1])
        assert got[2] == want[2]
        assert same_bits(got[3], want[3]) and same_bits(got[4], want[4])
    else:
        # 24 random-weight layers amplify any level flip: the oracle itself, fed the same embedding
        # with 1e-6 relative noise, ends about 3.5e-2 away. Fast mode must stay within twice the
        # oracle's own divergence (and under 0.1).
        sh, lys, final, table, kc, vc = params
        model = O.Qwen2(sh, lys, final, table)
        cos, sin = O.rope_tables(sh.rope_base, sh.head_dim, sh.capacity)
        h = O.dequantize_row(dtype, sh.vocab, sh.hidden, table, 1234)
        hp = (h * (1 + 1e-6 * np.random.default_rng(0).standard_normal(sh.hidden))).astype(np.float32)
        k1, v1, k2, v2 = kc.copy(), vc.copy(), kc.copy(), vc.copy()
        for layer in range(sh.layers):
            h = model.layer_forward(layer, k1, v1, 511, cos[511], sin[511], h, threads=8)
            hp = model.layer_forward(layer, k2, v2, 511, cos[511], sin[511], hp, threads=8)
        sensitivity = rel_l2(hp, h.astype(np.float64))
        e_h, e_l = rel_l2(got[0], want[0]), rel_l2(got[1], want[1])
        print(f"fast mode rel-L2: hidden {e_h:.3e} logits {e_l:.3e}; oracle under 1e-6 noise {sensitivity:.3e}")
        bound = min(0.1, 2 * max(sensitivity, FAST_TOLERANCE))
        assert e_h < bound and e_l < bound
