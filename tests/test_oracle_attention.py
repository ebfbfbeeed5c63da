"""The oracle's int8 attention (blocks/src/attention.rs:81-214) and its exponentials
(ops.rs:137-191), pinned by closed forms, the reference's stated error bound, and an f64
attention within the reference's Q7b32 stack tolerance (blocks/tests/stacks.rs:49-55)."""
import math

import numpy as np
import pytest

from oracle import oracle as O

TOL = 3e-2  # relative L2, blocks/tests/stacks.rs:49-55


def f64_attention(H, KV, D, I, Q, K, q, k, v):
    out = np.zeros((I * Q, H * D))
    for im in range(I):
        for h in range(H):
            kh = h // (H // KV)
            qm = q[im * Q:(im + 1) * Q, h * D:(h + 1) * D].astype(np.float64)
            km = k[im * K:(im + 1) * K, kh * D:(kh + 1) * D].astype(np.float64)
            vm = v[im * K:(im + 1) * K, kh * D:(kh + 1) * D].astype(np.float64)
            s = qm @ km.T / math.sqrt(D)
            p = np.exp(s - s.max(1, keepdims=True))
            out[im * Q:(im + 1) * Q, h * D:(h + 1) * D] = (p / p.sum(1, keepdims=True)) @ vm
    return out


def rel_l2(got, want):
    return float(np.linalg.norm(got - want) / np.linalg.norm(want))


def test_exp_fast_within_its_stated_bound_and_fused():
    xs = np.concatenate([np.linspace(-87.0, 0.0, 20001), -np.logspace(-8, 1.9, 2001)]).astype(np.float32)
    got = np.array([O.exp_fast(x) for x in xs], dtype=np.float64)
    want = np.exp(xs.astype(np.float64))
    assert np.max(np.abs(got - want) / want) < 6e-5  # ops.rs:137-139
    assert O.exp_fast(np.float32(0.0)) == 1.0 and O.exp_fast(np.float32(-200.0)) == O.exp_fast(np.float32(-87.0))
    # the same polynomial with each multiply and add rounded separately differs somewhere: the
    # oracle fuses them as the reference's mul_add does
    f = np.float32
    def unfused(x):
        n = f(np.rint(f(x) * f(1.4426950408889634)))
        r = f(f(x) - f(n * f(0.6931471805599453)))
        p = f(1.0 / 24.0)
        for c in (f(1.0 / 6.0), f(0.5), f(1.0), f(1.0)):
            p = f(f(p * r) + c)
        return f(p * np.ldexp(f(1.0), int(n)))
    assert any(unfused(x) != O.exp_fast(x) for x in xs[::97])


@pytest.mark.parametrize("fast", [False, True])
@pytest.mark.parametrize("n", [1, 7, 8, 9, 64, 100])
def test_exponentials_of_equal_scores_sum_to_their_count(fast, n):
    v, total = O.exponentials_apply(np.full(n, 2.5, np.float32), fast)
    assert np.all(v == 1.0) and total == np.float32(n)


@pytest.mark.parametrize("fast", [False, True])
def test_exponentials_keep_the_maximum_at_one_and_sum_their_values(fast):
    rng = np.random.default_rng(5)
    for n in (3, 8, 29, 257):
        s = (rng.standard_normal(n) * 4).astype(np.float32)
        v, total = O.exponentials_apply(s, fast)
        assert v[np.argmax(s)] == 1.0
        tol = 6e-5 if fast else 1e-6
        assert np.allclose(v, np.exp(s.astype(np.float64) - s.max()), rtol=tol, atol=0)
        assert abs(float(total) - math.fsum(map(float, v))) <= 1e-6 * float(total)


CASES = [  # heads, kv_heads, head_dim, images, queries, keys, fast
    (4, 2, 40, 2, 37, 53, False),
    (4, 2, 40, 2, 37, 53, True),
    (2, 2, 64, 1, 70, 200, False),
    (6, 1, 32, 3, 5, 9, True),
    (3, 3, 16, 1, 1, 1, False),
    (8, 2, 128, 1, 33, 300, True),
]


@pytest.mark.parametrize("case", CASES)
def test_attend_matches_f64_attention_within_the_stack_tolerance(case):
    H, KV, D, I, Q, K, fast = case
    rng = np.random.default_rng(sum(case))
    q = rng.standard_normal((I * Q, H * D)).astype(np.float32)
    k = rng.standard_normal((I * K, KV * D)).astype(np.float32)
    v = rng.standard_normal((I * K, KV * D)).astype(np.float32)
    got = O.attend(H, KV, D, I, Q, K, q, k, v, fast=fast)
    assert rel_l2(got, f64_attention(H, KV, D, I, Q, K, q, k, v)) < TOL


def test_attend_reads_heads_of_a_fused_row_by_stride_and_offset():
    H, KV, D, I, Q = 4, 2, 32, 2, 21
    rng = np.random.default_rng(3)
    row = (H + 2 * KV) * D
    qkv = rng.standard_normal((I * Q, row)).astype(np.float32)
    q, k, v = qkv[:, :H * D], qkv[:, H * D:(H + KV) * D], qkv[:, (H + KV) * D:]
    got = O.attend(H, KV, D, I, Q, Q, qkv, qkv, qkv, query_layout=(row, 0), key_layout=(row, H * D),
                   value_layout=(row, (H + KV) * D))
    want = O.attend(H, KV, D, I, Q, Q, np.ascontiguousarray(q), np.ascontiguousarray(k), np.ascontiguousarray(v))
    assert np.array_equal(got, want)
    assert rel_l2(got, f64_attention(H, KV, D, I, Q, Q, q, k, v)) < TOL


def test_attend_removes_the_keys_mean():
    """Softmax ignores a shift of every key by one vector (it adds a constant per query); the
    reference subtracts the keys' mean before quantizing (attention.rs:104-127), so a large
    shift leaves the quantized keys, and the output, almost unchanged."""
    H, KV, D, I, Q, K = 2, 1, 32, 1, 9, 40
    rng = np.random.default_rng(11)
    q = rng.standard_normal((I * Q, H * D)).astype(np.float32)
    k = rng.standard_normal((I * K, KV * D)).astype(np.float32)
    v = rng.standard_normal((I * K, KV * D)).astype(np.float32)
    shift = (rng.standard_normal(KV * D) * 64).astype(np.float32)
    base = O.attend(H, KV, D, I, Q, K, q, k, v)
    moved = O.attend(H, KV, D, I, Q, K, q, (k + shift).astype(np.float32), v)
    assert rel_l2(moved, base) < 1e-3
    assert rel_l2(moved, f64_attention(H, KV, D, I, Q, K, q, k, v)) < TOL
