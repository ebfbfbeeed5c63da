"""The committed golden vectors (tests/golden/make_golden.py) against the oracle on the CPU, and
their inputs against the reference test's generator (matmul.rs:772-780)."""

import hashlib
import os

import numpy as np
import pytest

from oracle import oracle as O
from gpu_data import activations, synthetic_table

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FORMATS = {"Q7b32": O.Q7B32, "Q4b32": O.Q4B32, "T2b128": O.T2B128, "Q8b32": O.Q8B32}


def load(name):
    with np.load(os.path.join(GOLDEN, name)) as z:
        return {k: z[k] for k in z.files}


def lcg(n, seed):
    state = seed & 0xFFFFFFFF
    out = np.empty(n, np.float32)
    for i in range(n):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32(state >> 8) / np.float32(1 << 24) * np.float32(2.0) - np.float32(1.0)
    return out


def test_golden_inputs_are_the_reference_test_inputs():
    g = load("lcg_25x128.npz")
    # first values of the LCG at seed 1 worked by hand: state_1 = 1664525 + 1013904223
    s1 = (1664525 + 1013904223) & 0xFFFFFFFF
    assert lcg(1, 1)[0] == np.float32(s1 >> 8) / np.float32(1 << 24) * np.float32(2.0) - np.float32(1.0)
    for rows in (1, 8, 11):
        assert np.array_equal(g[f"Q7b32/rows{rows}/x"], lcg(rows * 128, 7 + rows))
    x3 = g["Q7b32/rows3/x"]
    assert np.array_equal(x3[:128], lcg(384, 10)[:128]) and np.array_equal(x3[256:], lcg(384, 10)[256:])


@pytest.mark.parametrize("name", list(FORMATS))
def test_oracle_reproduces_the_golden_lcg_vectors(name):
    g = load("lcg_25x128.npz")
    dtype = FORMATS[name]
    table = O.encode(dtype, 25, 128, lcg(25 * 128, 1))
    assert np.array_equal(table, g[f"{name}/table"])
    for rows in (1, 3, 8, 11):
        p = f"{name}/rows{rows}/"
        q, s, c = O.quantize_rows(g[p + "x"], dtype)
        assert np.array_equal(q, g[p + "q"])
        assert np.array_equal(s.view(np.uint32), g[p + "scales"].view(np.uint32))
        assert np.array_equal(c, g[p + "corrections"])
        out, dots = O.matmul(dtype, 25, 128, table, q, s, c, rows, want_dots=True)
        assert np.array_equal(dots, g[p + "dots"])
        assert np.array_equal(out.view(np.uint32), g[p + "out"].view(np.uint32))


@pytest.mark.parametrize("name", ["Q7b32", "Q8b32"])
def test_oracle_reproduces_the_single_matvec_digest(name):
    g = load("matvec_4864x896_seed0.npz")
    dtype = FORMATS[name]
    table = synthetic_table(dtype, 4864, 896, seed=0)
    assert hashlib.sha256(table.tobytes()).digest() == g[f"{name}/table_sha256"].tobytes()
    x = activations(1, 896, seed=0).reshape(-1)
    q, s, c = O.quantize_rows(x, dtype)
    out, dots = O.matmul(dtype, 4864, 896, table, q, s, c, 1, want_dots=True)
    assert hashlib.sha256(out.tobytes()).digest() == g[f"{name}/out_sha256"].tobytes()
    assert hashlib.sha256(dots.tobytes()).digest() == g[f"{name}/dots_sha256"].tobytes()
    assert np.array_equal(out.reshape(-1)[:64].view(np.uint32), g[f"{name}/out_head"].view(np.uint32))
