"""Writes the golden vectors of the quantized product under tests/golden/ from the oracle.

The reference (Rust) cannot run here, so the vectors come from the oracle, whose functions are
pinned by the reference's known answers, closed forms and brute force (tests/test_oracle.py).
They freeze the reference test's own inputs (the LCG of matmul.rs:772-780, 25 x 128 weights,
rows 1 / 3 / 8 / 11: matmul.rs:809-843) and the single-matvec workload (4864 x 896, seed 0) so
that any later change to the oracle or the GPU path is caught against fixed bytes.

    python tests/golden/make_golden.py
"""

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.dirname(os.path.dirname(HERE)), os.path.dirname(HERE)]

from oracle import oracle as O  # noqa: E402
from gpu_data import activations, synthetic_table  # noqa: E402

FORMATS = {"Q7b32": O.Q7B32, "Q4b32": O.Q4B32, "T2b128": O.T2B128, "Q8b32": O.Q8B32}


def pseudo_random(n, seed):
    """matmul.rs:772-780: state = state * 1664525 + 1013904223 (u32); (state >> 8) / 2^24 * 2 - 1."""
    state = seed & 0xFFFFFFFF
    out = np.empty(n, np.float32)
    for i in range(n):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32(state >> 8) / np.float32(1 << 24) * np.float32(2.0) - np.float32(1.0)
    return out


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def lcg_case():
    outputs, width = 25, 128
    arrays = {}
    for name, dtype in FORMATS.items():
        table = O.encode(dtype, outputs, width, pseudo_random(outputs * width, 1))
        arrays[f"{name}/table"] = table
        for rows in (1, 3, 8, 11):
            x = pseudo_random(rows * width, 7 + rows)
            if rows == 3:  # a row of subnormals and zeros
                x[width:2 * width] = 0.0
                x[width + 5] = np.frombuffer(np.uint32(381).tobytes(), np.float32)[0]
                x[width + 70] = -np.frombuffer(np.uint32(94).tobytes(), np.float32)[0]
            q, s, c = O.quantize_rows(x, dtype)
            out, dots = O.matmul(dtype, outputs, width, table, q, s, c, rows, want_dots=True)
            p = f"{name}/rows{rows}/"
            arrays.update({p + "x": x, p + "q": q, p + "scales": s, p + "corrections": c, p + "dots": dots, p + "out": out})
    np.savez_compressed(os.path.join(HERE, "lcg_25x128.npz"), **arrays)


def single_matvec_case():
    """4864 x 896, seed 0 (tests/gpu_data.py's generator): levels uniform in [-127, 127] (Q8b32)
    and [-63, 63] (Q7b32), scales uniform in [1e-3, 1e-2]; x one row ~N(0,1), seed 0."""
    n, k = 4864, 896
    arrays, lines = {}, []
    x = activations(1, k, seed=0).reshape(-1)
    for name in ("Q7b32", "Q8b32"):
        dtype = FORMATS[name]
        table = synthetic_table(dtype, n, k, seed=0)
        q, s, c = O.quantize_rows(x, dtype)
        out, dots = O.matmul(dtype, n, k, table, q, s, c, 1, want_dots=True)
        arrays[f"{name}/table_sha256"] = np.frombuffer(bytes.fromhex(digest(table)), np.uint8)
        arrays[f"{name}/out_sha256"] = np.frombuffer(bytes.fromhex(digest(out)), np.uint8)
        arrays[f"{name}/dots_sha256"] = np.frombuffer(bytes.fromhex(digest(dots)), np.uint8)
        arrays[f"{name}/out_head"] = out.reshape(-1)[:64].copy()
        arrays[f"{name}/q"] = q
        arrays[f"{name}/scales"] = s
        lines.append(f"{name}: out sha256 {digest(out)}")
    np.savez_compressed(os.path.join(HERE, "matvec_4864x896_seed0.npz"), **arrays)
    return lines


if __name__ == "__main__":
    lcg_case()
    for line in single_matvec_case():
        print(line)
