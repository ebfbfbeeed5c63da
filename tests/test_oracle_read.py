"""The oracle's Reader::read (lm.rs:205-228): rows read in chunks through the stack.

The reference runs every layer over a chunk's rows before the next layer, and each row attends to
the keys up to its own position (Mask::Causal, transformer.rs:185-219). Causality fixes the result:
a chunked read must leave the same caches, the same last row and the same logits, bit for bit, as
decode steps of the same tokens one at a time (or_qwen2_step), whatever the chunk size. That pins
or_qwen2_read against the step the decoder tests already hold to the oracle.
"""

import numpy as np
import pytest

from oracle import oracle as O
from gpu_data import qwen2_model

SMALL = dict(hidden=128, layers=2, heads=4, kv_heads=2, head_dim=32, ffn=256, vocab=96, capacity=40)


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q4B32])
@pytest.mark.parametrize("chunk", [1, 3, 8, 64])
def test_chunked_read_equals_one_step_per_token(dtype, chunk):
    sh, lys, final, table, kc, vc = qwen2_model(dtype, seed=17, synthetic=False, **SMALL)
    model = O.Qwen2(sh, lys, final, table)
    ids = np.random.default_rng(chunk).integers(0, sh.vocab, 11).astype(np.int32)
    first = 5
    k1, v1 = kc.copy(), vc.copy()
    emb = model.embed(ids)
    assert same_bits(emb[3], O.dequantize_row(dtype, sh.vocab, sh.hidden, table, int(ids[3])))
    hidden, logits, token = model.read(k1, v1, emb, first, chunk)
    k2, v2 = kc.copy(), vc.copy()
    for i, t in enumerate(ids):
        h2, l2, t2 = model.step(k2, v2, int(t), first + i)
    assert same_bits(hidden, h2) and same_bits(logits, l2) and token == t2
    assert same_bits(k1, k2) and same_bits(v1, v2)
    # positions before `first` and after the last row are untouched
    assert same_bits(k1[:, :, :first], kc[:, :, :first]) and same_bits(k1[:, :, first + ids.size:], kc[:, :, first + ids.size:])


def test_read_past_the_cache_is_refused():
    sh, lys, final, table, kc, vc = qwen2_model(O.Q7B32, seed=3, synthetic=False, **SMALL)
    model = O.Qwen2(sh, lys, final, table)
    emb = model.embed(np.arange(6, dtype=np.int32))
    with pytest.raises(ValueError, match="holds every key"):
        model.read(kc.copy(), vc.copy(), emb, sh.capacity - 5, 4)
