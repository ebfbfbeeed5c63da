"""Tables streamed onto the device as a bundle store receives them (fg_upload_*, Store).

The reference's round-trip test pushes every part in 7-byte writes (compile/src/writer.rs:117-152)
through Store::write (bundle/src/store.rs:90-126). Here the same writes land on the device: the
table's bytes read back are the reference bytes, and its products are the oracle's to the bit.
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


def pieces(n, rng, lo=1, hi=1 << 20):
    """Ragged piece sizes covering n bytes: log-uniform between lo and hi, with empty pieces."""
    out, at = [], 0
    while at < n:
        size = 0 if rng.random() < 0.05 else int(np.exp(rng.uniform(np.log(lo), np.log(hi))))
        size = min(size, n - at)
        out.append((at, size))
        at += size
    return out


def stream(fk, dtype, rows, cols, data, sizes):
    up = fk.TableUpload(dtype, [rows, cols])
    for at, size in sizes:
        up.write(data[at:at + size])
    return up.end()


def check_table(fk, t, dtype, rows, cols, data, row_sets=(1, 40)):
    import torch
    assert np.array_equal(t.reference_bytes(), data)
    width = (rows + 3) // 4 * 4
    for r in row_sets:
        x = activations(r, cols, seed=r + cols)
        got = fk.matmul(t.matrix(), fk.Input(f32=torch.from_numpy(x.reshape(-1)).cuda()), range(0, width))
        torch.cuda.synchronize()
        q, s, c = O.quantize_rows(x.reshape(-1), dtype)
        want = O.matmul(dtype, rows, cols, data, q, s, c, r)
        assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dtype", [O.Q7B32, O.Q8B32, O.Q4B32, O.T2B128])
def test_seven_byte_writes(fk, dtype):
    """A 4864 x 896 table (4.9 MB for Q7b32: more than one staging buffer per format but T2b128)
    in 7-byte writes, the reference test's piece size; a ragged row count (the padding quad)."""
    rows, cols = (4863, 896) if dtype != O.T2B128 else (4863, 1024)
    print(f"seven-byte upload dtype {dtype}", flush=True)
    data = synthetic_table(dtype, rows, cols, seed=dtype)
    n = data.size
    t = stream(fk, dtype, rows, cols, data, [(at, min(7, n - at)) for at in range(0, n, 7)])
    check_table(fk, t, dtype, rows, cols, data)


def test_head_table_in_seven_byte_and_ragged_pieces(fk):
    """The 151936 x 896 Q7b32 head table (153 MB, 19 staging buffers): 7-byte writes over its
    first and last 3 MB (the start, the codes' end and the scales, the end of the table) and
    ragged pieces from 1 byte to 1 MiB between them."""
    rows, cols = 151936, 896
    data = synthetic_table(O.Q7B32, rows, cols, seed=11)
    n, codes_end = data.size, O.quant_len(O.Q7B32, rows, cols)
    rng = np.random.default_rng(5)
    head, tail = 3 << 20, codes_end - (1 << 20)
    sizes = [(at, min(7, head - at)) for at in range(0, head, 7)]
    sizes += [(head + a, s) for a, s in pieces(tail - head, rng)]
    sizes += [(at, min(7, n - at)) for at in range(tail, n, 7)]
    assert sum(s for _, s in sizes) == n
    t = stream(fk, O.Q7B32, rows, cols, data, sizes)
    check_table(fk, t, O.Q7B32, rows, cols, data, row_sets=(1, 5))


@pytest.mark.parametrize("dtype", [O.Q4B32, O.Q8B32])
def test_ragged_pieces_and_whole_writes(fk, dtype):
    rows, cols = 14336, 512
    data = synthetic_table(dtype, rows, cols, seed=3)
    rng = np.random.default_rng(dtype)
    check_table(fk, stream(fk, dtype, rows, cols, data, pieces(data.size, rng)), dtype, rows, cols, data)
    check_table(fk, stream(fk, dtype, rows, cols, data, [(0, data.size)]), dtype, rows, cols, data)


def test_upload_errors_and_restart(fk):
    rows, cols = 64, 256
    data = synthetic_table(O.Q7B32, rows, cols, seed=4)
    up = fk.TableUpload(O.Q7B32, [rows, cols])
    up.write(data[:1000])
    with pytest.raises(fk.FormatError, match=r"table upload: 1000 of \d+ bytes"):
        up.end()
    up.restart()  # store.rs:148-158: written again from byte 0
    up.write(data)
    with pytest.raises(fk.FormatError, match="write past its end"):
        up.write(b"x")
    t = up.end()
    check_table(fk, t, O.Q7B32, rows, cols, data, row_sets=(1,))
    with pytest.raises(fk.FormatError, match="whole groups of 128"):
        fk.TableUpload(O.T2B128, [4, 64])


def test_restart_after_staging_flushes(fk):
    """A restart once more than one 8 MiB staging buffer has gone to the device (copies in flight,
    codes already re-laid out, the second buffer in use): a 4864 x 2048 Q7b32 table (10.0 MB) written
    whole, restarted, then written again in ragged pieces; and the same through a Store's
    restart_part (store.rs:148-158) on a part holding that table and a bias."""
    rows, cols = 4864, 2048
    print(f"upload restart after flushes {rows} x {cols}", flush=True)
    data = synthetic_table(O.Q7B32, rows, cols, seed=21)
    rng = np.random.default_rng(22)
    up = fk.TableUpload(O.Q7B32, [rows, cols])
    up.write(data[: 9 << 20])
    up.write(data[9 << 20:])
    up.restart()
    for at, size in pieces(data.size, rng):
        up.write(data[at:at + size])
    check_table(fk, up.end(), O.Q7B32, rows, cols, data, row_sets=(1, 17))

    bias = rng.standard_normal(rows).astype(np.float32)
    other = synthetic_table(O.Q7B32, rows, cols, seed=23)  # the first attempt's bytes differ
    part = data.tobytes() + bias.tobytes()
    manifest = {"parts": [{"file": "w.bin", "bytes": len(part)}],
                "tensors": {"w": {"dtype": O.Q7B32, "shape": [rows, cols], "part": 0, "offset": 0},
                            "b": {"dtype": 0, "shape": [rows], "part": 0, "offset": data.size}}}
    store = fk.Store(manifest)
    first = other.tobytes() + bias.tobytes()
    for at, size in pieces(len(first) - 1000, rng):
        store.write(0, first[at:at + size])
    store.restart_part(0)
    for at, size in pieces(len(part), rng):
        store.write(0, part[at:at + size])
    store.end_part(0)
    check_table(fk, store.take("w"), O.Q7B32, rows, cols, data, row_sets=(1,))
    assert np.array_equal(store.take("b").bytes(), bias.view(np.uint8))


def test_store_streams_a_bundle_into_device_tables(fk):
    """compile/src/writer.rs:117-152 through the device: one part holding an f32 norm and a
    Q7b32 weight back to back, a blob part, every part pushed in 7-byte writes; then a second
    model-shaped part of two tables and a bias in ragged writes."""
    import torch
    norm = np.array([1.0, 2.0, 3.0], np.float32)
    values = ((np.arange(3 * 64, dtype=np.float32) - 90.0) / 9.0).reshape(3, 64)
    weight = O.encode(O.Q7B32, 3, 64, values)
    blob = b'{"a": 1}'
    qkv = synthetic_table(O.Q7B32, 1152, 896, seed=1)
    down = synthetic_table(O.Q4B32, 896, 4864, seed=2)
    bias = np.random.default_rng(3).standard_normal(1152).astype(np.float32)
    part0 = norm.tobytes() + weight.tobytes()
    part2 = qkv.tobytes() + bias.tobytes() + down.tobytes()
    manifest = {
        "parts": [{"file": "weights.bin", "bytes": len(part0)}, {"file": "vocab.json", "bytes": len(blob)},
                  {"file": "layer.bin", "bytes": len(part2)}],
        "tensors": {
            "norm": {"dtype": 0, "shape": [3], "part": 0, "offset": 0},
            "weight": {"dtype": O.Q7B32, "shape": [3, 64], "part": 0, "offset": 12},
            "qkv": {"dtype": O.Q7B32, "shape": [1152, 896], "part": 2, "offset": 0},
            "qkv_bias": {"dtype": 0, "shape": [1152], "part": 2, "offset": qkv.size},
            "down": {"dtype": O.Q4B32, "shape": [896, 4864], "part": 2, "offset": qkv.size + 4 * 1152},
        },
    }
    store = fk.Store(manifest)
    for index, data in ((0, part0), (1, blob)):
        for at in range(0, len(data), 7):
            store.write(index, data[at:at + 7])
        store.end_part(index)
    rng = np.random.default_rng(9)
    for at, size in pieces(len(part2), rng, hi=1 << 18):
        store.write(2, part2[at:at + size])
    with pytest.raises(fk.FormatError, match="is not loaded"):
        store.take("qkv")
    store.end_part(2)
    assert store.complete()
    assert np.array_equal(store.take("norm").bytes(), norm.view(np.uint8))
    assert np.array_equal(store.take("weight").reference_bytes(), weight)
    assert store.take_blob("vocab.json") == blob
    check_table(fk, store.take("qkv"), O.Q7B32, 1152, 896, qkv, row_sets=(1, 17))
    check_table(fk, store.take("down"), O.Q4B32, 896, 4864, down, row_sets=(1, 17))
    assert np.array_equal(store.take("qkv_bias").bytes(), bias.view(np.uint8))
    with pytest.raises(fk.FormatError, match="missing tensor"):
        store.take("qkv")
    torch.cuda.synchronize()
