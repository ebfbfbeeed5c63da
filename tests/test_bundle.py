"""The bundle store's routing on the host (bundle/src/store.rs), with no device table: f32 tensors
and blob parts written in 7-byte pieces (compile/src/writer.rs:117-152), the size checks of
Store::write and Store::end_part, restart_part, and a digest check through a caller's hasher."""

import hashlib

import numpy as np
import pytest


def manifest(parts, tensors):
    return {"parts": parts, "tensors": tensors}


def test_f32_tensors_and_blobs_stream_back():
    from fusor_kernels import Store
    a = np.arange(5, dtype=np.float32)
    b = np.linspace(-1, 1, 7).astype(np.float32)
    blob = b"tokenizer bytes"
    part0 = a.tobytes() + b.tobytes()
    m = manifest([{"file": "w.bin", "bytes": len(part0)}, {"file": "t.json", "bytes": len(blob)}],
                 {"a": {"dtype": 0, "shape": [5], "part": 0, "offset": 0},
                  "b": {"dtype": 0, "shape": [7], "part": 0, "offset": 20}})
    store = Store(m)
    for index, data in ((0, part0), (1, blob)):
        for at in range(0, len(data), 7):
            store.write(index, data[at:at + 7])
        assert not store.complete()
        store.end_part(index)
    assert store.complete()
    assert np.array_equal(store.take("a").bytes().view(np.float32), a)
    assert np.array_equal(store.take("b").bytes().view(np.float32), b)
    assert store.take_blob("t.json") == blob


def test_writes_past_the_end_and_short_parts_fail():
    from fusor_kernels import FormatError, Store
    m = manifest([{"file": "w.bin", "bytes": 8}], {"a": {"dtype": 0, "shape": [2], "part": 0, "offset": 0}})
    store = Store(m)
    store.write(0, b"1234")
    with pytest.raises(FormatError, match="w.bin: 4 of 8 bytes"):
        store.end_part(0)
    with pytest.raises(FormatError, match="w.bin: write past its end"):
        store.write(0, b"12345")
    with pytest.raises(FormatError, match="no part 3: the bundle has 1"):
        store.write(3, b"1")
    with pytest.raises(FormatError, match="is not loaded"):
        store.take("a")
    store.restart_part(0)
    store.write(0, np.array([1.5, 2.5], np.float32).tobytes())
    store.end_part(0)
    assert store.take("a").bytes().view(np.float32).tolist() == [1.5, 2.5]
    with pytest.raises(FormatError, match="missing tensor a"):
        store.take("a")


def test_overlapping_tensors_are_rejected():
    from fusor_kernels import FormatError, Store
    with pytest.raises(FormatError, match="overlap"):
        Store(manifest([{"file": "w.bin", "bytes": 12}], {"a": {"dtype": 0, "shape": [2], "part": 0, "offset": 0},
                                                           "b": {"dtype": 0, "shape": [2], "part": 0, "offset": 4}}))


def test_a_digest_mismatch_is_an_integrity_error():
    """store.rs:138-144, with a caller's hasher (here BLAKE2b standing in for BLAKE3)."""
    from fusor_kernels import IntegrityError, Store
    data = np.arange(4, dtype=np.float32).tobytes()
    good = hashlib.blake2b(data).hexdigest()
    for digest, ok in ((good, True), ("0" * 128, False)):
        store = Store(manifest([{"file": "w.bin", "bytes": 16, "blake3": digest}],
                               {"a": {"dtype": 0, "shape": [4], "part": 0, "offset": 0}}), hasher=hashlib.blake2b)
        for at in range(0, 16, 7):
            store.write(0, data[at:at + 7])
        if ok:
            store.end_part(0)
        else:
            with pytest.raises(IntegrityError):
                store.end_part(0)
