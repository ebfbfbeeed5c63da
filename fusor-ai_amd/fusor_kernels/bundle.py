"""A bundle's parts streamed into tensors, the quantized tables straight onto the device.

`Store` keeps bundle::Store's interface (bundle/src/store.rs): `write(part, bytes)` takes the next
bytes of a part, in order, and routes each range to the tensor or blob that owns it;
`end_part(part)` checks that the part is complete; `take(name)` hands a tensor out. What changes is
where a quantized table's bytes go: into a `TableUpload` (fg_upload_*), which streams them to the
device as they arrive, so `take` returns a device `Table` with no whole-table host copy. f32
tensors and blob parts stay on the host, as the reference keeps them.

The manifest (bundle/src/manifest.rs:8-44) is given as plain data: a list of parts
(`{"file", "bytes"}`) and a dict of tensors (`{name: {"dtype", "shape", "part", "offset"}}`). A
part's BLAKE3 digest is checked only when a `hasher` factory (an object with `update` and
`hexdigest`) is given and the part names a digest: the Python standard library has no BLAKE3, and
a host binding keeps the reference Store's own hashing.
"""

from bisect import bisect_right

from ._lib import Error, FormatError
from .tensor import DType, Tensor, TableUpload, byte_len


class IntegrityError(Error):
    """Error::Integrity: a part whose digest is not the manifest's."""


class _Slot:
    __slots__ = ("offset", "len", "name", "sink")

    def __init__(self, offset, length, name, sink):
        self.offset, self.len, self.name, self.sink = offset, length, name, sink


class Store:
    def __init__(self, manifest, hasher=None, stream=None):
        """Store::new (store.rs:49-88): every tensor's sink, the routing table of every part."""
        self.parts = list(manifest["parts"])
        self._hasher, self._stream = hasher, stream
        self._slots = [[] for _ in self.parts]
        holds = [False] * len(self.parts)
        for name, entry in manifest["tensors"].items():
            part = entry["part"]
            if not 0 <= part < len(self.parts):
                raise FormatError(f"{name}: no part {part}")
            dtype, shape = DType(entry["dtype"]), list(entry["shape"])
            size = byte_len(dtype, shape)
            self._slots[part].append(_Slot(int(entry["offset"]), size, name, (dtype, shape)))
            holds[part] = True
        self._blobs = {i: bytearray() for i, h in enumerate(holds) if not h}
        for i in self._blobs:
            self._slots[i].append(_Slot(0, int(self.parts[i]["bytes"]), None, None))
        for i, slots in enumerate(self._slots):
            slots.sort(key=lambda s: s.offset)
            end = 0
            for s in slots:  # check_layout: slots in the part, none overlapping
                if s.offset < end or s.offset + s.len > int(self.parts[i]["bytes"]):
                    raise FormatError(f"{self.parts[i]['file']}: tensors overlap or run past the part")
                end = s.offset + s.len
        self._starts = [[s.offset for s in slots] for slots in self._slots]
        for slots in self._slots:
            for s in slots:
                if s.name is not None:
                    s.sink = _TensorSink(*s.sink, stream)
        self._progress = [self._fresh() for _ in self.parts]

    def _fresh(self):
        return {"received": 0, "done": False, "hash": self._hasher() if self._hasher else None}

    def _part(self, part):
        if not 0 <= part < len(self.parts):
            raise FormatError(f"no part {part}: the bundle has {len(self.parts)}")
        return self.parts[part], self._progress[part]

    def write(self, part, data):
        """The next bytes of part `part` (store.rs:90-126): writes arrive in order."""
        entry, progress = self._part(part)
        data = memoryview(data).cast("B")
        start = progress["received"]
        end = start + data.nbytes
        if progress["done"] or end > int(entry["bytes"]):
            raise FormatError(f"{entry['file']}: write past its end")
        if progress["hash"] is not None:
            progress["hash"].update(data)
        progress["received"] = end
        slots = self._slots[part]
        first = max(0, bisect_right(self._starts[part], start) - 1)
        for s in slots[first:]:
            if s.offset >= end:
                break
            lo, hi = max(start, s.offset), min(end, s.offset + s.len)
            if lo >= hi:
                continue
            piece = data[lo - start:hi - start]
            if s.name is None:
                self._blobs[part].extend(piece)
            else:
                s.sink.write(piece)

    def end_part(self, part):
        """store.rs:129-146: the part's size (and digest), then its tables finished on the device."""
        entry, progress = self._part(part)
        if progress["received"] != int(entry["bytes"]):
            raise FormatError(f"{entry['file']}: {progress['received']} of {entry['bytes']} bytes")
        want = entry.get("blake3")
        if progress["hash"] is not None and want:
            got = progress["hash"].hexdigest()
            if got != want:
                raise IntegrityError(f"{entry['file']}: BLAKE3 {got} ≠ {want}")
        for s in self._slots[part]:
            if s.name is not None:
                s.sink.finish()
        progress["done"] = True

    def restart_part(self, part):
        """store.rs:148-158: forget what was written to the part."""
        self._part(part)
        for s in self._slots[part]:
            if s.name is not None:
                s.sink.restart()
        if part in self._blobs:
            self._blobs[part].clear()
        self._progress[part] = self._fresh()

    def complete(self):
        return all(p["done"] for p in self._progress)

    def take(self, name):
        """A tensor of a part that was ended: a device `Table` for a quantized matrix, else a host
        `Tensor`."""
        for part, slots in enumerate(self._slots):
            for s in slots:
                if s.name == name and not s.sink.taken:
                    if not self._progress[part]["done"]:
                        raise FormatError(f"{name} is not loaded")
                    return s.sink.take()
        raise FormatError(f"missing tensor {name}")

    def take_blob(self, file):
        for i, entry in enumerate(self.parts):
            if entry["file"] == file:
                if not self._progress[i]["done"]:
                    raise FormatError(f"{file} is not loaded")
                if i not in self._blobs:
                    raise FormatError(f"{file} holds tensors")
                return bytes(self._blobs.pop(i))
        raise FormatError(f"no part {file}")


class _TensorSink:
    """Where one tensor's bytes go: a device upload for a quantized matrix, host bytes otherwise.
    The upload (and its staging buffers) exists only while the tensor's bytes arrive: it starts
    at the first piece and ends at the last, so a part of many tables holds one upload at a time.
    The table is handed out only once its part has ended."""

    def __init__(self, dtype, shape, stream):
        self.dtype, self.shape, self.taken = dtype, shape, False
        self._stream = stream
        self._quantized = dtype.quant_format() is not None and len(shape) == 2
        self._size = byte_len(dtype, shape)
        self._received = 0
        self._upload = self._result = None
        self._host = bytearray()

    def write(self, piece):
        if not self._quantized:
            self._host.extend(piece)
            return
        if self._upload is None:
            self._upload = TableUpload(self.dtype, self.shape, self._stream)
        self._upload.write(piece)
        self._received += memoryview(piece).nbytes
        if self._received == self._size:
            self._result, self._upload = self._upload.end(), None

    def restart(self):
        self._upload = self._result = None  # an unfinished upload is freed with its object
        self._received = 0
        self._host.clear()

    def finish(self):
        if self._quantized and self._result is None:  # a table of no bytes
            self._result = TableUpload(self.dtype, self.shape, self._stream).end()

    def take(self):
        import numpy as np
        self.taken = True
        if self._quantized:
            return self._result
        return Tensor(self.dtype, self.shape, np.frombuffer(bytes(self._host), np.uint8).copy())
