"""Minimal GGUF container reading and writing for the host harness (tests, benchmark).

The reference opens a model with its own GGUF reader and MappedGgufModel
(src/model/gguf.cpp, src/model/mapped_gguf.cpp); a C++ host hands those views to
oq_model_upload directly.  This module gives the Python harness the same
tensor table: the little-endian GGUF v3 layout -- magic "GGUF", version, tensor count,
metadata count, metadata entries (key string, value type, value), tensor infos (name,
dimension count, dimensions, GGML type, offset relative to the data section), padding to
general.alignment (32 by default), tensor data.
"""
from __future__ import annotations

import mmap
import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
DEFAULT_ALIGNMENT = 32


@dataclass
class TensorInfo:
    name: str
    dims: list[int]
    type: int
    relative_offset: int
    absolute_offset: int = 0


@dataclass
class GgufFile:
    version: int
    metadata: dict
    tensors: list[TensorInfo]
    alignment: int
    data_offset: int
    file_size: int
    path: Path | None = None
    _mm: object = field(default=None, repr=False)

    def payload(self) -> np.ndarray:
        """The whole file as read-only bytes (mmap'd; tensor i's bytes start at its absolute_offset)."""
        return np.frombuffer(self._mm, dtype=np.uint8)


class _Reader:
    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, fmt):
        v = struct.unpack_from(fmt, self.buf, self.pos)[0]
        self.pos += struct.calcsize(fmt)
        return v

    def string(self):
        n = self.take("<Q")
        s = bytes(self.buf[self.pos:self.pos + n]).decode("utf-8")
        self.pos += n
        return s

    def value(self, t):
        if t in _SCALAR:
            return self.take(_SCALAR[t])
        if t == 8:
            return self.string()
        if t == 9:
            et, n = self.take("<I"), self.take("<Q")
            return [self.value(et) for _ in range(n)]
        raise ValueError(f"unknown GGUF metadata type {t}")


def read(path) -> GgufFile:
    path = Path(path)
    with open(path, "rb") as fh:
        mm = mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ)
    r = _Reader(mm)
    if bytes(mm[:4]) != b"GGUF":
        raise ValueError("not a GGUF file")
    r.pos = 4
    version = r.take("<I")
    n_tensors, n_kv = r.take("<Q"), r.take("<Q")
    meta = {}
    for _ in range(n_kv):
        key = r.string()
        meta[key] = r.value(r.take("<I"))
    tensors = []
    for _ in range(n_tensors):
        name = r.string()
        nd = r.take("<I")
        dims = [r.take("<Q") for _ in range(nd)]
        t = r.take("<I")
        off = r.take("<Q")
        tensors.append(TensorInfo(name, dims, t, off))
    align = int(meta.get("general.alignment", DEFAULT_ALIGNMENT))
    data_offset = (r.pos + align - 1) // align * align
    for t in tensors:
        t.absolute_offset = data_offset + t.relative_offset
    return GgufFile(version, meta, tensors, align, data_offset, len(mm), path, mm)


def write(path, tensors: list[tuple[str, list[int], int, np.ndarray]], metadata: dict | None = None,
          alignment: int = DEFAULT_ALIGNMENT, offsets: list[int] | None = None) -> None:
    """Writes GGUF v3 with string metadata and the tensors (name, dims, GGML type, bytes) laid out
    in order, each at an offset rounded up to the alignment -- the layout of the reference's test
    fixture writer (tests/test_phase1c.cpp:81-120).  `offsets` overrides the recorded relative
    offsets (the data is still written in order), to build malformed files."""
    meta = {"general.architecture": "oracle-test", "general.alignment": alignment}
    meta.update(metadata or {})
    out = bytearray(b"GGUF")
    out += struct.pack("<IQQ", 3, len(tensors), len(meta))

    def put_string(s):
        b = s.encode()
        out.extend(struct.pack("<Q", len(b)) + b)

    for k, v in meta.items():
        put_string(k)
        if isinstance(v, str):
            out.extend(struct.pack("<I", 8))
            put_string(v)
        else:
            out.extend(struct.pack("<II", 4, int(v)))
    override = offsets
    offsets, off = [], 0
    for _, _, _, data in tensors:
        offsets.append(off)
        off = (off + data.nbytes + alignment - 1) // alignment * alignment
    recorded = offsets if override is None else override
    for (name, dims, t, _), o in zip(tensors, recorded):
        put_string(name)
        out.extend(struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims))
        out.extend(struct.pack("<IQ", t, o))
    out.extend(b"\0" * ((-len(out)) % alignment))
    base = len(out)
    for (_, _, _, data), o in zip(tensors, offsets):
        out.extend(b"\0" * (base + o - len(out)))
        out.extend(np.ascontiguousarray(data).view(np.uint8).tobytes())
    Path(path).write_bytes(bytes(out))
