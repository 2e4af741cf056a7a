"""A minimal GGUF reader (and, for the tests, writer) — test infrastructure only.

Reads the header, metadata and tensor directory of a GGUF file, or of every shard of a split model
("-00001-of-0000N.gguf" with split.count), the way the reference's loader addresses tensor data:
(shard, absolute file offset) with the data section at each file's own general.alignment
(core/gguf.hpp:3-60, core/gguf.cpp:89-185). Tensor data stays on disk. The writer produces
single-file GGUF v3 files for the synthetic-model tests.
"""
from __future__ import annotations

import os
import re
import struct
from dataclasses import dataclass, field

GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30
GGML_Q2_0 = 42   # the reference's Q2_0 type id (core/formats.hpp:17)

# bytes per block and values per block of the types the tests read
_BLOCK = {GGML_F32: (4, 1), GGML_F16: (2, 1), GGML_BF16: (2, 1), GGML_Q8_0: (34, 32), GGML_Q2_0: (18, 64)}

# metadata value types
_U8, _I8, _U16, _I16, _U32, _I32, _F32, _BOOL, _STR, _ARR, _U64, _I64, _F64 = range(13)
_SCALAR = {_U8: "<B", _I8: "<b", _U16: "<H", _I16: "<h", _U32: "<I", _I32: "<i", _F32: "<f", _BOOL: "<?",
           _U64: "<Q", _I64: "<q", _F64: "<d"}


@dataclass
class Tensor:
    name: str
    dims: list
    type: int
    shard: int
    file_offset: int

    def nbytes(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        bb, per = _BLOCK[self.type]
        return n // per * bb


@dataclass
class Gguf:
    shards: list = field(default_factory=list)
    meta: dict = field(default_factory=dict)
    tensors: dict = field(default_factory=dict)

    def tensor(self, name: str):
        return self.tensors.get(name)

    def read(self, t: Tensor) -> bytes:
        with open(self.shards[t.shard], "rb") as f:
            f.seek(t.file_offset)
            return f.read(t.nbytes())


class _R:
    def __init__(self, f):
        self.f = f

    def u(self, fmt):
        n = struct.calcsize(fmt)
        b = self.f.read(n)
        if len(b) != n:
            raise ValueError("gguf: truncated file")
        return struct.unpack(fmt, b)[0]

    def s(self):
        n = self.u("<Q")
        return self.f.read(n).decode("utf-8", "replace")

    def value(self, vt):
        if vt in _SCALAR:
            return self.u(_SCALAR[vt])
        if vt == _STR:
            return self.s()
        if vt == _ARR:
            et, n = self.u("<I"), self.u("<Q")
            return [self.value(et) for _ in range(n)]
        raise ValueError(f"gguf: metadata type {vt}")


def _read_shard(g: Gguf, path: str, shard: int) -> None:
    with open(path, "rb") as f:
        r = _R(f)
        if f.read(4) != b"GGUF":
            raise ValueError(f"{path}: not a GGUF file")
        version = r.u("<I")
        if version < 2:
            raise ValueError(f"{path}: GGUF version {version}")
        nt, nkv = r.u("<Q"), r.u("<Q")
        align = 32
        for _ in range(nkv):
            key = r.s()
            v = r.value(r.u("<I"))
            if key == "general.alignment":
                align = int(v)
            g.meta.setdefault(key, v)   # the first shard's value wins
        infos = []
        for _ in range(nt):
            name = r.s()
            nd = r.u("<I")
            dims = [r.u("<Q") for _ in range(nd)]
            ty, off = r.u("<I"), r.u("<Q")
            infos.append((name, dims, ty, off))
        data = (f.tell() + align - 1) // align * align
        for name, dims, ty, off in infos:
            g.tensors[name] = Tensor(name, dims, ty, shard, data + off)


def open_gguf(path: str) -> Gguf:
    """The directory of a GGUF model: `path`, and its sibling shards if it is shard 1 of a split."""
    g = Gguf(shards=[path])
    _read_shard(g, path, 0)
    count = int(g.meta.get("split.count", 1))
    if count > 1:
        m = re.search(r"-00001-of-", path)
        if not m:
            raise ValueError(f"split.count {count} but the name has no -00001-of-: {path}")
        for s in range(2, count + 1):
            p = path[:m.start() + 1] + f"{s:05d}" + path[m.start() + 6:]
            g.shards.append(p)
            _read_shard(g, p, s - 1)
    return g


def write_gguf(path: str, tensors: list, meta: dict | None = None, align: int = 32) -> None:
    """A GGUF v3 file of (name, dims, ggml type, raw bytes) tensors and string / int metadata."""
    def s(x: str) -> bytes:
        b = x.encode()
        return struct.pack("<Q", len(b)) + b

    kv = dict(meta or {})
    kv.setdefault("general.alignment", align)
    head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv)))
    for k, v in kv.items():
        head += s(k)
        if isinstance(v, str):
            head += struct.pack("<I", _STR) + s(v)
        else:
            head += struct.pack("<I", _U32) + struct.pack("<I", int(v))
    off = 0
    offs = []
    for name, dims, ty, raw in tensors:
        offs.append(off)
        head += s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ty, off)
        off += (len(raw) + align - 1) // align * align
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * ((-len(head)) % align))
        for (_, _, _, raw), o in zip(tensors, offs):
            f.write(raw)
            f.write(b"\0" * ((-len(raw)) % align))
    assert os.path.getsize(path) > 0
