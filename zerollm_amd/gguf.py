"""GGUF container: reader (metadata, tensor infos, memory-mapped tensor data) and writer.

Mirrors zerollm's `readGGUF` / `GGUFFile` (src/gguf/reader.js:106-190) and the type table
(src/gguf/types.js:4-73), and its writer `buildGGUF` / `writeGGUF` (tools/gguf-writer.js:52-115). The
native loader in zerollm_amd/csrc/gguf.cpp parses the same format independently; this module is the host
side (metadata questions such as vocabulary compatibility, test fixtures, synthetic models).
"""
from __future__ import annotations

import os
import struct
from dataclasses import dataclass, field

import numpy as np

# GGUF metadata value types (src/gguf/types.js:4-7)
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)

# ggml tensor type ids (src/gguf/types.js:10-15)
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1 = 0, 1, 2, 3, 6, 7, 8, 9
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K = 10, 11, 12, 13, 14, 15
BF16 = 30

# (name, elements per block, bytes per block) (src/gguf/types.js:24-54)
TYPE_INFO = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20), 6: ("Q5_0", 32, 22),
    7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 9: ("Q8_1", 32, 36), 10: ("Q2_K", 256, 84), 11: ("Q3_K", 256, 110),
    12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210), 15: ("Q8_K", 256, 292),
    16: ("IQ2_XXS", 256, 66), 17: ("IQ2_XS", 256, 74), 18: ("IQ3_XXS", 256, 98), 19: ("IQ1_S", 256, 50),
    20: ("IQ4_NL", 32, 18), 21: ("IQ3_S", 256, 110), 22: ("IQ2_S", 256, 82), 23: ("IQ4_XS", 256, 136),
    24: ("I8", 1, 1), 25: ("I16", 1, 2), 26: ("I32", 1, 4), 27: ("I64", 1, 8), 28: ("F64", 1, 8),
    29: ("IQ1_M", 256, 56), 30: ("BF16", 1, 2),
}
TYPE_ID = {v[0]: k for k, v in TYPE_INFO.items()}

MAX_STRING = 1 << 30
MAX_ARRAY = 1 << 28


def type_name(t: int) -> str:
    return TYPE_INFO[t][0] if t in TYPE_INFO else f"type{t}"


def row_size(t: int, ne0: int) -> int:
    """Bytes in one row of ne0 elements (src/gguf/types.js:60-65)."""
    if t not in TYPE_INFO:
        raise ValueError(f"unknown ggml type id {t}")
    name, bs, ts = TYPE_INFO[t]
    if ne0 % bs:
        raise ValueError(f"row length {ne0} is not a multiple of block size {bs} for {name}")
    return ne0 // bs * ts


def tensor_bytes(t: int, dims) -> int:
    rows = 1
    for d in dims[1:]:
        rows *= d
    return row_size(t, dims[0] if dims else 1) * rows


@dataclass
class TensorInfo:
    name: str
    dims: list
    type: int
    offset: int
    abs_offset: int = 0
    n_elements: int = 0
    n_bytes: int | None = None


@dataclass
class GGUFFile:
    path: str
    file_size: int
    version: int
    metadata: dict
    tensors: list
    alignment: int
    data_start: int
    tensor_map: dict = field(default_factory=dict)

    def get(self, key, default=None):
        return self.metadata.get(key, default)

    def tensor(self, name):
        return self.tensor_map.get(name)

    def require_tensor(self, name):
        t = self.tensor_map.get(name)
        if t is None:
            raise KeyError(f"tensor not found in GGUF: {name}")
        return t

    def data(self, name) -> np.ndarray:
        """Raw bytes of a tensor as a read-only uint8 view over a memory map of the file."""
        t = self.require_tensor(name)
        if t.n_bytes is None:
            raise ValueError(f"tensor {name}: unknown type {t.type}")
        mm = np.memmap(self.path, dtype=np.uint8, mode="r", offset=t.abs_offset, shape=(t.n_bytes,))
        return mm

    def floats(self, name) -> np.ndarray:
        t = self.require_tensor(name)
        if t.type != F32:
            raise ValueError(f"tensor {name} is {type_name(t.type)}, expected F32")
        return np.frombuffer(self.data(name), dtype="<f4")


class _Cursor:
    def __init__(self, f, size):
        self.f = f
        self.size = size
        self.pos = 0

    def take(self, n):
        if self.pos + n > self.size:
            raise ValueError(f"GGUF: unexpected end of file at byte {self.pos} (need {n} more, file is {self.size} bytes)")
        b = self.f.read(n)
        if len(b) != n:
            raise ValueError("GGUF: short read")
        self.pos += n
        return b

    def unpack(self, fmt):
        return struct.unpack("<" + fmt, self.take(struct.calcsize("<" + fmt)))[0]

    def string(self):
        n = self.unpack("Q")
        if n > MAX_STRING:
            raise ValueError(f"GGUF: implausible string length {n}")
        return self.take(n).decode("utf-8", errors="replace")


_SCALAR = {UINT8: "B", INT8: "b", UINT16: "H", INT16: "h", UINT32: "I", INT32: "i", FLOAT32: "f",
           UINT64: "Q", INT64: "q", FLOAT64: "d"}


def _read_value(c: _Cursor, t: int):
    if t in _SCALAR:
        return c.unpack(_SCALAR[t])
    if t == BOOL:
        return c.unpack("B") != 0
    if t == STRING:
        return c.string()
    if t == ARRAY:
        et = c.unpack("I")
        n = c.unpack("Q")
        if n > MAX_ARRAY:
            raise ValueError(f"GGUF: implausible array length {n}")
        if et in _SCALAR:
            fmt = "<%d%s" % (n, _SCALAR[et])
            return list(struct.unpack(fmt, c.take(struct.calcsize(fmt))))
        return [_read_value(c, et) for _ in range(n)]
    raise ValueError(f"GGUF: unknown metadata value type {t}")


def read_gguf(path: str) -> GGUFFile:
    """Parse header, metadata and tensor infos (src/gguf/reader.js:136-190)."""
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        c = _Cursor(f, size)
        magic = c.take(4)
        if magic != b"GGUF":
            raise ValueError(f"not a GGUF file (magic {magic!r})")
        version = c.unpack("I")
        if version < 2 or version > 3:
            raise ValueError(f"unsupported GGUF version {version} (expected 2 or 3)")
        n_tensors = c.unpack("Q")
        n_kv = c.unpack("Q")
        if n_tensors > 1_000_000 or n_kv > 1_000_000:
            raise ValueError("GGUF: implausible tensor/metadata count (corrupt file?)")
        meta = {}
        for _ in range(n_kv):
            key = c.string()
            t = c.unpack("I")
            meta[key] = _read_value(c, t)
        alignment = meta.get("general.alignment", 32)
        if not isinstance(alignment, int) or alignment <= 0:
            raise ValueError(f"GGUF: bad general.alignment {alignment}")
        raw = []
        for _ in range(n_tensors):
            name = c.string()
            nd = c.unpack("I")
            if nd < 1 or nd > 8:
                raise ValueError(f"GGUF: tensor {name} has {nd} dims")
            dims = [c.unpack("Q") for _ in range(nd)]
            t = c.unpack("I")
            off = c.unpack("Q")
            raw.append(TensorInfo(name, dims, t, off))
        data_start = (c.pos + alignment - 1) // alignment * alignment
    for ti in raw:
        ti.n_elements = int(np.prod(ti.dims))
        ti.n_bytes = tensor_bytes(ti.type, ti.dims) if ti.type in TYPE_INFO else None
        ti.abs_offset = data_start + ti.offset
        if ti.n_bytes is not None and ti.abs_offset + ti.n_bytes > size:
            raise ValueError(f"GGUF: tensor {ti.name} extends past end of file (truncated download?): needs bytes up to "
                             f"{ti.abs_offset + ti.n_bytes}, file has {size}")
    g = GGUFFile(path, size, version, meta, raw, alignment, data_start)
    g.tensor_map = {t.name: t for t in raw}
    return g


# ----------------------------------------------------------------------------------------------- writer

class MetaKV:
    def __init__(self, key, type_, value, elem_type=None):
        self.key, self.type, self.value, self.elem_type = key, type_, value, elem_type


def _write_value(out: list, t: int, v, et=None):
    if t in _SCALAR:
        out.append(struct.pack("<" + _SCALAR[t], v))
    elif t == BOOL:
        out.append(struct.pack("<B", 1 if v else 0))
    elif t == STRING:
        b = v.encode("utf-8")
        out.append(struct.pack("<Q", len(b)))
        out.append(b)
    elif t == ARRAY:
        out.append(struct.pack("<IQ", et, len(v)))
        if et in _SCALAR:
            out.append(struct.pack("<%d%s" % (len(v), _SCALAR[et]), *v))
        else:
            for x in v:
                _write_value(out, et, x)
    else:
        raise ValueError(f"writer: unsupported value type {t}")


def write_gguf(path: str, metadata: list, tensors: list, alignment: int = 32, version: int = 3):
    """Write a GGUF file; tensors = [(name, dims, type, uint8 ndarray or bytes)] (tools/gguf-writer.js:66-115).
    Tensor data is streamed, so large models are written without a second in-memory copy."""
    meta = list(metadata)
    if alignment != 32 and not any(m.key == "general.alignment" for m in meta):
        meta.append(MetaKV("general.alignment", UINT32, alignment))
    head = [b"GGUF", struct.pack("<IQQ", version, len(tensors), len(meta))]
    for m in meta:
        _write_value(head, STRING, m.key)
        head.append(struct.pack("<I", m.type))
        _write_value(head, m.type, m.value, m.elem_type)
    off = 0
    offsets = []
    for name, dims, t, data in tensors:
        if t not in TYPE_INFO:
            raise ValueError(f"writer: unknown type {t}")
        expect = tensor_bytes(t, dims)
        n = len(data) if isinstance(data, (bytes, bytearray)) else data.nbytes
        if n != expect:
            raise ValueError(f"writer: tensor {name} has {n} bytes, expected {expect}")
        off = (off + alignment - 1) // alignment * alignment
        offsets.append(off)
        off += n
        _write_value(head, STRING, name)
        head.append(struct.pack("<I", len(dims)))
        head.append(struct.pack("<%dQ" % len(dims), *dims))
        head.append(struct.pack("<IQ", t, offsets[-1]))
    hb = b"".join(head)
    pad = (-len(hb)) % alignment
    hb += b"\0" * pad
    data_start = len(hb)
    with open(path, "wb") as f:
        f.write(hb)
        pos = data_start
        for (name, dims, t, data), o in zip(tensors, offsets):
            want = data_start + o
            if pos < want:
                f.write(b"\0" * (want - pos))
                pos = want
            buf = data if isinstance(data, (bytes, bytearray)) else np.ascontiguousarray(data).view(np.uint8).reshape(-1)
            f.write(buf if isinstance(buf, (bytes, bytearray)) else buf.tobytes())
            pos += len(buf)
