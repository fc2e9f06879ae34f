"""GGUF v3 reader and writer.

``open_gguf(path)`` mirrors openGGUF (src/gguf.js:17-83): it parses the
header, the key/value metadata (dropping tokenizer.* arrays as the reference
does) and the tensor table, aligns the data start to general.alignment
(default 32), and returns an object whose ``fetch(name)`` gives
``{name, dims, type, offset, buf}``.  The file is memory-mapped, so fetching a
tensor reads only its bytes.  ``write_gguf`` produces files in the same
format (used for synthetic models and tests).
"""
from __future__ import annotations

import struct

import numpy as np

from .formats import tensor_bytes

# value type ids of the GGUF spec
_U8, _I8, _U16, _I16, _U32, _I32, _F32, _BOOL, _STR, _ARR, _U64, _I64, _F64 = range(13)
_SCALAR = {_U8: "<B", _I8: "<b", _U16: "<H", _I16: "<h", _U32: "<I", _I32: "<i", _F32: "<f", _BOOL: "<?",
           _U64: "<Q", _I64: "<q", _F64: "<d"}


class GGUFError(ValueError):
    pass


class GGUFFile:
    def __init__(self, path: str, kv: dict, tensors: dict, data_start: int, mm: np.memmap):
        self.path, self.kv, self.tensors, self.data_start, self._mm = path, kv, tensors, data_start, mm

    def fetch(self, name: str) -> dict:
        t = self.tensors.get(name)
        if t is None:
            raise GGUFError(f"no tensor {name}")
        start = self.data_start + t["offset"]
        n = tensor_bytes(t["type"], t["dims"])
        if start + n > self._mm.size:
            raise GGUFError(f"tensor {name} extends past the end of the file")
        return dict(t, buf=self._mm[start:start + n])


def open_gguf(path: str) -> GGUFFile:
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    off = 0

    def take(n):
        nonlocal off
        if off + n > mm.size:
            raise GGUFError("truncated GGUF header")
        b = mm[off:off + n].tobytes()
        off += n
        return b

    def u32():
        return struct.unpack("<I", take(4))[0]

    def u64():
        return struct.unpack("<Q", take(8))[0]

    def string():
        return take(u64()).decode("utf-8")

    def value(t):
        if t == _STR:
            return string()
        if t == _ARR:
            et, n = u32(), u64()
            return [value(et) for _ in range(n)]
        fmt = _SCALAR.get(t)
        if fmt is None:
            raise GGUFError(f"unknown GGUF value type {t}")
        return struct.unpack(fmt, take(struct.calcsize(fmt)))[0]

    if take(4) != b"GGUF":
        raise GGUFError("not GGUF")
    version = u32()
    if version not in (2, 3):
        raise GGUFError(f"unsupported GGUF version {version}")
    n_tensors, n_kv = u64(), u64()
    kv = {}
    for _ in range(n_kv):
        k = string()
        t = u32()
        v = value(t)
        if not k.startswith("tokenizer."):
            kv[k] = v
    align = int(kv.get("general.alignment", 32))
    tensors = {}
    for _ in range(n_tensors):
        name = string()
        nd = u32()
        dims = [u64() for _ in range(nd)]
        typ = u32()
        offset = u64()
        tensors[name] = {"name": name, "dims": dims, "type": typ, "offset": offset}
    data_start = (off + align - 1) // align * align
    return GGUFFile(path, kv, tensors, data_start, mm)


def _pack_value(v):
    if isinstance(v, bool):
        return struct.pack("<I", _BOOL) + struct.pack("<?", v)
    if isinstance(v, int):
        return struct.pack("<I", _I64 if v < 0 else _U64) + struct.pack("<q" if v < 0 else "<Q", v)
    if isinstance(v, float):
        return struct.pack("<I", _F32) + struct.pack("<f", v)
    if isinstance(v, str):
        b = v.encode("utf-8")
        return struct.pack("<I", _STR) + struct.pack("<Q", len(b)) + b
    if isinstance(v, (list, tuple)):
        if all(isinstance(x, bool) for x in v):
            body = b"".join(struct.pack("<?", x) for x in v)
            return struct.pack("<IIQ", _ARR, _BOOL, len(v)) + body
        if all(isinstance(x, int) for x in v):
            body = b"".join(struct.pack("<i", x) for x in v)
            return struct.pack("<IIQ", _ARR, _I32, len(v)) + body
        if all(isinstance(x, float) for x in v):
            body = b"".join(struct.pack("<f", x) for x in v)
            return struct.pack("<IIQ", _ARR, _F32, len(v)) + body
    raise GGUFError(f"cannot encode metadata value {v!r}")


def write_gguf(path: str, kv: dict, tensors, alignment: int = 32) -> None:
    """tensors: iterable of (name, ggml_type, dims, data ndarray)."""
    tensors = list(tensors)
    head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv) + 1))

    def s(x):
        b = x.encode("utf-8")
        return struct.pack("<Q", len(b)) + b

    head += s("general.alignment") + struct.pack("<I", _U32) + struct.pack("<I", alignment)
    for k, v in kv.items():
        head += s(k) + _pack_value(v)
    offsets, off = [], 0
    for name, typ, dims, data in tensors:
        n = tensor_bytes(typ, dims)
        if np.asarray(data).nbytes != n:
            raise GGUFError(f"{name}: {np.asarray(data).nbytes} bytes, expected {n}")
        offsets.append(off)
        off = (off + n + alignment - 1) // alignment * alignment
    for (name, typ, dims, _), o in zip(tensors, offsets):
        head += s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", typ, o)
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * pad)
        pos = 0
        for (name, typ, dims, data), o in zip(tensors, offsets):
            if o > pos:
                f.write(b"\0" * (o - pos))
                pos = o
            b = np.ascontiguousarray(data).tobytes()
            f.write(b)
            pos += len(b)
