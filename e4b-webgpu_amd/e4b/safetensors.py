"""safetensors reader and writer (the loader.js interface of the reference).

``open_safetensors(path)`` mirrors openSafetensors (src/loader.js:4-24): the
file starts with a little-endian u64 header length n, then n bytes of JSON
mapping tensor names to {dtype, shape, data_offsets: [begin, end]} (offsets
relative to the end of the header), plus an optional ``__metadata__`` entry
that the index drops.  ``fetch(name)`` returns the index entry with ``buf``,
that tensor's bytes only (the file is memory-mapped, as the reference reads
one HTTP byte range per tensor).  ``bf16_to_f32`` (src/loader.js:26-32)
widens bf16 bits to f32 by a 16-bit shift; ``f32_scalar`` (:34-36) reads
the first f32 of a buffer, 0 when empty.  ``write_safetensors`` writes the
same format (tests, synthetic checkpoints).
"""
from __future__ import annotations

import json
import struct

import numpy as np

# element sizes of the dtypes the format names
DTYPE_BYTES = {"BOOL": 1, "U8": 1, "I8": 1, "F8_E4M3": 1, "F8_E5M2": 1, "I16": 2, "U16": 2, "F16": 2, "BF16": 2,
               "I32": 4, "U32": 4, "F32": 4, "I64": 8, "U64": 8, "F64": 8}


class SafetensorsError(ValueError):
    pass


class SafetensorsFile:
    def __init__(self, path: str, index: dict, base: int, mm: np.memmap):
        self.path, self.index, self.base, self._mm = path, index, base, mm

    def has(self, name: str) -> bool:
        return name in self.index

    def info(self, name: str) -> dict | None:
        return self.index.get(name)

    def fetch(self, name: str) -> dict:
        t = self.index.get(name)
        if t is None:
            raise SafetensorsError(f"tensor not found: {name}")
        a, b = t["data_offsets"]
        return dict(t, buf=np.asarray(self._mm[self.base + a:self.base + b]))


def open_safetensors(path: str) -> SafetensorsFile:
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    if mm.size < 8:
        raise SafetensorsError(f"{path}: shorter than the 8-byte header length")
    n = struct.unpack("<Q", mm[:8].tobytes())[0]
    if 8 + n > mm.size:
        raise SafetensorsError(f"{path}: header of {n} bytes extends past the end of the file")
    index = json.loads(mm[8:8 + n].tobytes().decode("utf-8"))
    index.pop("__metadata__", None)
    base = 8 + n
    for name, t in index.items():
        a, b = t["data_offsets"]
        count = int(np.prod(t["shape"], dtype=np.int64)) if t["shape"] else 1
        if not (0 <= a <= b and base + b <= mm.size) or b - a != count * DTYPE_BYTES.get(t["dtype"], 0):
            raise SafetensorsError(f"{name}: data_offsets {t['data_offsets']} do not hold {t['shape']} {t['dtype']}")
    return SafetensorsFile(path, index, base, mm)


def _bytes(buf) -> bytes:
    return bytes(buf) if isinstance(buf, (bytes, bytearray, memoryview)) else np.ascontiguousarray(buf).tobytes()


def bf16_to_f32(buf) -> np.ndarray:
    """bf16 bits (bytes or a u16 array) -> f32: each value is the high half of its f32."""
    u16 = np.frombuffer(_bytes(buf), np.uint16)
    return (u16.astype(np.uint32) << 16).view(np.float32)


def f32_scalar(buf) -> float:
    a = np.frombuffer(_bytes(buf), np.float32)
    return float(a[0]) if a.size else 0.0


def write_safetensors(path: str, tensors: dict, metadata: dict | None = None) -> None:
    """tensors: name -> (dtype string, shape, raw bytes or array); data packed
    in insertion order, header padded with spaces to a multiple of 8."""
    header, blobs, off = {}, [], 0
    if metadata:
        header["__metadata__"] = {str(k): str(v) for k, v in metadata.items()}
    for name, (dtype, shape, data) in tensors.items():
        raw = _bytes(data)
        count = int(np.prod(shape, dtype=np.int64)) if shape else 1
        if len(raw) != count * DTYPE_BYTES[dtype]:
            raise SafetensorsError(f"{name}: {len(raw)} bytes for {shape} {dtype}")
        header[name] = {"dtype": dtype, "shape": [int(s) for s in shape], "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header, separators=(",", ":")).encode("utf-8")
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)
