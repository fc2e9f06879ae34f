"""ggml tensor formats, repacking and seeded synthetic tensors.

``tensor_bytes`` mirrors src/gguf.js:5-15 (TYPE_SIZES / tensorBytes); the pack
functions call the library's repackers (replacing repackQ40 / repackQ6K,
src/engine-a4b.js:29-73); the synth functions call the library's counter-based
generators so every caller produces identical bytes.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import GGML_F16, GGML_F32, GGML_Q4_0, GGML_Q6_K, check, lib

# type id -> (block bytes, block elements), as src/gguf.js:5-9
TYPE_SIZES = {
    GGML_F32: (4, 1),
    GGML_F16: (2, 1),
    30: (2, 1),        # BF16
    GGML_Q4_0: (18, 32),
    6: (22, 32),       # Q5_0
    8: (34, 32),       # Q8_0
    12: (144, 256),    # Q4_K
    GGML_Q6_K: (210, 256),
}


def tensor_bytes(ggml_type: int, dims) -> int:
    bb, be = TYPE_SIZES[ggml_type]
    n = 1
    for d in dims:
        n *= int(d)
    if n % be:
        raise ValueError(f"{n} elements is not a whole number of type-{ggml_type} blocks")
    return n // be * bb


def _ptr(a: np.ndarray) -> C.c_void_p:
    return a.ctypes.data_as(C.c_void_p)


def q40_pack(ggml: np.ndarray, rows: int, cols: int) -> np.ndarray:
    ggml = np.ascontiguousarray(ggml, dtype=np.uint8)
    if ggml.nbytes != rows * (cols // 32) * 18:
        raise ValueError("q4_0 byte count does not match rows x cols")
    out = np.empty(lib.e4b_q40_packed_bytes(rows, cols), dtype=np.uint8)
    check(lib.e4b_q40_pack(_ptr(ggml), rows, cols, _ptr(out)), "e4b_q40_pack")
    return out


def q6k_pack(ggml: np.ndarray, rows: int, cols: int) -> np.ndarray:
    ggml = np.ascontiguousarray(ggml, dtype=np.uint8)
    if ggml.nbytes != rows * (cols // 256) * 210:
        raise ValueError("Q6_K byte count does not match rows x cols")
    out = np.empty(lib.e4b_q6k_packed_bytes(rows, cols), dtype=np.uint8)
    check(lib.e4b_q6k_pack(_ptr(ggml), rows, cols, _ptr(out)), "e4b_q6k_pack")
    return out


def synth_u64(seed: int, index: int) -> int:
    return int(lib.e4b_synth_u64(seed, index))


def synth_normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    check(lib.e4b_synth_normal_f32(seed, n, mean, std, _ptr(out)), "e4b_synth_normal_f32")
    return out


def synth_uniform_u32(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint32)
    check(lib.e4b_synth_uniform_u32(seed, n, lo, hi, _ptr(out)), "e4b_synth_uniform_u32")
    return out


def synth_q40(seed: int, rows: int, cols: int, sigma: float = 0.02) -> np.ndarray:
    out = np.empty(rows * (cols // 32) * 18, dtype=np.uint8)
    check(lib.e4b_synth_q40(seed, rows, cols, sigma, _ptr(out)), "e4b_synth_q40")
    return out


def synth_q6k(seed: int, rows: int, cols: int, sigma: float = 1e-3) -> np.ndarray:
    out = np.empty(rows * (cols // 256) * 210, dtype=np.uint8)
    check(lib.e4b_synth_q6k(seed, rows, cols, sigma, _ptr(out)), "e4b_synth_q6k")
    return out


def q6k_row(ggml, cols: int, row: int) -> np.ndarray:
    """Row `row` of a raw ggml Q6_K matrix [rows][cols] as f32 (the published
    block_q6_K layout: per 256 weights ql[128] low nibbles, qh[64] high bit
    pairs, 16 int8 group scales, f16 d; weight = d * scale * (q - 32), with
    q = 4 low bits | 2 high bits << 4 in ggml's element order)."""
    nsb = cols // 256
    raw = np.frombuffer(memoryview(np.ascontiguousarray(ggml)).cast("B"), np.uint8)
    blk = raw[row * nsb * 210:(row + 1) * nsb * 210].reshape(nsb, 210)
    ql = blk[:, :128].astype(np.int32)
    qh = blk[:, 128:192].astype(np.int32)
    sc = blk[:, 192:208].view(np.int8).astype(np.float32)
    d = blk[:, 208:210].copy().view(np.float16).astype(np.float32).reshape(nsb)
    y = np.empty((nsb, 256), np.float32)
    for half in range(2):
        l_lo, l_hi = ql[:, 64 * half:64 * half + 32], ql[:, 64 * half + 32:64 * half + 64]
        h = qh[:, 32 * half:32 * half + 32]
        q = [(l_lo & 15) | ((h & 3) << 4), (l_hi & 15) | (((h >> 2) & 3) << 4),
             (l_lo >> 4) | (((h >> 4) & 3) << 4), (l_hi >> 4) | (((h >> 6) & 3) << 4)]
        for j in range(4):
            for part in range(2):  # 16-element scale groups
                g = 8 * half + 2 * j + part
                s = slice(128 * half + 32 * j + 16 * part, 128 * half + 32 * j + 16 * part + 16)
                y[:, s] = (d * sc[:, g])[:, None] * (q[j][:, 16 * part:16 * part + 16] - 32).astype(np.float32)
    return y.reshape(-1)
