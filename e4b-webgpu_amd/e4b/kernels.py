"""Kernel-level entry points (parity tests and per-config benches).

Each wrapper takes DeviceBuffers and calls the matching C-ABI function; the
weights are device copies of the packed layouts from formats.py.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import DT_F16, DT_F32, check, lib
from .device import DeviceBuffer
from .formats import q40_pack, q6k_pack


def _vp(x) -> C.c_void_p:
    if x is None:
        return C.c_void_p(0)
    return C.c_void_p(x.ptr if isinstance(x, DeviceBuffer) else int(x))


class Q40Matrix:
    """A q4_0 matrix resident on the device in the library's packed layout."""

    def __init__(self, ggml: np.ndarray, rows: int, cols: int):
        self.rows, self.cols = rows, cols
        self.buf = DeviceBuffer.from_array(q40_pack(ggml, rows, cols))

    def gemv_dev(self, x: DeviceBuffer, x_dtype: int, y: DeviceBuffer, stream=None) -> None:
        check(lib.e4b_k_q40_gemv(_vp(self.buf), self.rows, self.cols, _vp(x), x_dtype, _vp(y), _vp(stream)),
              "e4b_k_q40_gemv")

    def geglu_dev(self, x: DeviceBuffer, out: DeviceBuffer, stream=None) -> None:
        """rows = [gate (ff) ; up (ff)]: out f16[ff] = gelu(gate . x) * (up . x)"""
        check(lib.e4b_k_q40_gemv_geglu(_vp(self.buf), self.rows // 2, self.cols, _vp(x), _vp(out), _vp(stream)),
              "e4b_k_q40_gemv_geglu")

    def gemm_dev(self, x: DeviceBuffer, m: int, y: DeviceBuffer, stream=None) -> None:
        """x f16[m][cols] -> y f32[m][rows] on the matrix cores"""
        check(lib.e4b_k_q40_gemm(_vp(self.buf), self.rows, self.cols, _vp(x), m, _vp(y), _vp(stream)),
              "e4b_k_q40_gemm")

    def gemm_geglu_dev(self, x: DeviceBuffer, m: int, out: DeviceBuffer, stream=None) -> None:
        """rows = [gate (ff) ; up (ff)]: x f16[m][cols] -> out f16[m][ff]"""
        check(lib.e4b_k_q40_gemm_geglu(_vp(self.buf), self.rows // 2, self.cols, _vp(x), m, _vp(out), _vp(stream)),
              "e4b_k_q40_gemm_geglu")

    def gemm(self, x: np.ndarray) -> np.ndarray:
        """Host convenience: x f16 [m][cols] -> f32 [m][rows]."""
        x = np.ascontiguousarray(x, np.float16)
        m = x.shape[0]
        xd = DeviceBuffer.from_array(x)
        yd = DeviceBuffer(m * self.rows * 4)
        self.gemm_dev(xd, m, yd)
        return yd.download(np.float32, m * self.rows).reshape(m, self.rows)

    def gemm_geglu(self, x: np.ndarray) -> np.ndarray:
        """Host convenience: x f16 [m][cols] -> f16 [m][rows / 2]."""
        x = np.ascontiguousarray(x, np.float16)
        m, ff = x.shape[0], self.rows // 2
        xd = DeviceBuffer.from_array(x)
        od = DeviceBuffer(m * ff * 2)
        self.gemm_geglu_dev(xd, m, od)
        return od.download(np.float16, m * ff).reshape(m, ff)

    def geglu_prenorm_dev(self, h_in: DeviceBuffer, resid, w_resid, w_in: DeviceBuffer, scale: float, eps: float,
                          h_out, out: DeviceBuffer, stream=None) -> None:
        """h = (h_in + rms(resid) * w_resid) * scale; x = f16(rms(h) * w_in); out = GeGLU(x)"""
        check(lib.e4b_k_q40_geglu_prenorm(_vp(self.buf), self.rows // 2, self.cols, _vp(h_in), _vp(resid),
                                          _vp(w_resid), _vp(w_in), C.c_float(scale), C.c_float(eps), _vp(h_out),
                                          _vp(out), _vp(stream)), "e4b_k_q40_geglu_prenorm")

    def geglu_prenorm(self, h_in, resid, w_resid, w_in, scale: float = 1.0, eps: float = 1e-6):
        """Host convenience: returns (h f32[cols], out f16[ff])."""
        dev = lambda a: None if a is None else DeviceBuffer.from_array(np.asarray(a, np.float32))  # noqa: E731
        hi, rd, wr, wi = dev(h_in), dev(resid), dev(w_resid), dev(w_in)
        ho = DeviceBuffer(self.cols * 4)
        out = DeviceBuffer(self.rows // 2 * 2)
        self.geglu_prenorm_dev(hi, rd, wr, wi, scale, eps, ho, out)
        return ho.download(np.float32, self.cols), out.download(np.float16, self.rows // 2)

    def geglu(self, x: np.ndarray) -> np.ndarray:
        xd = DeviceBuffer.from_array(x.astype(np.float16))
        out = DeviceBuffer(self.rows // 2 * 2)
        self.geglu_dev(xd, out)
        return out.download(np.float16, self.rows // 2)

    def gemv(self, x: np.ndarray) -> np.ndarray:
        """Host convenience: x is float32 or float16 [cols] -> float32 [rows]."""
        dt = DT_F16 if x.dtype == np.float16 else DT_F32
        xd = DeviceBuffer.from_array(x.astype(np.float16 if dt == DT_F16 else np.float32))
        yd = DeviceBuffer(self.rows * 4)
        self.gemv_dev(xd, dt, yd)
        return yd.download(np.float32, self.rows)


class Q6KMatrix:
    """A Q6_K matrix resident on the device in the library's packed layout."""

    def __init__(self, ggml: np.ndarray, rows: int, cols: int):
        self.rows, self.cols = rows, cols
        self.buf = DeviceBuffer.from_array(q6k_pack(ggml, rows, cols))

    def gemv_argmax_dev(self, x: DeviceBuffer, softcap: float, logits: DeviceBuffer | None,
                        amax: DeviceBuffer, stream=None) -> None:
        check(lib.e4b_k_q6k_gemv_argmax(_vp(self.buf), self.rows, self.cols, _vp(x), softcap, _vp(logits),
                                        _vp(amax), _vp(stream)), "e4b_k_q6k_gemv_argmax")

    def gemv_argmax(self, x: np.ndarray, softcap: float = 0.0):
        xd = DeviceBuffer.from_array(x.astype(np.float32))
        lg = DeviceBuffer(self.rows * 4)
        am = DeviceBuffer(8)
        self.gemv_argmax_dev(xd, softcap, lg, am)
        a = am.download(np.uint32, 2)
        return lg.download(np.float32, self.rows), int(a[0]), float(a[1:2].view(np.float32)[0])

    def row(self, r: int, mult: float = 1.0) -> np.ndarray:
        out = DeviceBuffer(self.cols * 4)
        check(lib.e4b_k_q6k_row(_vp(self.buf), self.rows, self.cols, r, mult, _vp(out), None), "e4b_k_q6k_row")
        return out.download(np.float32, self.cols)


def argmax(x: np.ndarray):
    xd = DeviceBuffer.from_array(np.ascontiguousarray(x, dtype=np.float32))
    am = DeviceBuffer(8)
    check(lib.e4b_k_argmax(_vp(xd), x.size, _vp(am), None), "e4b_k_argmax")
    a = am.download(np.uint32, 2)
    return int(a[0]), float(a[1:2].view(np.float32)[0])


def rope_inv_freq(theta: float, head_dim: int, angles: int) -> np.ndarray:
    """f32 RoPE inverse frequencies theta^(-2p/head_dim), p < angles."""
    out = np.zeros(max(angles, 1), np.float32)
    check(lib.e4b_rope_inv_freq(C.c_float(theta), head_dim, angles, out.ctypes.data_as(C.c_void_p)),
          "e4b_rope_inv_freq")
    return out[:angles]


class AttnLayer:
    """One layer's decode attention with its f16 KV cache resident on the device.

    Cache layout [kv_heads][slots][head_dim]; window > 0 is a sliding ring
    (position p in slot p % slots), window == 0 a global cache (slot p).
    """

    def __init__(self, q_heads: int, kv_heads: int, head_dim: int, slots: int, window: int,
                 theta: float, rope_angles: int, q_norm: np.ndarray, k_norm: np.ndarray, eps: float = 1e-6,
                 chunk: int = 0):
        self.qh, self.kvh, self.hd, self.slots, self.window = q_heads, kv_heads, head_dim, slots, window
        self.angles, self.eps, self.chunk = rope_angles, eps, chunk
        self.inv_freq = DeviceBuffer.from_array(rope_inv_freq(theta, head_dim, rope_angles)
                                                if rope_angles else np.zeros(1, np.float32))
        self.qw = DeviceBuffer.from_array(np.asarray(q_norm, np.float32))
        self.kw = DeviceBuffer.from_array(np.asarray(k_norm, np.float32))
        n = kv_heads * slots * head_dim
        self.kc = DeviceBuffer(n * 2)
        self.vc = DeviceBuffer(n * 2)
        self.out = DeviceBuffer(q_heads * head_dim * 2)
        self.qkv = DeviceBuffer((q_heads + 2 * kv_heads) * head_dim * 4)

    def load_cache(self, k: np.ndarray, v: np.ndarray) -> None:
        """k, v: f16 [kv_heads][slots][head_dim]"""
        self.kc.upload(np.ascontiguousarray(k, np.float16))
        self.vc.upload(np.ascontiguousarray(v, np.float16))

    def read_cache(self):
        shape = (self.kvh, self.slots, self.hd)
        n = self.kvh * self.slots * self.hd
        return (self.kc.download(np.float16, n).reshape(shape), self.vc.download(np.float16, n).reshape(shape))

    def step_dev(self, pos: int, stream=None) -> None:
        check(lib.e4b_k_attn_decode(_vp(self.qkv), _vp(self.qw), _vp(self.kw), _vp(self.inv_freq), self.angles,
                                    _vp(self.kc), _vp(self.vc), self.qh, self.kvh, self.hd, self.slots, self.window,
                                    pos, C.c_float(self.eps), self.chunk, _vp(self.out), _vp(stream)),
              "e4b_k_attn_decode")

    def step(self, qkv: np.ndarray, pos: int) -> np.ndarray:
        """qkv f32 [(qh + 2 kvh) * hd] raw projections -> f16 [qh * hd]"""
        self.qkv.upload(np.ascontiguousarray(qkv, np.float32))
        self.step_dev(pos)
        return self.out.download(np.float16, self.qh * self.hd)


def attn_prefill(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, window: int, p0: int) -> np.ndarray:
    """Causal attention of a prefill chunk (e4b_k_attn_prefill): q f32
    [m][q_heads][256] at positions p0 .. p0 + m - 1, caches f16
    [kv_heads][slots][256] holding every key needed; returns f16 [m][q_heads * 256]."""
    q = np.ascontiguousarray(q, np.float32)
    m, qh, hd = q.shape
    kvh, slots, _ = k_cache.shape
    qd = DeviceBuffer.from_array(q)
    kd = DeviceBuffer.from_array(np.ascontiguousarray(k_cache, np.float16))
    vd = DeviceBuffer.from_array(np.ascontiguousarray(v_cache, np.float16))
    od = DeviceBuffer(m * qh * hd * 2)
    check(lib.e4b_k_attn_prefill(_vp(qd), _vp(kd), _vp(vd), _vp(od), m, qh, kvh, slots, window, p0, _vp(None)),
          "e4b_k_attn_prefill")
    return od.download(np.float16, m * qh * hd).reshape(m, qh * hd)


class MoeLayer:
    """An A4B-style MoE FFN half-layer resident on the device.

    Weights in raw ggml q4_0 blocks (numpy uint8) and f32 vectors:
    dense_gate/dense_up [FF2][H], dense_down [H][FF2], exp_gate_up
    [E][2 FF][H] (gate rows then up rows per expert), exp_down [E][H][FF],
    router_w [E][H], router_scale / norms [H], pes [E].
    """

    def __init__(self, H: int, E: int, FF: int, FF2: int, t: dict, eps: float = 1e-6, layer_scale: float = 1.0):
        from ._lib import MoeWeightsC
        self.H, self.E, self.FF, self.FF2 = H, E, FF, FF2
        f = lambda a: DeviceBuffer.from_array(np.ascontiguousarray(a, np.float32))  # noqa: E731
        self._keep = {}
        for n in ("ffn_norm", "router_scale", "pre_ffw2", "router_w", "pes", "post_ffw1", "post_ffw2", "post_ffw"):
            self._keep[n] = f(t[n])
        dense_gu = np.concatenate([np.asarray(t["dense_gate"], np.uint8).reshape(-1),
                                   np.asarray(t["dense_up"], np.uint8).reshape(-1)])
        self._keep["dense_gate_up"] = DeviceBuffer.from_array(q40_pack(dense_gu, 2 * FF2, H))
        self._keep["exp_gate_up"] = DeviceBuffer.from_array(q40_pack(t["exp_gate_up"], E * 2 * FF, H))
        self._keep["dense_down"] = DeviceBuffer.from_array(q40_pack(t["dense_down"], H, FF2))
        self._keep["exp_down"] = DeviceBuffer.from_array(q40_pack(t["exp_down"], E * H, FF))
        w = MoeWeightsC()
        w.hidden, w.n_experts, w.expert_ffn, w.dense_ffn = H, E, FF, FF2
        w.eps, w.layer_scale = eps, layer_scale
        for n, b in self._keep.items():
            setattr(w, n, b.ptr)
        self.w = w
        self.h = DeviceBuffer(H * 4)
        self.h_out = DeviceBuffer(H * 4)
        self.idx = DeviceBuffer(64)
        self.wts = DeviceBuffer(64)
        self.dense = DeviceBuffer(H * 4)
        self.moe = DeviceBuffer(H * 4)

    def forward_dev(self, stream=None) -> None:
        check(lib.e4b_k_moe_layer(C.byref(self.w), _vp(self.h), _vp(self.h_out), _vp(self.idx), _vp(self.wts),
                                  _vp(self.dense), _vp(self.moe), _vp(stream)), "e4b_k_moe_layer")

    def forward(self, h: np.ndarray) -> dict:
        self.h.upload(np.ascontiguousarray(h, np.float32))
        self.forward_dev()
        return {"h_out": self.h_out.download(np.float32, self.H), "topk_idx": self.idx.download(np.uint32, 8),
                "topk_w": self.wts.download(np.float32, 8), "dense_out": self.dense.download(np.float32, self.H),
                "moe_out": self.moe.download(np.float32, self.H)}

    def prefill(self, h: np.ndarray) -> dict:
        """The half-layer over m token rows (e4b_k_moe_prefill): h f32 [m][H]."""
        h = np.ascontiguousarray(h, np.float32)
        m = h.shape[0]
        hd = DeviceBuffer.from_array(h)
        ho, dn, mo = DeviceBuffer(m * self.H * 4), DeviceBuffer(m * self.H * 4), DeviceBuffer(m * self.H * 4)
        ix, wt = DeviceBuffer(m * 32), DeviceBuffer(m * 32)
        check(lib.e4b_k_moe_prefill(C.byref(self.w), _vp(hd), m, _vp(ho), _vp(ix), _vp(wt), _vp(dn), _vp(mo), None),
              "e4b_k_moe_prefill")
        r = lambda b, dt, n: b.download(dt, n)  # noqa: E731
        return {"h_out": r(ho, np.float32, m * self.H).reshape(m, self.H),
                "topk_idx": r(ix, np.uint32, m * 8).reshape(m, 8), "topk_w": r(wt, np.float32, m * 8).reshape(m, 8),
                "dense_out": r(dn, np.float32, m * self.H).reshape(m, self.H),
                "moe_out": r(mo, np.float32, m * self.H).reshape(m, self.H)}

    def router_top8(self, h: np.ndarray):
        self.h.upload(np.ascontiguousarray(h, np.float32))
        check(lib.e4b_k_router_top8(C.byref(self.w), _vp(self.h), _vp(self.idx), _vp(self.wts), None),
              "e4b_k_router_top8")
        return self.idx.download(np.uint32, 8), self.wts.download(np.float32, 8)
