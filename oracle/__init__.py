"""ctypes wrapper of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, and only as the checker / CPU baseline.  The
product library never loads it.

Parity status of each restated function (how it is pinned) is listed in
tests/test_oracle.py; the C sources cite the reference file:line they follow.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


if not os.path.exists(LIB_PATH):
    build()
_lib = C.CDLL(LIB_PATH)

_vp, _i64, _i32, _u32, _cf, _u16 = C.c_void_p, C.c_int64, C.c_int, C.c_uint32, C.c_float, C.c_uint16
_sigs = {
    "orc_h2f": (_cf, [_u16]),
    "orc_f2h": (_u16, [_cf]),
    "orc_q40_dequant": (None, [_vp, _i64, _vp]),
    "orc_q40_gemv": (None, [_vp, _i64, _i64, _vp, _vp]),
    "orc_q6k_dequant": (None, [_vp, _i64, _cf, _vp]),
    "orc_q6k_dequant_row": (None, [_vp, _i64, _i64, _cf, _vp]),
    "orc_q6k_gemv": (None, [_vp, _i64, _i64, _vp, _cf, _vp]),
    "orc_argmax": (None, [_vp, _i64, _vp]),
    "orc_rmsnorm": (None, [_vp, _vp, _i64, _cf, _vp]),
    "orc_gelu_tanh": (_cf, [_cf]),
    "orc_router_topk": (None, [_vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp]),
    "orc_rope_inv_freq": (None, [_cf, _i32, _i32, _vp]),
    "orc_headprep": (None, [_vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _cf, _u32, _vp, _vp, _vp]),
    "orc_attn_ring": (None, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _u32, _vp]),
    "orc_attn_linear": (None, [_vp, _vp, _vp, _i32, _i32, _i32, _u32, _vp]),
    "orc_attn_split": (None, [_vp, _vp, _vp, _i32, _i32, _i32, _u32, _i32, _i32, _i32, _vp, _vp]),
    "orc_attn_combine": (None, [_vp, _vp, _i32, _i32, _i32, _i32, _vp]),
    "orc_kvring_recover": (_i64, [_i64, _i64, _i64]),
    "orc_kvring_check": (_i32, [_i32, _i32, _i32, _i32, _i32]),
    "orc_moe_ffn": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "orc_state_new": (_vp, [_vp]),
    "orc_state_free": (None, [_vp]),
    "orc_step": (_u32, [_vp, _vp, _u32, _u32, _vp, _vp]),
    "orc_kv_slot": (_i64, [_vp, _i32, _u32]),
    "orc_state_kcache": (_vp, [_vp, _i32]),
    "orc_state_vcache": (_vp, [_vp, _i32]),
    "orc_state_set_scoring": (None, [_vp, _i32]),
    "orc_state_set_keep_rows": (None, [_vp, _i32]),
    "orc_state_krow": (_vp, [_vp, _i32]),
    "orc_state_vrow": (_vp, [_vp, _i32]),
    "orc_state_kv_count": (_i64, [_vp]),
    "orc_state_route_margin": (C.c_double, [_vp]),
    "orc_moe_ffn_f": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "orc_state_layer_hidden": (_vp, [_vp, _i32]),
    "orc_state_layer_topk": (_vp, [_vp, _i32]),
    "orc_state_layer_margin": (C.c_double, [_vp, _i32]),
    "orc_state_force_topk": (None, [_vp, _i32, _vp]),
    "orc_state_score": (_vp, [_vp, _i32]),
    "orc_kv_keep": (_i64, [_vp, _i32, _i64, _i64, _i32, _i32, _vp]),
    "orc_kv_compact": (_i64, [_vp, _vp, _i32, _i32]),
    "orc_kv_gather_layer": (None, [_vp, _vp, _i32, _vp, _i64]),
    "orc_state_set_kv_count": (None, [_vp, _i64]),
    "orc_state_set_kv": (None, [_vp, _vp, _i32, _vp, _vp]),
}
for _n, (_r, _a) in _sigs.items():
    _f = getattr(_lib, _n)
    _f.restype = _r
    _f.argtypes = _a


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


def h2f(h: int) -> float:
    return float(_lib.orc_h2f(h))


def f2h(f: float) -> int:
    return int(_lib.orc_f2h(f))


def q40_dequant(blocks: np.ndarray) -> np.ndarray:
    blocks = _u8(blocks)
    nb = blocks.size // 18
    out = np.empty(nb * 32, np.float32)
    _lib.orc_q40_dequant(_p(blocks), nb, _p(out))
    return out


def q40_gemv(w: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    w, x = _u8(w), _f32(x)
    y = np.empty(rows, np.float32)
    _lib.orc_q40_gemv(_p(w), rows, cols, _p(x), _p(y))
    return y


def q6k_dequant(blocks: np.ndarray, mult: float = 1.0) -> np.ndarray:
    blocks = _u8(blocks)
    nb = blocks.size // 210
    out = np.empty(nb * 256, np.float32)
    _lib.orc_q6k_dequant(_p(blocks), nb, mult, _p(out))
    return out


def q6k_row(w: np.ndarray, cols: int, row: int, mult: float = 1.0) -> np.ndarray:
    w = _u8(w)
    out = np.empty(cols, np.float32)
    _lib.orc_q6k_dequant_row(_p(w), cols, row, mult, _p(out))
    return out


def q6k_gemv(w: np.ndarray, rows: int, cols: int, x: np.ndarray, softcap: float = 0.0) -> np.ndarray:
    w, x = _u8(w), _f32(x)
    y = np.empty(rows, np.float32)
    _lib.orc_q6k_gemv(_p(w), rows, cols, _p(x), softcap, _p(y))
    return y


def argmax(x: np.ndarray):
    x = _f32(x)
    out = np.zeros(2, np.uint32)
    _lib.orc_argmax(_p(x), x.size, _p(out))
    return int(out[0]), float(out[1:2].view(np.float32)[0])


def rmsnorm(x, w, eps: float = 1e-6) -> np.ndarray:
    x = _f32(x)
    w = None if w is None else _f32(w)
    y = np.empty_like(x)
    _lib.orc_rmsnorm(_p(x), _p(w), x.size, eps, _p(y))
    return y


def gelu_tanh(g: float) -> float:
    return float(_lib.orc_gelu_tanh(g))


def router_topk(x, W, pes, K: int):
    x, W, pes = _f32(x), _f32(W), _f32(pes)
    E, H = W.shape if W.ndim == 2 else (pes.size, x.size)
    idx = np.zeros(K, np.uint32)
    wts = np.zeros(K, np.float32)
    scores = np.zeros(E, np.float32)
    _lib.orc_router_topk(_p(x), _p(W), _p(pes), H, E, K, _p(idx), _p(wts), _p(scores))
    return idx, wts, scores


def rope_inv_freq(theta: float, head_dim: int, angles: int) -> np.ndarray:
    out = np.empty(angles, np.float32)
    _lib.orc_rope_inv_freq(theta, head_dim, angles, _p(out))
    return out


def headprep(qkv, qh, kvh, hd, angles, inv_freq, qw, kw, eps, pos):
    qkv, inv_freq, qw, kw = _f32(qkv), _f32(inv_freq), _f32(qw), _f32(kw)
    q = np.empty(qh * hd, np.float32)
    k = np.empty(kvh * hd, np.uint16)
    v = np.empty(kvh * hd, np.uint16)
    _lib.orc_headprep(_p(qkv), qh, kvh, hd, angles, _p(inv_freq), _p(qw), _p(kw), eps, pos, _p(q), _p(k), _p(v))
    return q, k, v


def attn_ring(q, kc, vc, qh, kvh, hd, ring, window, pos):
    q = _f32(q)
    kc, vc = np.ascontiguousarray(kc, np.uint16), np.ascontiguousarray(vc, np.uint16)
    out = np.empty(qh * hd, np.uint16)
    _lib.orc_attn_ring(_p(q), _p(kc), _p(vc), qh, kvh, hd, ring, window, pos, _p(out))
    return out


def attn_linear(q, kc, vc, qh, kvh, hd, length):
    q = _f32(q)
    kc, vc = np.ascontiguousarray(kc, np.uint16), np.ascontiguousarray(vc, np.uint16)
    out = np.empty(qh * hd, np.uint16)
    _lib.orc_attn_linear(_p(q), _p(kc), _p(vc), qh, kvh, hd, length, _p(out))
    return out


def attn_split(q, kc, vc, qh, kvh, hd, length, window, chunks, cs):
    q = _f32(q)
    kc, vc = np.ascontiguousarray(kc, np.uint16), np.ascontiguousarray(vc, np.uint16)
    po = np.empty(qh * chunks * hd, np.float32)
    pme = np.empty(qh * chunks * 2, np.float32)
    _lib.orc_attn_split(_p(q), _p(kc), _p(vc), qh, kvh, hd, length, window, chunks, cs, _p(po), _p(pme))
    return po, pme


def attn_combine(po, pme, qh, hd, n_chunks, chunks):
    po, pme = _f32(po), _f32(pme)
    out = np.empty(qh * hd, np.uint16)
    _lib.orc_attn_combine(_p(po), _p(pme), qh, hd, n_chunks, chunks, _p(out))
    return out


def kv_keep(score: np.ndarray, n: int, budget: int, protect: int) -> np.ndarray:
    """compactAll's keep list (src/engine-a4b.js:590-603) for one full layer
    from its [q_heads][scap] f32 score buffer over the first n slots."""
    sc = _f32(score)
    qh, scap = sc.shape
    keep = np.empty(max(n, 1), np.uint32)
    cnt = int(_lib.orc_kv_keep(_p(sc), qh, scap, n, budget, protect, _p(keep)))
    return keep[:cnt].copy()


def kvring_recover(t: int, mw: int, ring: int) -> int:
    return int(_lib.orc_kvring_recover(t, mw, ring))


def kvring_check(W: int, Cc: int, RING: int, NCHUNKS: int, GEN: int) -> int:
    """0 = SoundRec and Complete hold; 1 = SoundRec violated; 2 = Complete violated."""
    return int(_lib.orc_kvring_check(W, Cc, RING, NCHUNKS, GEN))


# ---- structures for the MoE half-layer and the full step --------------------
class MoeC(C.Structure):
    _fields_ = [
        ("hidden", _i32), ("n_experts", _i32), ("top_k", _i32), ("expert_ffn", _i32), ("dense_ffn", _i32),
        ("eps", _cf), ("layer_scale", _cf),
        ("ffn_norm", _vp), ("router_scale", _vp), ("pre_ffw2", _vp), ("router_w", _vp), ("pes", _vp),
        ("dense_gate", _vp), ("dense_up", _vp), ("dense_down", _vp), ("exp_gate_up", _vp), ("exp_down", _vp),
        ("post_ffw1", _vp), ("post_ffw2", _vp), ("post_ffw", _vp),
    ]


def moe_ffn(m: dict, h: np.ndarray, force=None):
    """m: dict of numpy arrays / ints keyed like orc_moe's fields.  force:
    the top_k experts the expert slots use instead of the router's own picks
    (weighted from the router's scores); the returned ids are then `force`."""
    keep = {}

    def arr(name, kind):
        a = _f32(m[name]) if kind == "f" else _u8(m[name])
        keep[name] = a
        return _p(a)

    s = MoeC()
    for k in ("hidden", "n_experts", "top_k", "expert_ffn", "dense_ffn"):
        setattr(s, k, int(m[k]))
    s.eps = float(m.get("eps", 1e-6))
    s.layer_scale = float(m.get("layer_scale", 1.0))
    for k in ("ffn_norm", "router_scale", "pre_ffw2", "router_w", "pes", "post_ffw1", "post_ffw2", "post_ffw"):
        setattr(s, k, arr(k, "f"))
    for k in ("dense_gate", "dense_up", "dense_down", "exp_gate_up", "exp_down"):
        setattr(s, k, arr(k, "u"))
    H, K = int(m["hidden"]), int(m["top_k"])
    h = _f32(h)
    idx = np.zeros(K, np.uint32)
    w = np.zeros(K, np.float32)
    dense = np.zeros(H, np.float32)
    moe = np.zeros(H, np.float32)
    hout = np.zeros(H, np.float32)
    if force is None:
        _lib.orc_moe_ffn(C.byref(s), _p(h), _p(idx), _p(w), _p(dense), _p(moe), _p(hout))
    else:
        f = np.ascontiguousarray(np.asarray(force, np.uint32).reshape(K))
        _lib.orc_moe_ffn_f(C.byref(s), _p(h), _p(f), None, _p(idx), _p(w), _p(dense), _p(moe), _p(hout), None)
    return idx, w, dense, moe, hout


class LayerC(C.Structure):
    _fields_ = [
        ("attn_norm", _vp), ("q_norm", _vp), ("k_norm", _vp), ("post_attn_norm", _vp), ("ffn_norm", _vp),
        ("post_ffw_norm", _vp), ("post_norm", _vp), ("layer_scale", _cf),
        ("wq", _vp), ("wk", _vp), ("wv", _vp), ("wo", _vp), ("wgate", _vp), ("wup", _vp), ("wdown", _vp),
        ("inp_gate", _vp), ("proj", _vp), ("moe", MoeC),
    ]


class ModelC(C.Structure):
    _fields_ = [
        ("hidden", _i32), ("layers", _i32), ("q_heads", _i32), ("kv_heads", _i32), ("head_dim", _i32),
        ("ffn", _i32), ("ple_dim", _i32), ("vocab", _i32), ("window", _i32), ("ring", _i32), ("max_seq", _i32),
        ("rope_angles", _i32), ("theta_local", _cf), ("theta_global", _cf), ("eps", _cf), ("softcap", _cf),
        ("layer_global", _vp), ("tok_embd", _vp), ("out_norm", _vp), ("ple_tab", _vp), ("ple_proj", _vp),
        ("ple_proj_norm", _vp), ("L", _vp),
        ("recipe", _i32), ("head_dim_full", _i32), ("rope_angles_full", _i32), ("layer_kv_heads", _vp),
    ]


class OracleModel:
    """Full decode step on the CPU over ggml-format tensors: the E4B recipe
    (dense GeGLU FFN, per-layer embeddings) or, with cfg["recipe"] == 1, the
    A4B recipe (MoE FFN half, per-layer KV heads, full layers with
    head_dim_full, rope_angles_full and V = K).

    ``tensors`` maps GGUF tensor names (the ones e4b.engine uses) to numpy
    arrays: q4_0 / Q6_K as uint8 block bytes, norms as float32.
    """

    _CFG_KEYS = ("hidden", "layers", "q_heads", "kv_heads", "head_dim", "ffn", "ple_dim", "vocab", "window",
                 "ring", "max_seq", "rope_angles")

    def __init__(self, cfg: dict, tensors: dict):
        self._keep = []
        self.cfg = dict(cfg)
        m = ModelC()
        for k in self._CFG_KEYS:
            setattr(m, k, int(cfg[k]))
        m.theta_local = float(cfg["theta_local"])
        m.theta_global = float(cfg["theta_global"])
        m.eps = float(cfg["eps"])
        m.softcap = float(cfg["softcap"])
        lg = np.ascontiguousarray(np.asarray(cfg["layer_global"], dtype=np.uint8))
        self._keep.append(lg)
        m.layer_global = _p(lg)

        def t(name, kind):
            a = tensors.get(name)
            if a is None:
                return None
            a = _f32(a) if kind == "f" else _u8(a)
            self._keep.append(a)
            return _p(a)

        m.tok_embd = t("token_embd.weight", "u")
        m.out_norm = t("output_norm.weight", "f")
        m.ple_tab = t("per_layer_token_embd.weight", "u")
        m.ple_proj = t("per_layer_model_proj.weight", "u")
        m.ple_proj_norm = t("per_layer_proj_norm.weight", "f")
        L = (LayerC * int(cfg["layers"]))()
        for i in range(int(cfg["layers"])):
            p = f"blk.{i}."
            ly = L[i]
            ly.attn_norm = t(p + "attn_norm.weight", "f")
            ly.q_norm = t(p + "attn_q_norm.weight", "f")
            ly.k_norm = t(p + "attn_k_norm.weight", "f")
            ly.post_attn_norm = t(p + "post_attention_norm.weight", "f")
            ly.ffn_norm = t(p + "ffn_norm.weight", "f")
            ly.post_ffw_norm = t(p + "post_ffw_norm.weight", "f")
            ly.post_norm = t(p + "post_norm.weight", "f")
            sc = tensors.get(p + "layer_output_scale.weight")
            ly.layer_scale = float(np.asarray(sc, np.float32).reshape(-1)[0]) if sc is not None else 1.0
            for fld, nm in (("wq", "attn_q"), ("wk", "attn_k"), ("wv", "attn_v"), ("wo", "attn_output"),
                            ("wgate", "ffn_gate"), ("wup", "ffn_up"), ("wdown", "ffn_down"),
                            ("inp_gate", "inp_gate"), ("proj", "proj")):
                setattr(ly, fld, t(p + nm + ".weight", "u"))
        recipe = int(cfg.get("recipe", 0))
        m.recipe = recipe
        if recipe == 1:
            m.head_dim_full = int(cfg.get("head_dim_full") or cfg["head_dim"])
            m.rope_angles_full = int(cfg.get("rope_angles_full") or cfg["rope_angles"])
            kvh = cfg.get("layer_kv_heads")
            if kvh is not None:
                kv = np.ascontiguousarray(np.asarray(kvh, dtype=np.int32))
                self._keep.append(kv)
                m.layer_kv_heads = _p(kv)
            H = int(cfg["hidden"])
            for i in range(int(cfg["layers"])):
                p = f"blk.{i}."
                mo = L[i].moe
                mo.hidden, mo.n_experts, mo.top_k = H, int(cfg["n_experts"]), 8
                mo.expert_ffn, mo.dense_ffn = int(cfg["expert_ffn"]), int(cfg["ffn"])
                mo.eps, mo.layer_scale = float(cfg["eps"]), L[i].layer_scale
                mo.ffn_norm = L[i].ffn_norm
                mo.router_scale = t(p + "ffn_gate_inp.scale", "f")
                mo.pre_ffw2 = t(p + "pre_ffw_norm_2.weight", "f")
                mo.router_w = t(p + "ffn_gate_inp.weight", "f")
                mo.pes = t(p + "ffn_down_exps.scale", "f")
                mo.dense_gate, mo.dense_up, mo.dense_down = L[i].wgate, L[i].wup, L[i].wdown
                mo.exp_gate_up = t(p + "ffn_gate_up_exps.weight", "u")
                mo.exp_down = t(p + "ffn_down_exps.weight", "u")
                mo.post_ffw1 = t(p + "post_ffw_norm_1.weight", "f")
                mo.post_ffw2 = t(p + "post_ffw_norm_2.weight", "f")
                mo.post_ffw = L[i].post_ffw_norm
        self._keep.append(L)
        m.L = C.cast(L, C.c_void_p)
        self._m = m
        self._state = _lib.orc_state_new(C.byref(m))

    def reset(self):
        _lib.orc_state_free(self._state)
        self._state = _lib.orc_state_new(C.byref(self._m))

    def step(self, token: int, pos: int, want_logits: bool = False, want_hidden: bool = False):
        lg = np.empty(int(self.cfg["vocab"]), np.float32) if want_logits else None
        hd = np.empty(int(self.cfg["hidden"]), np.float32) if want_hidden else None
        tok = int(_lib.orc_step(C.byref(self._m), self._state, token, pos, _p(lg), _p(hd)))
        return tok, lg, hd

    def set_scoring(self, on: bool) -> None:
        _lib.orc_state_set_scoring(self._state, int(bool(on)))

    def kv_count(self) -> int:
        return int(_lib.orc_state_kv_count(self._state))

    def route_margin(self) -> float:
        """A4B recipe: the smallest top-8 decision margin of the last step's
        layers, (8th - 9th largest router score) / max |score|."""
        return float(_lib.orc_state_route_margin(self._state))

    def layer_hidden(self, layer: int) -> np.ndarray:
        """The residual stream after `layer` in the last step (f32 [hidden])."""
        p = _lib.orc_state_layer_hidden(self._state, int(layer))
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), (int(self.cfg["hidden"]),)).copy()

    def layer_topk(self, layer: int) -> np.ndarray:
        """A4B recipe: the oracle's own top-8 experts at `layer` in the last
        step (before any forcing)."""
        p = _lib.orc_state_layer_topk(self._state, int(layer))
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint32)), (8,)).copy()

    def layer_margin(self, layer: int) -> float:
        """A4B recipe: (8th - 9th router score) / max |score| at `layer`."""
        return float(_lib.orc_state_layer_margin(self._state, int(layer)))

    def force_topk(self, layer: int, idx=None) -> None:
        """A4B recipe: the next steps' expert slots at `layer` use the 8
        experts `idx` (weighted from the oracle's own router scores), or the
        oracle's own picks again when idx is None."""
        if idx is None:
            _lib.orc_state_force_topk(self._state, int(layer), None)
        else:
            a = np.ascontiguousarray(np.asarray(idx, np.uint32).reshape(8))
            _lib.orc_state_force_topk(self._state, int(layer), _p(a))

    def set_keep_rows(self, on: bool) -> None:
        """With keep_rows the step attends to the K/V row handed over (set_kv)
        for the current token instead of writing its own there; its own rows
        are still computed and returned by rows()."""
        _lib.orc_state_set_keep_rows(self._state, int(bool(on)))

    def layer_shape(self, layer: int):
        """(kv_heads, head_dim) of a layer's caches."""
        c = self.cfg
        if int(c.get("recipe", 0)) == 1:
            kvh = c.get("layer_kv_heads")
            kvh = int(kvh[layer]) if kvh is not None else int(c["kv_heads"])
            glob = bool(c["layer_global"][layer])
            return kvh, int(c.get("head_dim_full") or c["head_dim"]) if glob else int(c["head_dim"])
        return int(c["kv_heads"]), int(c["head_dim"])

    def rows(self, layer: int):
        """(k, v) rows the last step computed for a layer, f16 bits [kv_heads][head_dim]."""
        kvh, hd = self.layer_shape(layer)
        out = []
        for fn in (_lib.orc_state_krow, _lib.orc_state_vrow):
            p = fn(self._state, layer)
            out.append(np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint16)), shape=(kvh * hd,)).copy().reshape(kvh, hd))
        return out[0], out[1]

    def score(self, layer: int) -> np.ndarray:
        """[q_heads][max_seq] accumulated attention mass of a full layer."""
        qh, ms = int(self.cfg["q_heads"]), int(self.cfg["max_seq"])
        p = _lib.orc_state_score(self._state, layer)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), shape=(qh, ms)).copy()

    def compact(self, budget: int, protect: int) -> int:
        """compactAll on every full layer; returns the new entry count."""
        return int(_lib.orc_kv_compact(C.byref(self._m), self._state, budget, protect))

    def compact_with(self, keeps: dict) -> None:
        """The gather of compactAll with given keep lists {layer: slots}
        (every full layer), then kv_count = their common length."""
        cnt = None
        for layer, keep in keeps.items():
            k = np.ascontiguousarray(np.asarray(keep, np.uint32))
            _lib.orc_kv_gather_layer(C.byref(self._m), self._state, int(layer), _p(k), int(k.size))
            cnt = int(k.size)
        if cnt is not None:
            _lib.orc_state_set_kv_count(self._state, cnt)

    def set_kv(self, layer: int, k: np.ndarray, v: np.ndarray) -> None:
        """Overwrite a layer's caches with f16 bits laid out [slots][kvh][hd]."""
        k = np.ascontiguousarray(k, np.uint16)
        v = np.ascontiguousarray(v, np.uint16)
        _lib.orc_state_set_kv(C.byref(self._m), self._state, int(layer), _p(k), _p(v))

    def set_kv_count(self, n: int) -> None:
        _lib.orc_state_set_kv_count(self._state, int(n))

    def kv_slot(self, is_global: bool, pos: int) -> int:
        return int(_lib.orc_kv_slot(C.byref(self._m), int(is_global), pos))

    def kcache(self, layer: int, n: int) -> np.ndarray:
        p = _lib.orc_state_kcache(self._state, layer)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint16)), shape=(n,)).copy()

    def vcache(self, layer: int, n: int) -> np.ndarray:
        p = _lib.orc_state_vcache(self._state, layer)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint16)), shape=(n,)).copy()

    def __del__(self):
        try:
            _lib.orc_state_free(self._state)
        except Exception:
            pass
