"""Engine: the host surface of the reference's decode engine over libe4b.

Mirrors the object returned by loadEngineA4B (src/engine-a4b.js:854-856):
``step(token, pos)``, ``argmax_fast()``, ``decode_chunk(start_pos, count)``,
``generate_fast(ids, max_new, eos)``, ``prefill(ids)``,
``generate_prefill(ids, max_new, eos)``, ``profile_step(token, pos)``,
``profile_prefill(ids)``, ``compact()``, ``generate_long(...)``,
``read_hidden()``.
The compute runs in libe4b.so (HIP, gfx950); this module only moves tensors
and calls the C ABI.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import ConfigC, ProfEntryC, check, lib
from .gguf import open_gguf
from .model import E4BConfig, Tensor


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# GGUF metadata keys of the E4B-shaped model (gemma3n-style prefix)
_KV = {
    "hidden": "embedding_length", "layers": "block_count", "q_heads": "attention.head_count",
    "kv_heads": "attention.head_count_kv", "head_dim": "attention.key_length", "ffn": "feed_forward_length",
    "ple_dim": "embedding_length_per_layer_input", "vocab": "vocab_size", "window": "attention.sliding_window",
    "rope_angles": "rope.dimension_count_half", "theta_local": "rope.freq_base_swa", "theta_global": "rope.freq_base",
    "eps": "attention.layer_norm_rms_epsilon", "softcap": "final_logit_softcapping",
}
ARCH = "e4b"
# the gemma4 MoE keys loadEngineA4B reads (src/engine-a4b.js:100-116); the
# full layers' head dim is key_length, the sliding layers' key_length_swa,
# head_count_kv is a per-layer array
_KV_A4B = {
    "hidden": "embedding_length", "layers": "block_count", "q_heads": "attention.head_count",
    "ffn": "feed_forward_length", "expert_ffn": "expert_feed_forward_length", "n_experts": "expert_count",
    "window": "attention.sliding_window", "eps": "attention.layer_norm_rms_epsilon",
    "softcap": "final_logit_softcapping", "head_dim_full": "attention.key_length",
    "head_dim": "attention.key_length_swa", "vocab": "vocab_size",
}
ARCH_A4B = "gemma4"
TOP_K = 8  # expert_used_count the MoE kernels select


def config_to_kv(cfg: E4BConfig) -> dict:
    if cfg.recipe == 1:
        kv = {"general.architecture": ARCH_A4B}
        for f, k in _KV_A4B.items():
            kv[f"{ARCH_A4B}.{k}"] = getattr(cfg, f)
        kv[f"{ARCH_A4B}.expert_used_count"] = TOP_K
        kv[f"{ARCH_A4B}.attention.head_count_kv"] = [int(cfg.layer_shape(i)[0]) for i in range(cfg.layers)]
        kv[f"{ARCH_A4B}.attention.sliding_window_pattern"] = [not bool(g) for g in cfg.layer_global]
        return kv
    kv = {"general.architecture": ARCH}
    for f, k in _KV.items():
        kv[f"{ARCH}.{k}"] = getattr(cfg, f)
    kv[f"{ARCH}.attention.sliding_window_pattern"] = [not bool(g) for g in cfg.layer_global]
    return kv


def _a4b_from_kv(kv: dict, arch: str, overrides: dict) -> E4BConfig:
    """The A4B recipe of a gemma4 key set, as e4b_gguf_config derives it."""
    args = {f: kv[f"{arch}.{k}"] for f, k in _KV_A4B.items() if f"{arch}.{k}" in kv}
    if int(kv.get(f"{arch}.expert_used_count", TOP_K)) != TOP_K:
        raise ValueError(f"expert_used_count {kv[f'{arch}.expert_used_count']} (the MoE kernels select {TOP_K})")
    args.update(recipe=1, ple_dim=0)
    kvh = kv.get(f"{arch}.attention.head_count_kv")
    if isinstance(kvh, (list, tuple)):
        args["layer_kv_heads"] = [int(x) for x in kvh]
        args["kv_heads"] = int(kvh[0])
    pat = kv.get(f"{arch}.attention.sliding_window_pattern")
    if pat is not None:
        args["layer_global"] = [0 if s else 1 for s in pat]
    args.update(overrides)
    hd = int(args.get("head_dim", E4BConfig.head_dim))
    hdf = int(args.get("head_dim_full", 512))
    args.update(rope_angles=hd // 2, rope_angles_full=int(0.25 * hdf / 2), theta_local=1e4, theta_global=1e6)
    args["ring"] = max(int(args.get("ring", E4BConfig.ring)), int(args.get("window", E4BConfig.window)) + 512)
    for f in ("eps", "softcap"):
        if f in args:
            args[f] = float(args[f])
    return E4BConfig(**args)


def config_from_kv(kv: dict, **overrides) -> E4BConfig:
    arch = kv.get("general.architecture", ARCH)
    if f"{arch}.expert_count" in kv:
        return _a4b_from_kv(kv, arch, overrides)
    args = {}
    for f, k in _KV.items():
        key = f"{arch}.{k}"
        if key in kv:
            args[f] = kv[key]
    pat = kv.get(f"{arch}.attention.sliding_window_pattern")
    if pat is not None:
        args["layer_global"] = [0 if s else 1 for s in pat]
    args.update(overrides)
    for f in ("theta_local", "theta_global", "eps", "softcap"):
        if f in args:
            args[f] = float(args[f])
    return E4BConfig(**args)


_INT_FIELDS = ("hidden", "layers", "q_heads", "kv_heads", "head_dim", "ffn", "ple_dim", "vocab", "window", "ring",
               "max_seq", "rope_angles", "attn_chunk", "max_prompt", "flags", "recipe", "head_dim_full",
               "rope_angles_full", "n_experts", "expert_ffn")
_FLOAT_FIELDS = ("theta_local", "theta_global", "eps", "softcap")


def gguf_config(path: str, **overrides) -> E4BConfig:
    """The engine configuration of a GGUF file as the library reads it
    (e4b_gguf_config); fields the file cannot hold (ring, max_seq, ...) come
    from the E4BConfig defaults or `overrides`."""
    base = E4BConfig(**overrides)
    c = ConfigC()
    for f in _INT_FIELDS:
        setattr(c, f, int(getattr(base, f)))
    for f in _FLOAT_FIELDS:
        setattr(c, f, float(getattr(base, f)))
    lg = np.zeros(4096, np.uint8)
    kvh = np.zeros(4096, np.int32)
    check(lib.e4b_gguf_config(path.encode(), C.byref(c), _p(lg), _p(kvh), lg.size), "e4b_gguf_config")
    args = {f: getattr(c, f) for f in _INT_FIELDS}
    args.update({f: float(getattr(c, f)) for f in _FLOAT_FIELDS})
    if c.layer_global:
        args["layer_global"] = [int(x) for x in lg[:c.layers]]
    elif "layer_global" in overrides:
        args["layer_global"] = list(overrides["layer_global"])
    if c.layer_kv_heads:
        args["layer_kv_heads"] = [int(x) for x in kvh[:c.layers]]
    elif "layer_kv_heads" in overrides:
        args["layer_kv_heads"] = list(overrides["layer_kv_heads"])
    return E4BConfig(**args)


# long-context constants of the reference (src/engine-a4b.js:18-20)
KV_BUDGET = 640   # full-layer entries after a compaction
KV_DECAP = 768    # decode recompaction threshold
KV_PROTECT = 64   # newest entries always kept


class Engine:
    def __init__(self, cfg: E4BConfig, tensors=None):
        self.cfg = cfg
        c = ConfigC()
        for f in _INT_FIELDS:
            setattr(c, f, int(getattr(cfg, f)))
        for f in _FLOAT_FIELDS:
            setattr(c, f, float(getattr(cfg, f)))
        self._lg = np.ascontiguousarray(np.asarray(cfg.layer_global, np.uint8))
        c.layer_global = _p(self._lg)
        self._kvh = None
        if cfg.layer_kv_heads:
            self._kvh = np.ascontiguousarray(np.asarray(cfg.layer_kv_heads, np.int32))
            c.layer_kv_heads = _p(self._kvh)
        ctx = lib.e4b_create(C.byref(c))
        if not ctx:
            check(-1, "e4b_create")
        self.ctx = C.c_void_p(ctx)
        if tensors is not None:
            for t in (tensors.values() if isinstance(tensors, dict) else tensors):
                self.set_tensor(t.name, t.ggml_type, t.dims, t.data)
            self.finalize()

    # ---- loading (src/gguf.js fetch -> upload) ------------------------------
    def set_tensor(self, name: str, ggml_type: int, dims, data) -> None:
        data = np.ascontiguousarray(data)
        d = (C.c_int64 * len(dims))(*[int(x) for x in dims])
        check(lib.e4b_set_tensor(self.ctx, name.encode(), int(ggml_type), d, len(dims), _p(data), data.nbytes),
              f"e4b_set_tensor({name})")

    def finalize(self) -> None:
        check(lib.e4b_finalize(self.ctx), "e4b_finalize")

    @classmethod
    def load_native(cls, path: str, **overrides) -> "Engine":
        """Load through the library's own GGUF loader (e4b_gguf_config +
        e4b_load_gguf: the file is memory-mapped and uploaded tensor by
        tensor without passing through Python)."""
        cfg = gguf_config(path, **overrides)
        eng = cls(cfg)
        check(lib.e4b_load_gguf(eng.ctx, path.encode()), "e4b_load_gguf")
        eng.finalize()
        return eng

    @classmethod
    def from_gguf(cls, path: str, **overrides) -> "Engine":
        g = open_gguf(path)
        arch = g.kv.get("general.architecture", ARCH)
        emb = g.tensors.get("token_embd.weight")
        if f"{arch}.vocab_size" not in g.kv and emb is not None and len(emb["dims"]) >= 2:
            overrides.setdefault("vocab", int(emb["dims"][1]))  # the embedding's row count
        cfg = config_from_kv(g.kv, **overrides)
        eng = cls(cfg)
        for name in g.tensors:
            t = g.fetch(name)
            eng.set_tensor(name, t["type"], t["dims"], t["buf"])
        eng.finalize()
        return eng

    # ---- the token loop -----------------------------------------------------
    def step(self, token: int, pos: int, want_logits: bool = False):
        """One decode step (src/engine-a4b.js:695-705); returns the argmax
        token, plus the logits when asked."""
        am = C.c_uint32(0)
        lg = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        check(lib.e4b_step(self.ctx, int(token), int(pos), _p(lg), C.byref(am)), "e4b_step")
        return (int(am.value), lg) if want_logits else int(am.value)

    def argmax_fast(self) -> int:
        am = C.c_uint32(0)
        check(lib.e4b_argmax(self.ctx, C.byref(am)), "e4b_argmax")
        return int(am.value)

    def prefill(self, ids) -> int:
        ids = np.ascontiguousarray(np.asarray(ids, np.uint32))
        am = C.c_uint32(0)
        check(lib.e4b_prefill(self.ctx, _p(ids), ids.size, C.byref(am)), "e4b_prefill")
        return int(am.value)

    def decode_chunk(self, start_pos: int, count: int) -> np.ndarray:
        """GPU-fed greedy decode (src/engine-a4b.js:786-824): `count` tokens,
        each fed with the previous argmax, starting at start_pos."""
        out = np.empty(count, np.uint32)
        check(lib.e4b_decode(self.ctx, int(start_pos), int(count), _p(out)), "e4b_decode")
        return out

    def prefill_steps(self, ids) -> int:
        """The prompt token by token through the decode step (generateFast's
        prompt loop, src/engine-a4b.js:826-829), GPU-side between tokens."""
        ids = np.ascontiguousarray(np.asarray(ids, np.uint32))
        am = C.c_uint32(0)
        check(lib.e4b_prefill_steps(self.ctx, _p(ids), ids.size, C.byref(am)), "e4b_prefill_steps")
        return int(am.value)

    def generate_fast(self, ids, max_new: int, eos=(106, 1)) -> list:
        """generateFast (src/engine-a4b.js:826-848): the prompt through the
        decode step token by token, then GPU-fed chunks of <= 8 with an EOS
        check after each chunk readback."""
        return self._generate(self.prefill_steps(ids), len(ids), max_new, eos)

    def generate_prefill(self, ids, max_new: int, eos=(106, 1)) -> list:
        """generatePrefill (src/engine-a4b.js:659-681): the batched prefill,
        then the same GPU-fed decode loop as generate_fast."""
        return self._generate(self.prefill(ids), len(ids), max_new, eos)

    def _generate(self, g0: int, n_prompt: int, max_new: int, eos) -> list:
        eos = set(eos)
        out = [g0]
        if g0 in eos:
            return out
        pos, done = n_prompt, 1
        while done < max_new:
            n = min(8, max_new - done)
            toks = self.decode_chunk(pos, n)
            pos += n
            stop = False
            for t in toks.tolist():
                out.append(int(t))
                if t in eos:
                    stop = True
                    break
            done += n
            if stop:
                break
        return out[:max_new]

    # ---- per-dispatch profiles (src/engine-a4b.js:707-779) ---------------------
    def _profile(self, fn, *args) -> dict:
        out = (ProfEntryC * 64)()
        n = check(fn(self.ctx, *args, out, 64), fn.__name__)
        return {out[i].name.decode(): {"us": float(out[i].us), "n": int(out[i].n)} for i in range(min(n, 64))}

    def profile_step(self, token: int, pos: int) -> dict:
        """profileStep: one step with a timed span per dispatch, summed per
        kernel role -> {role: {"us", "n"}} (ranking only).  Runs a real step."""
        return self._profile(lib.e4b_profile_step, int(token), int(pos))

    def profile_prefill(self, ids) -> dict:
        """profilePrefill: one batched-prefill chunk (the first <= 512 tokens)
        with a timed span per dispatch, summed per role.  Leaves the caches
        holding the chunk; prefill again before decoding."""
        ids = np.ascontiguousarray(np.asarray(ids, np.uint32))
        return self._profile(lib.e4b_profile_prefill, _p(ids), ids.size)

    # ---- full-layer KV budget (src/engine-a4b.js:587-657) ------------------------
    def kv_count(self) -> int:
        """Entries in the full layers' caches (the reference's kvCount)."""
        return check(lib.e4b_kv_count(self.ctx), "e4b_kv_count")

    def read_scores(self, layer: int) -> np.ndarray:
        """Accumulated attention mass [q_heads][max_seq] of a full layer
        (needs FLAG_KV_SCORE)."""
        out = np.empty((self.cfg.q_heads, self.cfg.max_seq), np.float32)
        check(lib.e4b_read_scores(self.ctx, int(layer), _p(out)), "e4b_read_scores")
        return out

    def compact(self, budget: int = KV_BUDGET, protect: int = KV_PROTECT) -> int:
        """compactAll (src/engine-a4b.js:587-617); returns the new entry count."""
        return check(lib.e4b_kv_compact(self.ctx, int(budget), int(protect)), "e4b_kv_compact")

    def generate_long(self, ids, max_new: int, eos=(106, 1), budget: int = KV_BUDGET, protect: int = KV_PROTECT,
                      decap: int = KV_DECAP) -> list:
        """generateLong (src/engine-a4b.js:620-657): prefill; when the full
        layers hold more than `decap` entries, one scored probe step on the
        whole cache, then compaction to `budget`; then GPU-fed chunks of <= 8,
        compacting again before a chunk would pass `decap`.  Needs
        FLAG_KV_SCORE."""
        eos = set(eos)
        g0 = self.prefill(ids)
        out = [g0]
        if g0 in eos:
            return out
        pos, done = len(ids), 1
        if self.kv_count() > decap:
            t = int(self.decode_chunk(pos, 1)[0])
            pos += 1
            out.append(t)
            done = 2
            self.compact(budget, protect)
            if t in eos:
                return out
        while done < max_new:
            if self.kv_count() + 8 > decap:
                self.compact(budget, protect)
            n = min(8, max_new - done)
            toks = self.decode_chunk(pos, n)
            pos += n
            stop = False
            for t in toks.tolist():
                out.append(int(t))
                if t in eos:
                    stop = True
                    break
            done += n
            if stop:
                break
        return out[:max_new]

    def time_decode(self, start_pos: int, count: int) -> float:
        ms = C.c_float(0)
        check(lib.e4b_time_decode(self.ctx, int(start_pos), int(count), C.byref(ms)), "e4b_time_decode")
        return float(ms.value)

    # ---- inspection -----------------------------------------------------------
    def read_hidden(self) -> np.ndarray:
        out = np.empty(self.cfg.hidden, np.float32)
        check(lib.e4b_read_hidden(self.ctx, _p(out)), "e4b_read_hidden")
        return out

    def read_layer_hidden(self, layer: int) -> np.ndarray:
        """The residual stream after `layer` in the last decode step."""
        out = np.empty(self.cfg.hidden, np.float32)
        check(lib.e4b_read_layer_hidden(self.ctx, int(layer), _p(out)), "e4b_read_layer_hidden")
        return out

    def read_topk(self, layer: int):
        """A4B recipe: (expert ids [8], router weights [8]) of `layer` in the
        last decode step."""
        idx = np.empty(8, np.uint32)
        w = np.empty(8, np.float32)
        check(lib.e4b_read_topk(self.ctx, int(layer), _p(idx), _p(w)), "e4b_read_topk")
        return idx, w

    def read_logits(self) -> np.ndarray:
        out = np.empty(self.cfg.vocab, np.float32)
        check(lib.e4b_read_logits(self.ctx, _p(out)), "e4b_read_logits")
        return out

    def kv_slots(self, layer: int) -> int:
        return check(lib.e4b_kv_slots(self.ctx, layer), "e4b_kv_slots")

    def read_kv(self, layer: int):
        """(k, v) caches of a layer as uint16 (f16 bits) [kv_heads][slots][head_dim]."""
        slots = self.kv_slots(layer)
        kvh, hd, _, _ = self.cfg.layer_shape(layer)
        shape = (kvh, slots, hd)
        k = np.empty(shape, np.uint16)
        v = np.empty(shape, np.uint16)
        check(lib.e4b_read_kv(self.ctx, layer, _p(k), _p(v)), "e4b_read_kv")
        return k, v

    def reset(self) -> None:
        check(lib.e4b_reset(self.ctx), "e4b_reset")

    def close(self) -> None:
        if getattr(self, "ctx", None):
            lib.e4b_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
