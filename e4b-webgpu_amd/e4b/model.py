"""Model descriptions and seeded random-init tensors.

The benchmark's "E4B-shaped q4_0" model combines Gemma-3n-E4B shapes (35 layers,
hidden 2048, GeGLU FFN 16384, 4 sliding : 1 global, per-layer embeddings of
256) with the A4B engine's formats (q4_0 linears, Q6_K tied embedding /
lm-head, f16 KV ring).  recipe = 1 describes the model the reference's live
engine loads (src/engine-a4b.js:100-199, the 26B-A4B MoE): hidden 2816, 16 q
heads, per-layer KV heads, full layers with head dim 512, a quarter of their
pairs rotated and V = K, and a MoE FFN half (128 experts, top 8, expert FFN
704) beside a dense GeGLU branch (2112).  Tensor names follow the GGUF
naming of each family; dims are ggml order (ne0 = row length).
"""
from __future__ import annotations

import dataclasses
from dataclasses import dataclass, field

import numpy as np

from ._lib import GGML_F32, GGML_Q4_0, GGML_Q6_K
from . import formats


@dataclass
class E4BConfig:
    hidden: int = 2048
    layers: int = 35
    q_heads: int = 8
    kv_heads: int = 2
    head_dim: int = 256
    ffn: int = 16384
    ple_dim: int = 256
    vocab: int = 262144
    window: int = 512
    ring: int = 1024
    max_seq: int = 4096
    rope_angles: int = 128
    theta_local: float = 1e4
    theta_global: float = 1e6
    eps: float = 1e-6
    softcap: float = 30.0
    layer_global: list = field(default_factory=list)
    attn_chunk: int = 0
    max_prompt: int = 0
    flags: int = 0
    # recipe 1 (A4B, src/engine-a4b.js:100-116): the full layers' head dim
    # and rotated pairs, the MoE shape, KV heads per layer (empty: kv_heads)
    recipe: int = 0
    head_dim_full: int = 0
    rope_angles_full: int = 0
    n_experts: int = 0
    expert_ffn: int = 0
    layer_kv_heads: list = field(default_factory=list)

    def __post_init__(self):
        if not self.layer_global:
            period = 6 if self.recipe == 1 else 5
            self.layer_global = [1 if i % period == period - 1 else 0 for i in range(self.layers)]

    def layer_shape(self, layer: int):
        """(kv_heads, head_dim, rotated pairs, V = K) of a layer."""
        glob = bool(self.layer_global[layer])
        kvh = self.layer_kv_heads[layer] if self.layer_kv_heads else self.kv_heads
        if self.recipe == 1 and glob:
            return kvh, self.head_dim_full or self.head_dim, self.rope_angles_full or self.rope_angles, True
        return kvh, self.head_dim, self.rope_angles, False

    def as_dict(self) -> dict:
        return dataclasses.asdict(self)

    def bytes_per_token(self, pos: int) -> int:
        """Algorithmic HBM bytes of one decode step at position `pos`: every
        weight read once (q4_0 18 B / 32, Q6_K 210 B / 256), the K/V rows the
        attention reads, the PLE table row and the logits written."""
        H, F, PD, L = self.hidden, self.ffn, self.ple_dim, self.layers
        qkv = (self.q_heads + 2 * self.kv_heads) * self.head_dim
        q40 = lambda r, c: r * c // 32 * 18  # noqa: E731
        per_layer = q40(qkv, H) + q40(H, self.q_heads * self.head_dim) + q40(2 * F, H) + q40(H, F)
        if PD:
            per_layer += q40(PD, H) + q40(H, PD)
        kv_row = 2 * self.kv_heads * self.head_dim * 2  # K and V, f16
        kv = 0
        for g in self.layer_global:
            live = pos + 1 if g else min(pos + 1, self.window)
            kv += live * kv_row
        head = self.vocab * H // 256 * 210 + self.vocab * 4
        ple = (q40(L * PD, H) + L * PD // 256 * 210) if PD else 0
        emb = H // 256 * 210
        if self.recipe == 1:
            return self._a4b_bytes(pos) + head + emb
        return L * per_layer + kv + head + ple + emb

    def _a4b_bytes(self, pos: int) -> int:
        """Per-token weight and KV bytes of the A4B recipe's layers: q|k(|v),
        o, the router (f32), the dense branch and the 8 active experts."""
        H, F, E, FE, QH = self.hidden, self.ffn, self.n_experts, self.expert_ffn, self.q_heads
        q40 = lambda r, c: r * c // 32 * 18  # noqa: E731
        total = 0
        for layer, g in enumerate(self.layer_global):
            kvh, hd, _, keqv = self.layer_shape(layer)
            total += q40((QH + (1 if keqv else 2) * kvh) * hd, H) + q40(H, QH * hd)
            total += E * H * 4 + q40(2 * F, H) + q40(H, F) + 8 * (q40(2 * FE, H) + q40(H, FE))
            live = pos + 1 if g else min(pos + 1, self.window)
            total += live * 2 * kvh * hd * 2
        return total


def tiny_config(**kw) -> E4BConfig:
    """Small model with the same code path (hidden 256, 5 layers, 1 global)."""
    base = dict(hidden=256, layers=5, q_heads=8, kv_heads=2, head_dim=256, ffn=512, ple_dim=256, vocab=1000,
                window=8, ring=16, max_seq=64, rope_angles=128)
    base.update(kw)
    return E4BConfig(**base)


def a4b_config(**kw) -> E4BConfig:
    """The A4B recipe at the reference model's shapes (src/engine-a4b.js
    :100-116): 30 layers, hidden 2816, 16 q heads, head dims 256 / 512 (a
    quarter of the full layers' pairs rotated), window 1024 in a 1536-slot
    ring, dense FFN 2112, 128 experts of 704; 5 sliding : 1 full layer and 8
    / 2 KV heads per sliding / full layer for random-init models (a GGUF
    file gives its own)."""
    base = dict(recipe=1, hidden=2816, layers=30, q_heads=16, kv_heads=8, head_dim=256, head_dim_full=512,
                ffn=2112, ple_dim=0, vocab=262144, window=1024, ring=1536, max_seq=4096, rope_angles=128,
                rope_angles_full=64, n_experts=128, expert_ffn=704)
    base.update(kw)
    cfg = E4BConfig(**base)
    if not cfg.layer_kv_heads:
        cfg.layer_kv_heads = [2 if g else cfg.kv_heads for g in cfg.layer_global]
    return cfg


def tiny_a4b_config(**kw) -> E4BConfig:
    """Small A4B-recipe model (hidden 256, 4 layers, the last one full)."""
    base = dict(hidden=256, layers=4, q_heads=8, kv_heads=4, ffn=128, vocab=1000, window=8, ring=16, max_seq=64,
                n_experts=16, expert_ffn=64, layer_global=[0, 0, 0, 1], layer_kv_heads=[4, 2, 4, 1])
    base.update(kw)
    return a4b_config(**base)


@dataclass
class Tensor:
    name: str
    ggml_type: int
    dims: tuple  # ggml order
    data: np.ndarray  # uint8 block bytes (quantized) or float32


def synth_tensors(cfg: E4BConfig, seed: int = 0, lin_sigma: float = 0.02, emb_sigma: float = 1e-3):
    """Random-init tensors of the E4B-shaped model (benchmark config c4):
    q4_0 linears with d = f16(|N(0, lin_sigma)|/8), Q6_K embedding / PLE table
    with d = f16(|N(0, emb_sigma)|), norm weights 1, layer scalars 1."""
    H, F, PD, L, V = cfg.hidden, cfg.ffn, cfg.ple_dim, cfg.layers, cfg.vocab
    QH, KVH, HD = cfg.q_heads, cfg.kv_heads, cfg.head_dim
    out = {}
    counter = [0]

    def sub():
        counter[0] += 1
        return (seed * 1000003 + counter[0]) & 0xFFFFFFFFFFFFFFFF

    def q40(name, rows, cols):
        out[name] = Tensor(name, GGML_Q4_0, (cols, rows), formats.synth_q40(sub(), rows, cols, lin_sigma))

    def q6k(name, rows, cols):
        out[name] = Tensor(name, GGML_Q6_K, (cols, rows), formats.synth_q6k(sub(), rows, cols, emb_sigma))

    def ones(name, n):
        sub()
        out[name] = Tensor(name, GGML_F32, (n,), np.ones(n, np.float32))

    q6k("token_embd.weight", V, H)
    ones("output_norm.weight", H)
    if cfg.recipe == 1:
        _synth_a4b_layers(cfg, out, sub, q40, ones, lin_sigma)
        return out
    if PD:
        q6k("per_layer_token_embd.weight", V, L * PD)
        q40("per_layer_model_proj.weight", L * PD, H)
        ones("per_layer_proj_norm.weight", PD)
    for i in range(L):
        p = f"blk.{i}."
        ones(p + "attn_norm.weight", H)
        q40(p + "attn_q.weight", QH * HD, H)
        q40(p + "attn_k.weight", KVH * HD, H)
        q40(p + "attn_v.weight", KVH * HD, H)
        ones(p + "attn_q_norm.weight", HD)
        ones(p + "attn_k_norm.weight", HD)
        q40(p + "attn_output.weight", H, QH * HD)
        ones(p + "post_attention_norm.weight", H)
        ones(p + "ffn_norm.weight", H)
        q40(p + "ffn_gate.weight", F, H)
        q40(p + "ffn_up.weight", F, H)
        q40(p + "ffn_down.weight", H, F)
        ones(p + "post_ffw_norm.weight", H)
        if PD:
            q40(p + "inp_gate.weight", PD, H)
            q40(p + "proj.weight", H, PD)
            ones(p + "post_norm.weight", H)
        out[p + "layer_output_scale.weight"] = Tensor(p + "layer_output_scale.weight", GGML_F32, (1,),
                                                      np.ones(1, np.float32))
    return out


def _synth_a4b_layers(cfg, out, sub, q40, ones, lin_sigma):
    """Layers of the A4B recipe: per-layer q|k(|v) widths, the dense branch,
    the router (f32 [E][H] ~ N(0, 0.02), as benchmark config c3), its input
    scale and the per-expert output scales (1), the expert tensors (3-d, one
    [2 FE][H] gate|up and one [H][FE] down matrix per expert) and the
    branch norms."""
    H, F, E, FE, QH = cfg.hidden, cfg.ffn, cfg.n_experts, cfg.expert_ffn, cfg.q_heads
    for i in range(cfg.layers):
        p = f"blk.{i}."
        kvh, hd, _, keqv = cfg.layer_shape(i)
        ones(p + "attn_norm.weight", H)
        q40(p + "attn_q.weight", QH * hd, H)
        q40(p + "attn_k.weight", kvh * hd, H)
        if not keqv:
            q40(p + "attn_v.weight", kvh * hd, H)
        ones(p + "attn_q_norm.weight", hd)
        ones(p + "attn_k_norm.weight", hd)
        q40(p + "attn_output.weight", H, QH * hd)
        ones(p + "post_attention_norm.weight", H)
        ones(p + "ffn_norm.weight", H)
        q40(p + "ffn_gate.weight", F, H)
        q40(p + "ffn_up.weight", F, H)
        q40(p + "ffn_down.weight", H, F)
        ones(p + "post_ffw_norm.weight", H)
        ones(p + "pre_ffw_norm_2.weight", H)
        ones(p + "post_ffw_norm_1.weight", H)
        ones(p + "post_ffw_norm_2.weight", H)
        name = p + "ffn_gate_inp.weight"
        out[name] = Tensor(name, GGML_F32, (H, E), formats.synth_normal(sub(), E * H, 0.0, 0.02))
        ones(p + "ffn_gate_inp.scale", H)
        ones(p + "ffn_down_exps.scale", E)
        name = p + "ffn_gate_up_exps.weight"
        out[name] = Tensor(name, GGML_Q4_0, (H, 2 * FE, E), formats.synth_q40(sub(), E * 2 * FE, H, lin_sigma))
        name = p + "ffn_down_exps.weight"
        out[name] = Tensor(name, GGML_Q4_0, (FE, H, E), formats.synth_q40(sub(), E * H, FE, lin_sigma))
        out[p + "layer_output_scale.weight"] = Tensor(p + "layer_output_scale.weight", GGML_F32, (1,),
                                                      np.ones(1, np.float32))


def norm_weights_random(tensors: dict, seed: int = 1, lo: float = 0.5, hi: float = 1.5) -> dict:
    """Replace the f32 norm and scale vectors by U(lo, hi) so that tests see
    every weight (the MoE router matrix keeps its N(0, 0.02) draw)."""
    rng = np.random.default_rng(seed)
    for t in tensors.values():
        if t.name.endswith("ffn_gate_inp.weight"):
            continue
        if t.ggml_type == GGML_F32 and t.data.size > 1:
            t.data = rng.uniform(lo, hi, t.data.size).astype(np.float32)
    return tensors
