"""GPU parity of the batched prefill (MFMA GEMMs + per-token kernels) with the
CPU oracle.

Attention kernel (e4b_k_attn_prefill): each query of a chunk at position p
against orc.attn_linear (global layer, keys [0, p]) or orc.attn_ring
(sliding ring with slot-scan position recovery, kernels/attnf32.wgsl) over the
same cache, including slots that already hold the chunk's later positions --
the ring is sized so every live key keeps its slot (ring >= window + M - 1),
and the recovered position of a later key is never live.  Tolerance: within
ATTN_TOL of max|out| (f16 output, as the decode attention test).

Engine: e4b_prefill (batched, several chunks when the prompt exceeds
ring - window + 1) in lock-step with the oracle's token-by-token step
(tests/test_engine_gpu.py tolerances: greedy tokens bit-exact outside
near-ties, logits within 1e-3 of the logit range, KV caches within 1e-2 max /
1e-3 mean relative), and against the engine's own token-by-token prefill
(E4B_FLAG_STEP_PREFILL) at E4B width with 512- and 520-token prompts.
"""
import numpy as np
import pytest

import oracle as orc
from e4b._lib import FLAG_STEP_PREFILL
from e4b.engine import Engine
from e4b.kernels import attn_prefill
from e4b.model import E4BConfig, norm_weights_random, synth_tensors, tiny_config
from tests.test_engine_gpu import KV_MAX_TOL, KV_MEAN_TOL, LOGIT_TOL, TIE_TOL, build, lockstep
from tests.util import top2_margin

pytestmark = pytest.mark.gpu

ATTN_TOL = 2e-3
HD = 256


@pytest.mark.parametrize("gqa,kvh,slots,window,p0,m,seed", [
    (4, 2, 4096, 0, 0, 512, 1),      # c4 prompt, global layer
    (4, 2, 4096, 0, 1000, 100, 2),   # a later chunk of a global layer
    (4, 2, 1024, 512, 0, 513, 3),    # the largest chunk a 1024-slot ring allows
    (4, 2, 1024, 512, 900, 200, 4),  # ring wraps inside the chunk
    (4, 2, 1024, 512, 3000, 37, 5),  # ragged chunk deep in the ring
    (4, 1, 64, 32, 100, 33, 6),      # small ring at its chunk limit, one KV group
    (4, 2, 1024, 512, 7, 1, 7),      # a single token
    (4, 2, 8320, 0, 8000, 64, 8),    # deep global chunk: 8 key splits of 1024
    # two q heads per KV group (the A4B sliding layers: 16 q / 8 KV heads,
    # window 1024, ring 1536) and one: 32- and 64-query workgroup tiles
    (2, 8, 1536, 1024, 0, 512, 9),   # the A4B prompt
    (2, 8, 1536, 1024, 1300, 237, 10),  # ring wraps, ragged last tile
    (2, 3, 64, 32, 100, 33, 11),     # small ring at its chunk limit
    (2, 2, 1024, 512, 5, 1, 12),     # a single token
    (2, 2, 4096, 0, 2000, 90, 13),   # global layer
    (1, 4, 1024, 512, 600, 77, 14),  # one q head per KV head
])
def test_attn_prefill(gqa, kvh, slots, window, p0, m, seed):
    qh = gqa * kvh
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((m, qh, HD)).astype(np.float32)
    k = (0.25 * rng.standard_normal((kvh, slots, HD))).astype(np.float16)
    v = rng.standard_normal((kvh, slots, HD)).astype(np.float16)
    got = attn_prefill(q, k, v, window, p0).astype(np.float64)
    ko = np.ascontiguousarray(k.transpose(1, 0, 2)).view(np.uint16)  # oracle layout [slot][kvh][hd]
    vo = np.ascontiguousarray(v.transpose(1, 0, 2)).view(np.uint16)
    worst = 0.0
    for i in range(m):
        pos = p0 + i
        if window:
            want = orc.attn_ring(q[i].ravel(), ko, vo, qh, kvh, HD, slots, window, pos)
        else:
            want = orc.attn_linear(q[i].ravel(), ko, vo, qh, kvh, HD, pos + 1)
        want = want.view(np.float16).astype(np.float64)
        err = np.abs(got[i] - want).max() / np.abs(want).max()
        worst = max(worst, err)
        assert err < ATTN_TOL, f"query {i} (pos {pos}): rel err {err:.3e}"
    print(f"attn prefill gqa={gqa} kvh={kvh} slots={slots} window={window} p0={p0} m={m}: worst rel err {worst:.2e}")


def test_attn_prefill_rejects_short_ring():
    q = np.zeros((40, 8, HD), np.float32)
    k = np.zeros((2, 64, HD), np.float16)
    with pytest.raises(Exception):
        attn_prefill(q, k, k, 32, 0)  # 64 slots < 32 + 40 - 1


def _kv_check(eng, om, cfg, layer):
    k, v = eng.read_kv(layer)
    slots = k.shape[1]
    ok = om.kcache(layer, slots * cfg.kv_heads * cfg.head_dim).reshape(slots, cfg.kv_heads, cfg.head_dim)
    ov = om.vcache(layer, slots * cfg.kv_heads * cfg.head_dim).reshape(slots, cfg.kv_heads, cfg.head_dim)
    ok, ov = ok.transpose(1, 0, 2), ov.transpose(1, 0, 2)
    assert np.array_equal(np.any(k != 0, axis=(0, 2)), np.any(ok != 0, axis=(0, 2))), f"layer {layer}: written slots"
    for a, b in ((k, ok), (v, ov)):
        fa = a.view(np.float16).astype(np.float64)
        fb = b.view(np.float16).astype(np.float64)
        d = np.abs(fa - fb)
        assert d.max() <= KV_MAX_TOL * np.abs(fb).max(), f"layer {layer} cache values (max)"
        assert d.mean() <= KV_MEAN_TOL * np.abs(fb).mean(), f"layer {layer} cache values (mean)"


@pytest.mark.parametrize("n_prompt", [1, 9, 40])
def test_tiny_batched_prefill_lockstep(n_prompt):
    # tiny config: window 8, ring 16 -> chunks of 9 tokens; 40 tokens = five
    # chunks with the ring wrapping twice
    cfg = tiny_config()
    eng, om = build(cfg, 31 + n_prompt)
    prompt = np.random.default_rng(n_prompt).integers(0, cfg.vocab, n_prompt)
    toks, ties, o_lg = lockstep(eng, om, prompt, 10)
    print(f"tiny batched prefill {n_prompt}: near-ties {ties}")
    assert len(ties) == 0
    err = float(np.max(np.abs(eng.read_logits() - o_lg)) / np.max(np.abs(o_lg)))
    assert err < LOGIT_TOL
    for layer in range(cfg.layers):
        _kv_check(eng, om, cfg, layer)


def test_tiny_batched_prefill_hidden_and_logits():
    # after the prefill alone: the last token's hidden state and logits
    cfg = tiny_config(layers=3, layer_global=[0, 1, 0])
    eng, om = build(cfg, 77)
    prompt = np.random.default_rng(5).integers(0, cfg.vocab, 23)
    g = eng.prefill(prompt)
    for i, t in enumerate(prompt):
        o_tok, o_lg, o_h = om.step(int(t), i, want_logits=True, want_hidden=True)
    lg = eng.read_logits()
    err = float(np.max(np.abs(lg - o_lg)) / np.max(np.abs(o_lg)))
    herr = float(np.max(np.abs(eng.read_hidden() - o_h)) / np.max(np.abs(o_h)))
    print(f"tiny prefill-only logits err {err:.2e} hidden err {herr:.2e}")
    assert err < LOGIT_TOL and herr < LOGIT_TOL
    assert g == o_tok or top2_margin(o_lg) < TIE_TOL * np.abs(o_lg).max()
    assert eng.argmax_fast() == g


def test_tiny_no_ple_batched_prefill():
    cfg = tiny_config(ple_dim=0)
    eng, om = build(cfg, 55)
    prompt = np.random.default_rng(6).integers(0, cfg.vocab, 20)
    toks, ties, o_lg = lockstep(eng, om, prompt, 6)
    assert len(ties) == 0
    for layer in range(cfg.layers):
        _kv_check(eng, om, cfg, layer)


@pytest.mark.parametrize("n", [512, 520])
def test_c4_width_prefill_matches_step_prefill(n):
    # E4B width (5 layers, one global): a 512-token prompt (one chunk) and a
    # 520-token one (chunks of 512 and 8) through the batched prefill and
    # through the decode step; same continuation, logits and KV
    cfg = E4BConfig(layers=5, max_seq=1024, layer_global=[0, 0, 0, 0, 1])
    tensors = norm_weights_random(synth_tensors(cfg, 13), 14)
    a = Engine(cfg, tensors)
    b = Engine(E4BConfig(layers=5, max_seq=1024, layer_global=[0, 0, 0, 0, 1], flags=FLAG_STEP_PREFILL), tensors)
    prompt = np.random.default_rng(15).integers(0, cfg.vocab, n)
    ga, gb = a.prefill(prompt), b.prefill(prompt)
    la, lb = a.read_logits(), b.read_logits()
    err = float(np.max(np.abs(la - lb)) / np.max(np.abs(lb)))
    print(f"c4-width {n}-token prefill: batched {ga} step {gb}, logits err {err:.2e}")
    assert err < LOGIT_TOL
    assert ga == gb or top2_margin(lb) < TIE_TOL * np.abs(lb).max()
    for layer in range(cfg.layers):
        ka, va = a.read_kv(layer)
        kb, vb = b.read_kv(layer)
        for x, y in ((ka, kb), (va, vb)):
            fx = x.view(np.float16).astype(np.float64)
            fy = y.view(np.float16).astype(np.float64)
            d = np.abs(fx - fy)
            assert d.max() <= KV_MAX_TOL * np.abs(fy).max(), f"layer {layer} cache (max)"
            assert d.mean() <= KV_MEAN_TOL * np.abs(fy).mean(), f"layer {layer} cache (mean)"
    # the decode continuation from both
    ta = a.decode_chunk(n, 8)
    tb = b.decode_chunk(n, 8)
    print(f"continuations {ta.tolist()} / {tb.tolist()}")
    assert np.array_equal(ta, tb)


@pytest.mark.parametrize("n2", [9, 18, 19])
def test_prefill_again_after_decode_matches_fresh_engine(n2):
    # a second prefill (positions restart at 0) over caches that still hold
    # the first prompt and its decode: every key a query reads is rewritten
    # first, so tokens, logits and the written cache rows equal a fresh
    # engine's; n2 covers one chunk exactly (9 = ring - window + 1), two, and
    # two plus one token
    cfg = tiny_config()
    tensors = norm_weights_random(synth_tensors(cfg, 83), 84)
    a, b = Engine(cfg, tensors), Engine(cfg, tensors)
    rng = np.random.default_rng(n2)
    p1 = rng.integers(0, cfg.vocab, 30)
    p2 = rng.integers(0, cfg.vocab, n2)
    a.prefill(p1)
    a.decode_chunk(30, 10)
    ga, gb = a.prefill(p2), b.prefill(p2)
    assert ga == gb
    assert np.array_equal(a.read_logits(), b.read_logits())
    ta, tb = a.decode_chunk(n2, 8), b.decode_chunk(n2, 8)
    assert np.array_equal(ta, tb)
    assert np.array_equal(a.read_logits(), b.read_logits())


def test_long_prompt_batched_equals_step_prefill():
    # 2000 tokens through 223 ring-limited chunks of 9; the global layer's
    # later chunks split their up to 2000 keys over 8 workgroups.  The batched
    # prefill and the token-by-token prefill of the same engine agree on the
    # continuation, the logits and every cache.
    cfg = tiny_config(layers=3, layer_global=[0, 1, 0], max_seq=2048)
    tensors = norm_weights_random(synth_tensors(cfg, 91), 92)
    a = Engine(cfg, tensors)
    b = Engine(tiny_config(layers=3, layer_global=[0, 1, 0], max_seq=2048, flags=FLAG_STEP_PREFILL), tensors)
    prompt = np.random.default_rng(93).integers(0, cfg.vocab, 2000)
    ga, gb = a.prefill(prompt), b.prefill(prompt)
    la, lb = a.read_logits(), b.read_logits()
    err = float(np.max(np.abs(la - lb)) / np.max(np.abs(lb)))
    print(f"2000-token prompt: batched {ga} step {gb}, logits err {err:.2e}")
    assert err < LOGIT_TOL
    assert ga == gb or top2_margin(lb) < TIE_TOL * np.abs(lb).max()
    for layer in range(cfg.layers):
        ka, va = a.read_kv(layer)
        kb, vb = b.read_kv(layer)
        for x, y in ((ka, kb), (va, vb)):
            fx = x.view(np.float16).astype(np.float64)
            fy = y.view(np.float16).astype(np.float64)
            d = np.abs(fx - fy)
            assert d.max() <= KV_MAX_TOL * np.abs(fy).max(), f"layer {layer} cache (max)"
            assert d.mean() <= KV_MEAN_TOL * np.abs(fy).mean(), f"layer {layer} cache (mean)"
    assert np.array_equal(a.decode_chunk(2000, 8), b.decode_chunk(2000, 8))
