"""The persistent layer loop (E4B_FLAG_PERSISTENT, k_persist.hip) against
the CPU oracle and against the kernel-chain engine.

The persistent kernel computes every layer of a step in one cooperative
launch; its phases hand vectors over through tagged words in device memory.
Tolerances are the engine tests' (tests/test_engine_gpu.py): tokens equal
unless the oracle's top-2 margin is a near-tie (2e-3 of max |logit|),
logits and hidden state within 1e-3 of max |oracle|, KV slot sets bit-exact
and values within 1e-2 (max) / 1e-3 (mean).  Against the kernel chain (same
weights, same inputs) the tokens must match and the logits agree within the
same 1e-3.
"""
import numpy as np
import pytest

import oracle as orc
from e4b._lib import FLAG_PERSISTENT
from e4b.engine import Engine
from e4b.model import E4BConfig, norm_weights_random, synth_tensors, tiny_config
from tests.test_engine_gpu import KV_MAX_TOL, KV_MEAN_TOL, LOGIT_TOL, TIE_TOL, lockstep
from tests.util import top2_margin

pytestmark = pytest.mark.gpu


def _pair(cfg, seed):
    tensors = norm_weights_random(synth_tensors(cfg, seed), seed + 1)
    import dataclasses
    pcfg = dataclasses.replace(cfg, flags=cfg.flags | FLAG_PERSISTENT)
    eng = Engine(pcfg, tensors)
    om = orc.OracleModel(cfg.as_dict(), {n: t.data for n, t in tensors.items()})
    return eng, om, tensors


def _kv_close(eng, om, cfg, layer):
    k, v = eng.read_kv(layer)
    slots = k.shape[1]
    n = slots * cfg.kv_heads * cfg.head_dim
    ok = om.kcache(layer, n).reshape(slots, cfg.kv_heads, cfg.head_dim).transpose(1, 0, 2)
    ov = om.vcache(layer, n).reshape(slots, cfg.kv_heads, cfg.head_dim).transpose(1, 0, 2)
    assert np.array_equal(np.any(k != 0, axis=(0, 2)), np.any(ok != 0, axis=(0, 2))), f"layer {layer} slots"
    for a, b in ((k, ok), (v, ov)):
        fa, fb = a.view(np.float16).astype(np.float64), b.view(np.float16).astype(np.float64)
        d = np.abs(fa - fb)
        assert d.max() <= KV_MAX_TOL * np.abs(fb).max(), f"layer {layer} (max)"
        assert d.mean() <= KV_MEAN_TOL * np.abs(fb).mean(), f"layer {layer} (mean)"


def test_persistent_tiny_lockstep():
    cfg = tiny_config()
    eng, om, _ = _pair(cfg, 11)
    prompt = np.random.default_rng(0).integers(0, cfg.vocab, 12)
    toks, ties, o_lg = lockstep(eng, om, prompt, 40)
    err = float(np.abs(eng.read_logits() - o_lg).max() / np.abs(o_lg).max())
    print(f"persistent tiny: {len(toks)} tokens, near-ties {ties}, logits err {err:.2e}")
    assert not ties and err < LOGIT_TOL
    for layer in range(cfg.layers):
        _kv_close(eng, om, cfg, layer)


def test_persistent_step_api_hidden_and_logits():
    cfg = tiny_config(layers=3, layer_global=[0, 1, 0])
    eng, om, _ = _pair(cfg, 23)
    for pos, t in enumerate(np.random.default_rng(3).integers(0, cfg.vocab, 20)):
        g, lg = eng.step(int(t), pos, want_logits=True)
        o_tok, o_lg, o_h = om.step(int(t), pos, want_logits=True, want_hidden=True)
        assert g == o_tok or top2_margin(o_lg) < TIE_TOL * np.abs(o_lg).max()
    err = float(np.abs(lg - o_lg).max() / np.abs(o_lg).max())
    herr = float(np.abs(eng.read_hidden() - o_h).max() / np.abs(o_h).max())
    print(f"persistent step api: logits err {err:.2e}, hidden err {herr:.2e}")
    assert err < LOGIT_TOL and herr < LOGIT_TOL


def test_persistent_matches_kernel_chain_e4b_width():
    # E4B-width layers (hidden 2048, ffn 16384, 256 blocks), 5 layers: the
    # persistent engine and the kernel chain on the same weights and tokens
    cfg = E4BConfig(layers=5, max_seq=512, layer_global=[0, 0, 0, 0, 1])
    eng, om, tensors = _pair(cfg, 3)
    chain = Engine(cfg, tensors)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab, 40)
    a = eng.generate_prefill(prompt, 24, eos=())
    la = eng.read_logits()
    b = chain.generate_prefill(prompt, 24, eos=())
    lb = chain.read_logits()
    err = float(np.abs(la - lb).max() / np.abs(lb).max())
    print(f"persistent vs chain: {a[:6]}... / {b[:6]}..., logits err {err:.2e}")
    assert a == b and err < LOGIT_TOL


@pytest.mark.slow
def test_persistent_c4_full_model_lockstep():
    cfg = E4BConfig(max_seq=1024)
    eng, om, _ = _pair(cfg, 0)
    prompt = np.random.default_rng(2).integers(0, cfg.vocab, 8)
    toks, ties, o_lg = lockstep(eng, om, prompt, 16)
    err = float(np.abs(eng.read_logits() - o_lg).max() / np.abs(o_lg).max())
    print(f"persistent c4 full: near-ties {ties}, logits err {err:.2e}")
    assert not ties and err < LOGIT_TOL
