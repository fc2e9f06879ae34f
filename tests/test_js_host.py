"""The JS host (N-API addon + engine.js, Node) over the same C ABI.

CPU: the addon loads and exports the engine surface; the Node GGUF reader
parses a file written by e4b.gguf.write_gguf into the same metadata, tensor
table and tensor bytes as the Python reader (open_gguf, itself the
restatement of src/gguf.js).

GPU: a tiny model written to GGUF, loaded once by the Python host
(Engine.from_gguf) and once by the JS host (node run_greedy.js); greedy
generation (batched prefill + GPU-fed decode) and the step API give the
same tokens on both (the same library and inputs: bit-identical).
"""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from e4b.engine import Engine, config_to_kv
from e4b.gguf import open_gguf, write_gguf
from e4b.model import norm_weights_random, synth_tensors, tiny_config

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
JS = os.path.join(ROOT, "e4b-webgpu_amd", "js")
NODE = shutil.which("node")

_needs_node = pytest.mark.skipif(NODE is None or not os.path.exists(os.path.join(JS, "e4b_napi.node")),
                                reason="node or the N-API addon is missing (build() makes the addon)")


def _node(code: str) -> str:
    return subprocess.run([NODE, "-e", code], cwd=JS, check=True, capture_output=True, text=True,
                          timeout=120).stdout


def _write_model(path, cfg, seed):
    tensors = norm_weights_random(synth_tensors(cfg, seed), seed + 1)
    write_gguf(str(path), config_to_kv(cfg), [(t.name, t.ggml_type, t.dims, t.data) for t in tensors.values()])
    return tensors


@_needs_node
def test_addon_exports_engine_surface():
    out = _node("const a = require('./e4b_napi.node'); console.log(JSON.stringify(Object.keys(a).sort()), a.version())")
    keys = json.loads(out.split()[0])
    for k in ("create", "setTensor", "finalize", "step", "prefill", "prefillSteps", "decode", "argmax", "readHidden",
              "readLogits", "kvCount", "readScores", "kvCompact", "profileStep", "profilePrefill", "reset", "destroy",
              "lastError", "deviceCount", "version"):
        assert k in keys
    assert "gfx950" in out


@_needs_node
def test_node_gguf_reader_matches_python(tmp_path):
    cfg = tiny_config(layers=2, layer_global=[0, 1])
    path = tmp_path / "m.gguf"
    _write_model(path, cfg, 3)
    g = open_gguf(str(path))
    code = f"""
const {{ openGGUF }} = require('./gguf');
(async () => {{
  const g = openGGUF({json.dumps(str(path))});
  const out = {{ kv: g.kv, dataStart: g.dataStart, tensors: {{}} }};
  for (const n of Object.keys(g.tensors)) {{
    const t = await g.fetch(n);
    let h = 0; for (const b of t.buf) h = (h * 31 + b) >>> 0;
    out.tensors[n] = {{ dims: t.dims, type: t.type, offset: t.offset, n: t.buf.length, h }};
  }}
  g.close();
  console.log(JSON.stringify(out));
}})();
"""
    js = json.loads(_node(code))
    assert js["dataStart"] == g.data_start
    for k, v in g.kv.items():
        jv = js["kv"][k]
        if isinstance(v, float):
            assert abs(jv - v) <= 1e-6 * max(1.0, abs(v))
        else:
            assert jv == v, k
    assert set(js["tensors"]) == set(g.tensors)
    for n, t in g.tensors.items():
        buf = np.asarray(g.fetch(n)["buf"])
        h = 0
        for b in buf.tobytes():
            h = (h * 31 + b) & 0xFFFFFFFF
        jt = js["tensors"][n]
        assert jt["dims"] == list(t["dims"]) and jt["type"] == t["type"] and jt["offset"] == t["offset"]
        assert jt["n"] == buf.size and jt["h"] == h, n


@_needs_node
@pytest.mark.gpu
def test_js_host_matches_python_host(tmp_path):
    cfg = tiny_config()
    path = tmp_path / "tiny.gguf"
    _write_model(path, cfg, 41)
    prompt = [int(x) for x in np.random.default_rng(41).integers(0, cfg.vocab, 12)]
    over = {"ring": cfg.ring, "maxSeq": cfg.max_seq}
    r = subprocess.run([NODE, os.path.join(JS, "run_greedy.js"), str(path), ",".join(map(str, prompt)), "24",
                        json.dumps(over)], check=True, capture_output=True, text=True, timeout=300)
    js = json.loads(r.stdout.strip().splitlines()[-1])
    eng = Engine.from_gguf(str(path), ring=cfg.ring, max_seq=cfg.max_seq)
    gen = eng.generate_fast(prompt, 24, eos=())
    eng.reset()
    steps = [eng.step(t, i) for i, t in enumerate(prompt)]
    h = eng.read_hidden()
    print(f"js host: generate {js['generate'][:8]}..., python {gen[:8]}...")
    assert js["generate"] == gen
    assert js["steps"] == steps
    assert abs(js["hidden_l2"] - float(np.sqrt((h.astype(np.float64) ** 2).sum()))) <= 1e-5 * js["hidden_l2"]


@_needs_node
@pytest.mark.gpu
def test_js_host_oracle_lockstep(tmp_path):
    # the JS host against the CPU oracle directly: generateFast's tokens are
    # replayed through orc_step (each oracle step fed the JS host's previous
    # token), every token equal to the oracle's argmax unless the oracle's
    # top-2 margin is a near-tie, final logits within 1e-3 of their range;
    # generatePrefill (batched prefill) yields the same tokens; both profiles
    # name the step's and the prefill chunk's kernel roles
    import oracle as orc
    from tests.util import top2_margin
    cfg = tiny_config(layers=3, layer_global=[0, 0, 1])
    path = tmp_path / "lock.gguf"
    tensors = _write_model(path, cfg, 47)
    prompt = [int(x) for x in np.random.default_rng(47).integers(0, cfg.vocab, 10)]
    over = {"ring": cfg.ring, "maxSeq": cfg.max_seq}
    lg_path = tmp_path / "logits.f32"
    env = dict(os.environ, E4B_LOGITS_OUT=str(lg_path))
    r = subprocess.run([NODE, os.path.join(JS, "run_greedy.js"), str(path), ",".join(map(str, prompt)), "20",
                        json.dumps(over)], check=True, capture_output=True, text=True, timeout=300, env=env)
    js = json.loads(r.stdout.strip().splitlines()[-1])
    toks = js["generate"]
    om = orc.OracleModel(cfg.as_dict(), {n: t.data for n, t in tensors.items()})
    for i, t in enumerate(prompt):
        o_tok, o_lg, _ = om.step(t, i, want_logits=True)
    ties = []
    for k in range(len(toks)):
        if toks[k] != o_tok:
            assert top2_margin(o_lg) < 2e-3 * np.abs(o_lg).max(), f"token {k}: js {toks[k]} vs oracle {o_tok}"
            ties.append(k)
        if k + 1 < len(toks):
            o_tok, o_lg, _ = om.step(toks[k], len(prompt) + k, want_logits=True)
    js_lg = np.fromfile(lg_path, np.float32)
    err = float(np.abs(js_lg - o_lg).max() / np.abs(o_lg).max())
    print(f"js host vs oracle: {len(toks)} tokens compared, near-ties {ties}, final logits err {err:.2e}")
    assert err < 1e-3
    assert js["generate_prefill"] == toks or ties
    for key, want in (("profile_step", ("embed", "qkv", "attn_sliding", "attn_global", "o_proj", "gate_up_geglu",
                                          "down", "ple", "lm_head")),
                      ("profile_prefill", ("embed_rows", "gemm_qkv", "attn_prefill", "gemm_gate_up_geglu"))):
        roles = {name: (n, pos) for name, n, pos in js[key]}
        for role in want:
            assert role in roles and roles[role][1], (key, role)
    assert dict((n, c) for n, c, _ in js["profile_step"])["qkv"] == cfg.layers


@_needs_node
@pytest.mark.gpu
def test_js_generate_long_matches_python_host(tmp_path):
    # generateLong (src/engine-a4b.js:620-657) on both hosts with a small
    # budget: probe step, compaction and recompactions take the same path
    from e4b._lib import FLAG_KV_SCORE
    cfg = tiny_config(layers=2, layer_global=[0, 1], max_seq=128)  # room for the driver's generateFast leg
    path = tmp_path / "long.gguf"
    _write_model(path, cfg, 61)
    prompt = [int(x) for x in np.random.default_rng(61).integers(0, cfg.vocab, 30)]
    over = {"ring": cfg.ring, "maxSeq": cfg.max_seq, "flags": FLAG_KV_SCORE}
    opts = {"budget": 16, "protect": 4, "decap": 24}
    r = subprocess.run([NODE, os.path.join(JS, "run_greedy.js"), str(path), ",".join(map(str, prompt)), "40",
                        json.dumps(over), json.dumps(opts)], check=True, capture_output=True, text=True, timeout=300)
    js = json.loads(r.stdout.strip().splitlines()[-1])
    eng = Engine.from_gguf(str(path), ring=cfg.ring, max_seq=cfg.max_seq, flags=FLAG_KV_SCORE)
    out = eng.generate_long(prompt, 40, eos=(), **opts)
    assert js["generate_long"] == out
    assert js["kv_count"] == eng.kv_count() <= opts["decap"]


@pytest.mark.gpu
def test_native_gguf_engine_oracle_lockstep(tmp_path):
    # an engine loaded through the library's own GGUF loader (e4b_load_gguf)
    # against the CPU oracle built from the same file's tensors
    import oracle as orc
    from tests.test_engine_gpu import lockstep
    cfg = tiny_config(layers=3, layer_global=[0, 1, 0])
    path = tmp_path / "native.gguf"
    tensors = _write_model(path, cfg, 57)
    eng = Engine.load_native(str(path), ring=cfg.ring, max_seq=cfg.max_seq)
    om = orc.OracleModel(cfg.as_dict(), {n: t.data for n, t in tensors.items()})
    prompt = np.random.default_rng(57).integers(0, cfg.vocab, 11)
    toks, ties, o_lg = lockstep(eng, om, prompt, 16)
    err = float(np.abs(eng.read_logits() - o_lg).max() / np.abs(o_lg).max())
    print(f"native gguf engine vs oracle: near-ties {ties}, logits err {err:.2e}")
    assert not ties and err < 1e-3


@pytest.mark.gpu
def test_native_gguf_loader_matches_python_loader(tmp_path):
    # the library's own mmap loader (e4b_gguf_config + e4b_load_gguf) and the
    # Python reader feeding e4b_set_tensor build the same engine
    cfg = tiny_config(layers=3, layer_global=[0, 0, 1])
    path = tmp_path / "m.gguf"
    _write_model(path, cfg, 52)
    prompt = [int(x) for x in np.random.default_rng(52).integers(0, cfg.vocab, 10)]
    a = Engine.load_native(str(path), ring=cfg.ring, max_seq=cfg.max_seq)
    b = Engine.from_gguf(str(path), ring=cfg.ring, max_seq=cfg.max_seq)
    ga, gb = a.generate_fast(prompt, 16, eos=()), b.generate_fast(prompt, 16, eos=())
    assert ga == gb
    assert np.array_equal(a.read_logits(), b.read_logits())


@_needs_node
def test_node_config_a4b_matches_python(tmp_path):
    # the JS loader's configFromKV reads a gemma4 key set (src/engine-a4b.js
    # :100-116) into the same A4B configuration as the Python and native
    # readers, the vocabulary from the embedding's rows when absent
    from e4b.engine import gguf_config
    from e4b.model import tiny_a4b_config
    cfg = tiny_a4b_config(layer_global=[0, 1, 0, 1], layer_kv_heads=[2, 1, 8, 2])
    kv = config_to_kv(cfg)
    del kv["gemma4.vocab_size"]
    path = tmp_path / "a4b.gguf"
    write_gguf(str(path), kv, [(t.name, t.ggml_type, t.dims, t.data) for t in synth_tensors(cfg, 3).values()])
    code = f"""
const {{ openGGUF }} = require('./gguf');
const {{ configFromKV }} = require('./engine');
const g = openGGUF({json.dumps(str(path))});
const emb = g.tensors['token_embd.weight'];
console.log(JSON.stringify(configFromKV(g.kv, {{ vocab: emb.dims[1], maxSeq: {cfg.max_seq} }})));
g.close();
"""
    js = json.loads(_node(code))
    nat = gguf_config(str(path), max_seq=cfg.max_seq)
    for jf, pf in (("recipe", "recipe"), ("hidden", "hidden"), ("layers", "layers"), ("qHeads", "q_heads"),
                   ("kvHeads", "kv_heads"), ("headDim", "head_dim"), ("headDimFull", "head_dim_full"),
                   ("ropeAngles", "rope_angles"), ("ropeAnglesFull", "rope_angles_full"), ("ffn", "ffn"),
                   ("nExperts", "n_experts"), ("expertFfn", "expert_ffn"), ("pleDim", "ple_dim"), ("vocab", "vocab"),
                   ("window", "window"), ("ring", "ring"), ("maxSeq", "max_seq"), ("layerGlobal", "layer_global"),
                   ("layerKvHeads", "layer_kv_heads")):
        assert js[jf] == getattr(nat, pf), jf
    for jf, pf in (("thetaLocal", "theta_local"), ("thetaGlobal", "theta_global"), ("eps", "eps"),
                   ("softcap", "softcap")):
        assert abs(js[jf] - getattr(nat, pf)) <= 1e-6 * abs(getattr(nat, pf)), jf
    assert nat.vocab == cfg.vocab and nat.layer_kv_heads == [2, 1, 8, 2]
