"""The resident harness's correctness commands (resident-a4b.html:96-101:
gate, gate2, stats) in both hosts (e4b/resident.py, js/resident.js).

CPU: the goldens reader and the gate's reporting on a stand-in engine
(MATCH / MISMATCH lines, the first divergence, GATE PASS / FAIL, the
prompt filter), the hosts' Q6_K row decoders against the oracle's.

GPU: a tiny A4B-recipe model written to a gemma4 GGUF file with a goldens
file in the goldens-a4b.json layout whose greedy ids come from the CPU
oracle; both hosts pass the gate and the batched-prefill gate on it, a
goldens file with one id changed fails at that index; stats reports the
embedding row and every layer's residual stream, equal between the hosts
and to the oracle's per-layer hidden state within 1e-3.  (The real-model
gate against goldens/goldens-a4b.json needs the 14.4 GB 26B-A4B GGUF, which
is not in this image.)
"""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle as orc
from e4b import formats
from e4b.resident import gate, load_goldens, stats
from tests.util import top2_margin

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
JS = os.path.join(ROOT, "e4b-webgpu_amd", "js")
NODE = shutil.which("node")
_has_node = NODE is not None and os.path.exists(os.path.join(JS, "e4b_napi.node"))
EOS = (106, 1)
TIE_TOL = 2e-3    # an argmax top-2 margin below this (of max |logit|) is a near-tie
ROUTE_TIE = 1e-3  # a top-8 decision margin (of max |score|) below this is a routing near-tie


class _Stub:
    """generate_fast / generate_prefill returning fixed sequences."""

    def __init__(self, seqs):
        self.seqs = seqs
        self.calls = []

    def generate_fast(self, ids, n):
        self.calls.append(("fast", tuple(ids), n))
        return self.seqs[tuple(ids)][:n]

    def generate_prefill(self, ids, n):
        self.calls.append(("prefill", tuple(ids), n))
        return self.seqs[tuple(ids)][:n]


def test_gate_reporting(tmp_path):
    gold = {"prompts": [{"input_ids": [2, 5], "generated_ids": [7, 8, 9]},
                        {"input_ids": [3], "generated_ids": [4, 4, 4]}]}
    path = tmp_path / "g.json"
    path.write_text(json.dumps(gold))
    g = load_goldens(str(path))
    lines = []
    stub = _Stub({(2, 5): [7, 8, 9], (3,): [4, 6, 4]})
    assert not gate(stub, g, n=3, log=lines.append)
    assert lines == ["[p0] MATCH got=[7, 8, 9] want=[7, 8, 9]", "[p1] MISMATCH got=[4, 6, 4] want=[4, 4, 4]",
                     "[p1] first divergence at 1", "GATE FAIL"]
    lines.clear()
    assert gate(stub, g, n=3, p=0, batched=True, log=lines.append)
    assert lines == ["[p0] MATCH got=[7, 8, 9] want=[7, 8, 9]", "GATE2 PASS"]
    assert stub.calls[-1] == ("prefill", (2, 5), 3)
    lines.clear()
    short = _Stub({(2, 5): [7, 8], (3,): [4, 4, 4]})  # stopped early (an EOS)
    assert not gate(short, g, n=3, log=lines.append)
    assert lines[1] == "[p0] first divergence at 2"
    bad = tmp_path / "bad.json"
    bad.write_text(json.dumps({"prompts": [{"input_ids": [1]}]}))
    with pytest.raises(ValueError):
        load_goldens(str(bad))


def test_q6k_row_decoders_match_the_oracle():
    w = formats.synth_q6k(9, 6, 768)
    for r in range(6):
        want = orc.q6k_row(w, 768, r)
        np.testing.assert_array_equal(formats.q6k_row(w, 768, r), want)
    if _has_node:
        code = ("const r = require('./resident.js'); const fs = require('fs');"
                "const b = fs.readFileSync(process.argv[1]); const out = [];"
                "for (let i = 0; i < 6; i++) out.push(Array.from(r.q6kRow(b, 768, i)));"
                "console.log(JSON.stringify(out));")
        import tempfile
        with tempfile.NamedTemporaryFile(suffix=".bin") as f:
            f.write(w.tobytes())
            f.flush()
            out = subprocess.run([NODE, "-e", code, f.name], cwd=JS, check=True, capture_output=True, text=True,
                                 timeout=60).stdout
        js = np.array(json.loads(out), np.float32)
        for r in range(6):
            np.testing.assert_array_equal(js[r], orc.q6k_row(w, 768, r))


def _model_and_goldens(tmp_path, n_new=12):
    from e4b.engine import config_to_kv
    from e4b.gguf import write_gguf
    from e4b.model import norm_weights_random, synth_tensors, tiny_a4b_config
    cfg = tiny_a4b_config(ring=8 + 512)
    tensors = norm_weights_random(synth_tensors(cfg, 159), 160)  # margins 1.7e-2 / 1.4e-3
    path = tmp_path / "a4b.gguf"
    write_gguf(str(path), config_to_kv(cfg), [(t.name, t.ggml_type, t.dims, t.data) for t in tensors.values()])
    om = orc.OracleModel(cfg.as_dict(), {n: t.data for n, t in tensors.items()})
    rng = np.random.default_rng(161)
    prompts = []
    margin, route = np.inf, np.inf  # the smallest argmax / top-8 margins of the golden steps
    for k in range(3):
        ids = [int(x) for x in rng.integers(0, cfg.vocab, 5 + 3 * k)]
        om.reset()
        gen = []

        def step(t, pos):
            nonlocal margin, route
            tok, lg, _ = om.step(t, pos, want_logits=True)
            margin = min(margin, top2_margin(lg) / np.abs(lg).max())
            route = min(route, om.route_margin())
            return tok

        for p, t in enumerate(ids):
            tok = step(t, p)
        for i in range(n_new):
            gen.append(int(tok))
            if tok in EOS:  # generateFast stops after an end-of-turn id
                break
            tok = step(tok, len(ids) + i)
        prompts.append({"text": f"synthetic {k}", "input_ids": ids, "generated_ids": gen, "generated_text": ""})
    # exact greedy ids are the bar only away from near-ties (the engine's
    # other tests allow an argmax or expert difference below these margins)
    assert margin > TIE_TOL and route > ROUTE_TIE, (margin, route)
    gold = tmp_path / "goldens.json"
    gold.write_text(json.dumps({"prompts": prompts}))
    return cfg, tensors, path, gold, prompts


@pytest.mark.gpu
def test_resident_gate_and_stats_both_hosts(tmp_path):
    from e4b._lib import FLAG_LAYER_HIDDEN
    from e4b.engine import Engine
    cfg, tensors, path, gold, prompts = _model_and_goldens(tmp_path)
    g = load_goldens(str(gold))
    eng = Engine.load_native(str(path), ring=cfg.ring, max_seq=cfg.max_seq, flags=FLAG_LAYER_HIDDEN)
    lines = []
    ok = gate(eng, g, n=12, log=lines.append)
    ok2 = gate(eng, g, n=12, batched=True, log=lines.append)
    print("\n".join(lines))
    assert ok and ok2, "the engine's greedy ids differ from the oracle's"
    bad = json.loads(gold.read_text())
    bad["prompts"][1]["generated_ids"][4] = (bad["prompts"][1]["generated_ids"][4] + 1) % cfg.vocab
    badp = tmp_path / "bad.json"
    badp.write_text(json.dumps(bad))
    lines = []
    assert not gate(eng, load_goldens(str(badp)), n=12, log=lines.append)
    assert "[p1] first divergence at 4" in lines and lines[-1] == "GATE FAIL"
    # stats: the oracle's residual stream after every layer at the same step
    emb = tensors["token_embd.weight"].data
    res = stats(eng, g, emb, log=print)
    om = orc.OracleModel(cfg.as_dict(), {n: t.data for n, t in tensors.items()})
    ids = prompts[0]["input_ids"]
    for p, t in enumerate(ids):
        om.step(t, p)
    assert res[0]["name"] == "embed"
    want_emb = orc.q6k_row(emb, cfg.hidden, ids[-1], float(np.float32(np.sqrt(cfg.hidden))))
    np.testing.assert_allclose(res[0]["meanAbs"], np.mean(np.abs(want_emb)), rtol=1e-6)
    for layer in range(cfg.layers):
        oh = om.layer_hidden(layer).astype(np.float64)
        assert res[layer + 1]["name"] == f"layer{layer}"
        gh = eng.read_layer_hidden(layer).astype(np.float64)
        err = np.abs(gh - oh).max() / (oh.max() - oh.min())
        assert err < 1e-3, f"layer {layer}: hidden err {err:.2e} of range"
        np.testing.assert_allclose(res[layer + 1]["meanAbs"], np.mean(np.abs(oh)), rtol=1e-3)
    eng.close()
    if not _has_node:
        pytest.skip("node or the N-API addon is missing")
    outs = {}
    for mode in ("gate", "gate2", "stats"):
        r = subprocess.run([NODE, os.path.join(JS, "resident.js"), str(path), str(gold), mode, "12"],
                           capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, r.stderr
        outs[mode] = r.stdout.strip().splitlines()
    print("\n".join(outs["gate"] + outs["stats"]))
    assert outs["gate"][-1] == "GATE PASS" and outs["gate2"][-1] == "GATE2 PASS"
    assert [ln.split(" got=")[0] for ln in outs["gate"][:-1]] == [f"[p{i}] MATCH" for i in range(3)]
    assert len(outs["stats"]) == cfg.layers + 1
    for ln, r in zip(outs["stats"], res):
        name, ma = ln.split(": meanAbs=")
        assert name == r["name"]
        np.testing.assert_allclose(float(ma.split()[0]), r["meanAbs"], rtol=0, atol=1e-4)
    r = subprocess.run([NODE, os.path.join(JS, "resident.js"), str(path), str(badp), "gate", "12", "1"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 1 and "[p1] first divergence at 4" in r.stdout
