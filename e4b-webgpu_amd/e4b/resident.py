"""The resident harness's correctness commands over the engine
(resident-a4b.html:96-101 and its runCmd branches, :115-206):

  gate   for every prompt of a goldens file (or only prompt p): the first n
         generated ids by generateFast (the prompt through the decode step,
         then GPU-fed decode) against the file's greedy ids; one
         "[p<i>] MATCH|MISMATCH got=[...] want=[...]" line per prompt, the
         first divergence on a mismatch, then "GATE PASS" or "GATE FAIL".
  gate2  the same after the batched prefill (generatePrefill).
  stats  prompt 0 stepped up to its last token, then the last token's step;
         the embedding row and the residual stream after every layer as
         "layer<l>: meanAbs=... first4=[...]" (a NaN / explosion check),
         stopping at the first non-finite layer.

A goldens file is JSON {"prompts": [{"input_ids": [...], "generated_ids":
[...], ...}, ...]} (the layout of goldens/goldens-a4b.json).

    python -m e4b.resident model.gguf goldens.json gate [--n 24] [--p 1]
    python -m e4b.resident model.gguf goldens.json stats
"""
from __future__ import annotations

import argparse
import json
import math
import sys

import numpy as np

from ._lib import FLAG_LAYER_HIDDEN
from .formats import q6k_row


def load_goldens(path: str) -> dict:
    with open(path) as f:
        g = json.load(f)
    if not isinstance(g, dict) or not isinstance(g.get("prompts"), list):
        raise ValueError(f"{path}: not a goldens file (no 'prompts' list)")
    for i, p in enumerate(g["prompts"]):
        if not isinstance(p.get("input_ids"), list) or not isinstance(p.get("generated_ids"), list):
            raise ValueError(f"{path}: prompt {i} lacks input_ids / generated_ids")
    return g


def gate(eng, goldens: dict, n: int = 24, p=None, batched: bool = False, log=print) -> bool:
    """Token match of greedy generation against the goldens (gate / gate2)."""
    all_pass = True
    for pi, g in enumerate(goldens["prompts"]):
        if p is not None and pi != p:
            continue
        want = [int(t) for t in g["generated_ids"][:n]]
        gen = eng.generate_prefill if batched else eng.generate_fast
        got = [int(t) for t in gen([int(t) for t in g["input_ids"]], len(want))]
        match = got == want
        all_pass = all_pass and match
        log(f"[p{pi}] {'MATCH' if match else 'MISMATCH'} got={json.dumps(got)} want={json.dumps(want)}")
        if not match:
            first = next((i for i in range(max(len(got), len(want)))
                          if i >= len(got) or i >= len(want) or got[i] != want[i]), -1)
            log(f"[p{pi}] first divergence at {first}")
    log(("GATE2 " if batched else "GATE ") + ("PASS" if all_pass else "FAIL"))
    return all_pass


def _line(name: str, h: np.ndarray) -> dict:
    ma = float(np.mean(np.abs(h.astype(np.float64))))
    return {"name": name, "meanAbs": ma, "first4": [float(x) for x in h[:4]], "finite": math.isfinite(ma)}


def stats(eng, goldens: dict, embd_q6k=None, log=print) -> list:
    """Per-layer hidden meanAbs of prompt 0's last token.  The engine must be
    created with E4B_FLAG_LAYER_HIDDEN; embd_q6k (the raw Q6_K bytes of
    token_embd.weight) adds the embedding row's line."""
    ids = [int(t) for t in goldens["prompts"][0]["input_ids"]]
    for pos, t in enumerate(ids[:-1]):
        eng.step(t, pos)
    eng.step(ids[-1], len(ids) - 1)
    out = []
    if embd_q6k is not None:
        H = eng.cfg.hidden
        out.append(_line("embed", q6k_row(embd_q6k, H, ids[-1]) * np.float32(math.sqrt(H))))
    for layer in range(eng.cfg.layers):
        out.append(_line(f"layer{layer}", eng.read_layer_hidden(layer)))
    for r in out:
        log(f"{r['name']}: meanAbs={r['meanAbs']:.4f} first4={[round(x, 4) for x in r['first4']]}")
        if not r["finite"]:
            break
    return out


def main(argv=None) -> int:
    from .engine import Engine
    from .gguf import open_gguf

    ap = argparse.ArgumentParser()
    ap.add_argument("model")
    ap.add_argument("goldens")
    ap.add_argument("mode", choices=["gate", "gate2", "stats"])
    ap.add_argument("--n", type=int, default=24)
    ap.add_argument("--p", type=int, default=None)
    a = ap.parse_args(argv)
    goldens = load_goldens(a.goldens)
    eng = Engine.load_native(a.model, flags=FLAG_LAYER_HIDDEN)
    try:
        if a.mode == "stats":
            emb = open_gguf(a.model).fetch("token_embd.weight")["buf"]
            res = stats(eng, goldens, emb)
            return 0 if all(r["finite"] for r in res) else 1
        return 0 if gate(eng, goldens, a.n, a.p, batched=a.mode == "gate2") else 1
    finally:
        eng.close()


if __name__ == "__main__":
    sys.exit(main())
