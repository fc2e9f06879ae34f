"""Device-side timeline of graph-replayed decode steps.

The trace build of the library (``make -C e4b-webgpu_amd/csrc trace`` ->
``e4b-webgpu_amd/libe4b_trace.so``) makes every workgroup of every decode
kernel append (t_entry, t_exit, tag, workgroup) from the chip's real-time
counter to one device buffer (csrc/trace.h).  The records survive hipGraph
replay, so this module reports what a kernel-trace profiler cannot see here:
each kernel's span inside the captured step (first workgroup's entry to the
last workgroup's exit) and the gap the graph leaves before it.

    E4B_LIBRARY=e4b-webgpu_amd/libe4b_trace.so python -m e4b.timeline [--workload c4|a4b] [--steps N]

(run from e4b-webgpu_amd/, or with it on sys.path).  Prints a markdown table
per kernel role: launches per token, mean span, mean gap before it, and the
per-token sum of spans and gaps.
"""
from __future__ import annotations

import argparse
import ctypes as C
import os
import sys

import numpy as np

from ._lib import check, lib

TR_NAMES = {1: "q40", 2: "attn", 3: "ple", 4: "embed", 5: "ple_prep", 6: "tail", 7: "lm_head", 8: "feedback",
            9: "attn_gen", 10: "attn_merge", 11: "moe_router", 12: "moe_gu", 13: "moe_down", 14: "moe_tail",
            15: "rownorm"}

REC = np.dtype([("t0", "<u8"), ("t1", "<u8"), ("tag", "<u4"), ("blk", "<u4"), ("hw_id", "<u4"), ("xcc", "<u4"),
                ("mark", "<u4", (4,)), ("pad", "<u4", (4,))])


def tag_name(tag: int) -> str:
    fam, v = tag >> 16, tag & 0xFFFF
    name = TR_NAMES.get(fam, f"family{fam}")
    if fam == 1:
        prok = (v & 31) - 8
        epi = (v >> 5) & 7
        r = 1 << ((v >> 8) & 15)
        kind = {0: "f32", 1: "geglu", 2: "gelu_mul"}.get(epi, str(epi))
        pro = {0: "", -1: " attn-combine prologue", -2: " layer-boundary prologue",
               -3: " attn-combine prologue (4 heads of 256 a slice)",
               -4: " attn-combine prologue (4 heads of 512 a slice)"}.get(prok, f" prologue H={256 * prok}")
        extra = (" kw4" if (v >> 12) & 1 else "") + (" ksplit" if (v >> 13) & 1 else "") + \
            (" batched" if (v >> 14) & 1 else "")
        return f"q40 {kind} r{r}{pro}{extra}"
    if fam == 2:
        return "attn " + ("global" if v else "sliding")
    if fam == 9:
        return f"attn_gen hd{v}"
    return name


def capture(run, cap: int = 1 << 22) -> np.ndarray:
    """Run `run()` with the trace on; the records, sorted by entry time."""
    check(lib.e4b_trace_start(cap), "e4b_trace_start")
    try:
        run()
        n = C.c_size_t(0)
        buf = np.zeros(cap, REC)
        check(lib.e4b_trace_read(C.c_void_p(buf.ctypes.data), cap, C.byref(n)), "e4b_trace_read")
        if n.value > cap:
            raise RuntimeError(f"trace overflow: {n.value} records for a {cap}-record buffer")
        recs = buf[: n.value]
    finally:
        check(lib.e4b_trace_stop(), "e4b_trace_stop")
    return recs[np.argsort(recs["t0"], kind="stable")]


def launches(recs: np.ndarray) -> list:
    """Split entry-sorted records into launches.  Launches of one stream are
    ordered (every workgroup of launch k exits before any of launch k+1
    enters) and consecutive launches of the decode step differ in tag, so a
    launch is a maximal run of one tag."""
    out = []
    if recs.size == 0:
        return out
    tags = recs["tag"]
    cut = np.flatnonzero(np.diff(tags.astype(np.int64)) != 0) + 1
    for a, b in zip(np.r_[0, cut], np.r_[cut, recs.size]):
        seg = recs[a:b]
        out.append({"tag": int(seg["tag"][0]), "wgs": int(b - a), "t0": int(seg["t0"].min()),
                    "t1": int(seg["t1"].max()), "t0_med": float(np.median(seg["t0"])),
                    "t1_med": float(np.median(seg["t1"]))})
    return out


def summarize(ls: list, khz: int, tokens: int) -> str:
    """Markdown table per kernel role (tag), spans and gaps in microseconds."""
    us = 1e3 / khz  # microseconds per tick
    roles = {}
    order = []
    for i, l in enumerate(ls):
        gap = (l["t0"] - ls[i - 1]["t1"]) * us if i > 0 else 0.0
        r = roles.setdefault(l["tag"], {"n": 0, "span": 0.0, "gap": 0.0, "wgs": l["wgs"], "ramp": 0.0, "tail": 0.0})
        if l["tag"] not in order:
            order.append(l["tag"])
        r["n"] += 1
        r["span"] += (l["t1"] - l["t0"]) * us
        r["gap"] += gap
        r["ramp"] += (l["t0_med"] - l["t0"]) * us
        r["tail"] += (l["t1"] - l["t1_med"]) * us
    lines = ["| kernel | WGs | launches/token | span us | gap before us | median WG entry after first us | "
             "last exit after median us | per token us (span + gap) |",
             "|---|---:|---:|---:|---:|---:|---:|---:|"]
    total = 0.0
    for t in sorted(order, key=lambda t: -(roles[t]["span"] + roles[t]["gap"])):
        r = roles[t]
        n = r["n"]
        per_tok = (r["span"] + r["gap"]) / tokens
        total += per_tok
        lines.append(f"| {tag_name(t)} | {r['wgs']} | {n / tokens:.0f} | {r['span'] / n:.2f} | {r['gap'] / n:.2f} | "
                     f"{r['ramp'] / n:.2f} | {r['tail'] / n:.2f} | {per_tok:.1f} |")
    wall = (ls[-1]["t1"] - ls[0]["t0"]) * us / tokens if ls else 0.0
    lines.append(f"\nPer token: {total:.1f} us of spans and gaps; first entry to last exit {wall:.1f} us "
                 f"over {tokens} tokens ({len(ls)} launches).")
    return "\n".join(lines)


def cu_key(rec) -> tuple:
    """(XCD, shader engine, shader array, CU) of a record (HW_ID fields:
    CU_ID [11:8], SH_ID [12], SE_ID [15:13])."""
    hw = int(rec["hw_id"])
    return (int(rec["xcc"]) & 15, (hw >> 13) & 7, (hw >> 12) & 1, (hw >> 8) & 15)


def placement(recs: np.ndarray, ls: list, khz: int, top: int = 4) -> str:
    """For the `top` roles by time: how many workgroups each CU ran per
    launch, and the mean exit time (after the launch's first entry) of the
    workgroups on CUs that ran k of them; and the mean and latest exit per
    XCD.  Uneven placement shows as later exits on the CUs that ran more."""
    us = 1e3 / khz
    bounds = []
    i = 0
    for l in ls:
        bounds.append((i, i + l["wgs"]))
        i += l["wgs"]
    by_tag = {}
    for l, (a, b) in zip(ls, bounds):
        by_tag.setdefault(l["tag"], []).append((l, a, b))
    ranked = sorted(by_tag, key=lambda t: -sum(x[0]["t1"] - x[0]["t0"] for x in by_tag[t]))[:top]
    out = []
    for t in ranked:
        per_k = {}
        per_x = {}
        for l, a, b in by_tag[t]:
            seg = recs[a:b]
            keys = [cu_key(r) for r in seg]
            cnt = {}
            for k in keys:
                cnt[k] = cnt.get(k, 0) + 1
            for r, k in zip(seg, keys):
                e = (int(r["t1"]) - l["t0"]) * us
                per_k.setdefault(cnt[k], []).append(e)
                per_x.setdefault(k[0], []).append(e)
        ks = " ".join(f"{k} WGs/CU: {len(v)} WGs, exit {np.mean(v):.2f} us" for k, v in sorted(per_k.items()))
        xs = " ".join(f"x{x} {np.mean(v):.2f}/{np.max(v):.2f}" for x, v in sorted(per_x.items()))
        out.append(f"- {tag_name(t)}: {ks}; per XCD mean/max exit: {xs}")
    return "\n".join(out)


def phases(recs: np.ndarray, khz: int) -> str:
    """Per kernel role, the mean workgroup lifetime (entry to wave 0's exit)
    and the mean time after entry of each phase mark (csrc/trace.h)."""
    us = 1e3 / khz
    lines = ["| kernel | WG records | WG lifetime us | mark 0 | mark 1 | mark 2 | mark 3 |", "|---|---:|---:|---:|---:|---:|---:|"]
    tags = np.unique(recs["tag"])
    rows = []
    for t in tags:
        seg = recs[recs["tag"] == t]
        life = float(np.mean(seg["t1"].astype(np.float64) - seg["t0"])) * us
        ms = []
        for i in range(4):
            m = seg["mark"][:, i]
            m = m[m > 0]
            ms.append(f"{float(np.mean(m)) * us:.2f}" if m.size else "-")
        rows.append((life * seg.size, f"| {tag_name(int(t))} | {seg.size} | {life:.2f} | " + " | ".join(ms) + " |"))
    lines += [r for _, r in sorted(rows, key=lambda x: -x[0])]
    return "\n".join(lines)


def _engine(workload: str, steps: int):
    from . import formats
    from .engine import Engine
    from .model import E4BConfig, a4b_config, synth_tensors

    prompt_len = 512
    if workload == "a4b":
        cfg = a4b_config(max_seq=max(1024, prompt_len + steps + 64))
    else:
        cfg = E4BConfig(max_seq=max(1024, prompt_len + steps + 64))
    eng = Engine(cfg, synth_tensors(cfg, seed=0))
    prompt = formats.synth_uniform_u32(7, prompt_len, 0, cfg.vocab)
    eng.prefill(prompt)
    return eng, prompt_len


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="c4", choices=["c4", "a4b"])
    ap.add_argument("--steps", type=int, default=32)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--save", default=None, help="also write the raw workgroup records (numpy .npy) here")
    a = ap.parse_args(argv)
    eng, p0 = _engine(a.workload, a.warmup + a.steps)
    eng.time_decode(p0, a.warmup)
    ms = [0.0]

    def run():
        ms[0] = eng.time_decode(p0 + a.warmup, a.steps)

    recs = capture(run)
    if a.save:
        np.save(a.save, recs)
    khz = C.c_int(0)
    check(lib.e4b_trace_clock_khz(C.byref(khz)), "e4b_trace_clock_khz")
    ls = launches(recs)
    print(f"workload {a.workload}: {a.steps} graph-replayed tokens at positions {p0 + a.warmup}.."
          f"{p0 + a.warmup + a.steps - 1}, {ms[0] / a.steps * 1e3:.1f} us/token by HIP events "
          f"(trace build); {recs.size} workgroup records, clock {khz.value} kHz\n")
    print(summarize(ls, khz.value, a.steps))
    print("\nPhase marks (mean microseconds after the workgroup's entry; GEMV: 0 loads issued, 1 input vector "
          "ready, 2 dot products done, 3 rows reduced; attention: 0 loads issued, 1 head prep done, 2 scores "
          "done, 3 P.V merged; PLE: 0 loads issued, 1 prologue done, 2 gate done; MoE gate/up: 0 dense rows and "
          "inputs requested, 1 top-8 picks in LDS, 2 expert rows requested, 3 dot products done; MoE router: 0 "
          "loads issued, 1 residual rms formed, 2 router input staged, 3 score written; MoE down (expert "
          "blocks): 0 rows requested, 1 slot outputs staged, 2 dot products done):\n")
    print(phases(recs, khz.value))
    print("\nWorkgroup placement (microseconds after each launch's first entry):\n")
    print(placement(recs, ls, khz.value))
    eng.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
