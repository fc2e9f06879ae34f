"""Benchmark of the batch-1 decode path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c4|c3|c3p|c2|c1|c0|prefill|long|a4b] [--no-cpu]

Prints ONE JSON line (rank 0).  Workloads (the benchmark configs):
  c0  one q4_0 GEMV 16384x2048 (x f32), weights rotated over >512 MB so the
      256 MB MALL cannot serve them; a step = one GEMV.
  c1  Q6_K lm-head 262144x2048 + softcap + argmax; a step = one launch.
  c2  one layer's decode attention: global at 4096 positions, sliding
      (window 512, ring 1024) at positions 4095 and 300; a step = one layer.
  c3  A4B-style MoE half-layer (hidden 2816, 128 experts top-8); a step =
      one layer (4 launches), weights rotated over 3 copies.
  c4  the E4B-shaped decode loop; a step = one greedy decode token (the
      config also reports the batched prefill of the 512-token prompt).
  prefill  the 512-token c4 prompt through the batched prefill (MFMA
      GEMMs); a step = one whole prefill.
  c3p the c3 MoE half-layer over a 512-token chunk (expert-grouped
      GEMMs); a step = one layer.
  long  the c4 model at an 8192-token context: decode on the whole cache,
      then after compaction of the full layers to the 640-entry budget
      (generateLong's schedule); a step = one decode token after compaction.
  a4b the reference's live model shape (Gemma-4 26B-A4B MoE, 30 layers,
      hidden 2816, 128 experts top-8) through the A4B recipe; a step = one
      greedy decode token.
`roofline` is measured live with HIP events on the launch stream; the CPU
baseline times the oracle (the C restatement, OpenMP) on a bounded sample.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "e4b-webgpu_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
METRIC = "batch-1 decode tokens/s (E4B-shape q4_0) + achieved HBM GB/s % of peak"
MALL_BYTES = 256 << 20
# HBM bytes per launch of the dominant c4 kernel from two rocprofv3 counter
# runs (FETCH_SIZE, WRITE_SIZE per dispatch, each scaled by the same counter
# on a 256 MiB copy kernel: x2.000 and x1.000); commands and raw values in
# profiles/geglu_dominant_traffic.md.  Re-measure when the kernel changes.
GEGLU_TRAFFIC_BYTES = int(18609.6 * 1024 * 2.0 + 40.0 * 1024 * 1.0)
# The same two counter runs for the other configs' timed kernels (per launch
# or per layer; commands and raw values in profiles/gemv_c0.md,
# profiles/lmhead_c1.md, profiles/attn_c2.md and profiles/moe_c3.md).
C0_TRAFFIC_BYTES = int(9289.4 * 1024 * 2.0 + 64.0 * 1024)
C1_TRAFFIC_BYTES = int(215623.7 * 1024 * 2.0 + 1088.6 * 1024)
C2_GLOBAL_TRAFFIC_BYTES = int((4242.3 + 277.0) * 1024 * 2.0 + (530.0 + 4.0) * 1024)
C3_TRAFFIC_BYTES = int(19468.1 * 1024 * 2.0 + 75.2 * 1024)
# A4B whole decode step at positions 513-530 (profiles/decode_a4b_traffic.md):
# FETCH_SIZE 1,270,208.5 KiB x 2.0 + WRITE_SIZE 11,299.5 KiB per token
A4B_STEP_TRAFFIC_BYTES = int(1270208.5 * 1024 * 2.0 + 11299.5 * 1024)


def _cpu_cores() -> int:
    try:
        return int(os.environ.get("OMP_NUM_THREADS") or len(os.sched_getaffinity(0)))
    except Exception:
        return os.cpu_count() or 1


def bench_c0(steps: int, warmup: int, cpu: bool) -> dict:
    import ctypes as C

    from e4b import formats
    from e4b._lib import DT_F32_HL, check, lib
    from e4b.device import DeviceBuffer, Event
    from e4b.kernels import Q40Matrix

    rows, cols = 16384, 2048
    w = formats.synth_q40(0, rows, cols, 0.02)
    x = formats.synth_normal(1000, cols)
    wbytes = rows * (cols // 32) * 18
    algo = wbytes + cols * 4 + rows * 4
    ncopy = max(2, (2 * MALL_BYTES) // wbytes + 1)
    mats = [Q40Matrix(w, rows, cols) for _ in range(ncopy)]
    xd = DeviceBuffer.from_array(x)
    hl = DeviceBuffer(cols * 4)
    check(lib.e4b_split_f32(C.c_void_p(xd.ptr), cols, C.c_void_p(hl.ptr), None), "split")
    y = DeviceBuffer(rows * 4)
    for i in range(warmup):
        mats[i % ncopy].gemv_dev(hl, DT_F32_HL, y)
    e0, e1 = Event(), Event()
    e0.record()
    for i in range(steps):
        mats[i % ncopy].gemv_dev(hl, DT_F32_HL, y)
    e1.record()
    ms = e0.elapsed_ms(e1) / steps
    gbs = algo / (ms * 1e-3) / 1e9
    out = {
        "metric": "q4_0 GEMV GB/s (config c0)", "value": round(gbs, 2), "unit": "GB/s",
        "ms_per_step": ms, "dtype": "q4_0 x f32 (f32 accumulate)",
        "config": {"workload": "c0: q4_0 GEMV 16384x2048, x f32", "weight_copies_rotated": ncopy},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": C0_TRAFFIC_BYTES,
                     "kernel": "k_q40_gemv", "algorithmic_bytes_per_launch": algo},
    }
    if cpu:
        import oracle as orc
        t0 = time.perf_counter()
        n = 0
        while time.perf_counter() - t0 < 10.0:
            orc.q40_gemv(w, rows, cols, x)
            n += 1
        dt = (time.perf_counter() - t0) / n
        out["cpu_baseline"] = {"value": round(algo / dt / 1e9, 3), "unit": "GB/s", "cores": _cpu_cores(),
                               "kind": "port", "sample": f"{n} oracle GEMVs 16384x2048 (~10 s)"}
    return out


def bench_c1(steps: int, warmup: int, cpu: bool) -> dict:
    from e4b import formats
    from e4b.device import DeviceBuffer, Event
    from e4b.kernels import Q6KMatrix

    rows, cols = 262144, 2048
    w = formats.synth_q6k(0, rows, cols, 1e-3)
    x = formats.synth_normal(77, cols)
    M = Q6KMatrix(w, rows, cols)
    wbytes = rows * (cols // 256) * 210
    algo = wbytes + cols * 4 + rows * 4 + 8
    xd = DeviceBuffer.from_array(x)
    lg = DeviceBuffer(rows * 4)
    am = DeviceBuffer(8)
    for _ in range(warmup):
        M.gemv_argmax_dev(xd, 30.0, lg, am)
    e0, e1 = Event(), Event()
    e0.record()
    for _ in range(steps):
        M.gemv_argmax_dev(xd, 30.0, lg, am)
    e1.record()
    ms = e0.elapsed_ms(e1) / steps
    gbs = algo / (ms * 1e-3) / 1e9
    out = {
        "metric": "Q6_K lm-head+argmax GB/s (config c1)", "value": round(gbs, 2), "unit": "GB/s",
        "ms_per_step": ms, "dtype": "q6_K x f32 (f32 accumulate)",
        "config": {"workload": "c1: Q6_K lm-head 262144x2048 + softcap 30 + argmax"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": C1_TRAFFIC_BYTES,
                     "kernel": "k_q6k_gemv_argmax", "algorithmic_bytes_per_launch": algo},
    }
    if cpu:
        import oracle as orc
        t0 = time.perf_counter()
        n = 0
        while time.perf_counter() - t0 < 10.0:
            orc.q6k_gemv(w, rows, cols, x, 30.0)
            n += 1
        dt = (time.perf_counter() - t0) / n
        out["cpu_baseline"] = {"value": round(algo / dt / 1e9, 3), "unit": "GB/s", "cores": _cpu_cores(),
                               "kind": "port", "sample": f"{n} oracle lm-heads 262144x2048 (~10 s)"}
    return out


def bench_c2(steps: int, warmup: int, cpu: bool) -> dict:
    """One layer's decode attention (e4b_k_attn_decode: head prep + RoPE, K/V
    row write, split-K partials, then the log-sum-exp combine launch) at the
    three c2 points: a global layer at position 4095 over 4096 cached
    positions (theta 1e6), and a sliding layer (window 512, 1024-slot ring,
    theta 1e4) at position 4095 (wrapped ring) and 300.  Each case rotates
    over enough cache copies (>= 512 MB) that the 256 MB MALL cannot serve
    the next launch; a step = one layer's attention.  Algorithmic bytes per
    layer: the live K/V rows (2 KB a position) + the raw qkv f32 (12 KB) +
    the f16 output (4 KB) + the new K/V row (2 KB)."""
    from e4b.device import Event
    from e4b.kernels import AttnLayer

    QH, KVH, HD = 8, 2, 256
    rng = np.random.default_rng(0)
    qw = (1.0 + 0.1 * rng.standard_normal(HD)).astype(np.float32)
    kw = (0.25 * (1.0 + 0.1 * rng.standard_normal(HD))).astype(np.float32)
    qkv = rng.standard_normal((QH + 2 * KVH) * HD).astype(np.float32)
    cases = [("global", 4096, 0, 1e6, 4095), ("sliding", 1024, 512, 1e4, 4095), ("sliding", 1024, 512, 1e4, 300)]
    res = []
    for kind, slots, window, theta, pos in cases:
        cache_bytes = 2 * KVH * slots * HD * 2
        ncopy = max(2, (2 * MALL_BYTES) // cache_bytes + 1)
        k = (0.25 * rng.standard_normal((KVH, slots, HD))).astype(np.float16)
        v = rng.standard_normal((KVH, slots, HD)).astype(np.float16)
        layers = []
        for _ in range(ncopy):
            L = AttnLayer(QH, KVH, HD, slots, window, theta, 128, qw, kw)
            L.load_cache(k, v)
            L.qkv.upload(qkv)
            layers.append(L)
        live = min(pos + 1, window) if window else pos + 1
        algo = live * KVH * HD * 2 * 2 + qkv.size * 4 + QH * HD * 2 + KVH * HD * 2 * 2
        for i in range(warmup):
            layers[i % ncopy].step_dev(pos)
        e0, e1 = Event(), Event()
        e0.record()
        for i in range(steps):
            layers[i % ncopy].step_dev(pos)
        e1.record()
        ms = e0.elapsed_ms(e1) / steps
        res.append({"layer": kind, "pos": pos, "live_positions": live, "algorithmic_bytes": algo,
                    "us_per_layer": round(ms * 1e3, 3), "gbs": round(algo / (ms * 1e-3) / 1e9, 1),
                    "cache_copies_rotated": ncopy})
        del layers
    g = res[0]
    out = {
        "metric": "decode attention GB/s, global layer at 4096 positions (config c2)", "value": g["gbs"],
        "unit": "GB/s", "ms_per_step": g["us_per_layer"] / 1e3, "dtype": "f16 KV, f32 softmax and accumulate",
        "config": {"workload": "c2: GQA 8q/2kv x 256, split-K 64-position chunks + combine; global 4096 "
                               "positions (theta 1e6), sliding window 512 / ring 1024 (theta 1e4)",
                   "cases": res},
        "roofline": {"bound": "hbm", "achieved": g["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(g["gbs"] / HBM_PEAK_GBS, 4), "traffic": C2_GLOBAL_TRAFFIC_BYTES,
                     "kernel": "k_attn_split + k_attn_combine (global layer, pos 4095)",
                     "algorithmic_bytes_per_launch": g["algorithmic_bytes"]},
    }
    if cpu:
        import oracle as orc
        inv = orc.rope_inv_freq(1e6, HD, 128)
        kc = (0.25 * rng.standard_normal((4096, KVH, HD))).astype(np.float16).view(np.uint16)
        vc = rng.standard_normal((4096, KVH, HD)).astype(np.float16).view(np.uint16)
        t0 = time.perf_counter()
        n = 0
        while time.perf_counter() - t0 < 10.0:
            q, _, _ = orc.headprep(qkv, QH, KVH, HD, 128, inv, qw, kw, 1e-6, 4095)
            orc.attn_linear(q, kc, vc, QH, KVH, HD, 4096)
            n += 1
        dt = (time.perf_counter() - t0) / n
        out["cpu_baseline"] = {"value": round(g["algorithmic_bytes"] / dt / 1e9, 3), "unit": "GB/s",
                               "cores": _cpu_cores(), "kind": "port",
                               "sample": f"{n} oracle global-layer attentions at 4096 positions (~10 s)"}
    return out


def bench_c3(steps: int, warmup: int, cpu: bool) -> dict:
    """One A4B-style MoE FFN half-layer (router + top-8, dense and 8 expert
    GeGLU FFNs, slot-combined down, tail).  Three independent copies of the
    layer's weights (about 1 GB) are rotated so the 256 MB MALL cannot serve
    the next launch."""
    from e4b import formats
    from e4b.device import Event
    from e4b.kernels import MoeLayer

    H, E, FF, FF2 = 2816, 128, 704, 2112
    q = lambda rows, cols, s: formats.synth_q40(s, rows, cols, 0.02)  # noqa: E731
    ones = np.ones(H, np.float32)
    layers = []
    for c in range(3):
        t = {"ffn_norm": ones, "router_scale": ones, "pre_ffw2": ones, "post_ffw1": ones, "post_ffw2": ones,
             "post_ffw": ones, "router_w": formats.synth_normal(10 + c, E * H, 0.0, 0.02).reshape(E, H),
             "pes": np.ones(E, np.float32), "dense_gate": q(FF2, H, 100 * c + 1), "dense_up": q(FF2, H, 100 * c + 2),
             "dense_down": q(H, FF2, 100 * c + 3), "exp_gate_up": q(E * 2 * FF, H, 100 * c + 4),
             "exp_down": q(E * H, FF, 100 * c + 5)}
        L = MoeLayer(H, E, FF, FF2, t)
        L.h.upload(formats.synth_normal(500 + c, H))
        layers.append(L)
        if c == 0:
            t0 = t
    blk = lambda rows, cols: rows * cols // 32 * 18  # noqa: E731
    algo = (E * H * 4 + 8 * (blk(2 * FF, H) + blk(H, FF)) + blk(2 * FF2, H) + blk(H, FF2)
            + 9 * H * 4 + E * 4)
    for i in range(warmup):
        layers[i % 3].forward_dev()
    e0, e1 = Event(), Event()
    e0.record()
    for i in range(steps):
        layers[i % 3].forward_dev()
    e1.record()
    ms = e0.elapsed_ms(e1) / steps
    gbs = algo / (ms * 1e-3) / 1e9
    out = {
        "metric": "MoE decode layer GB/s (config c3)", "value": round(gbs, 2), "unit": "GB/s", "ms_per_step": ms,
        "dtype": "q4_0 x f16 (f32 accumulate), f32 router",
        "config": {"workload": "c3: A4B-style MoE half-layer, hidden 2816, 128 experts top-8, expert ffn 704, "
                               "dense ffn 2112", "algorithmic_bytes_per_layer": algo},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": C3_TRAFFIC_BYTES,
                     "kernel": "k_moe_router + k_moe_gu + k_moe_down + k_moe_tail (one layer)",
                     "algorithmic_bytes_per_launch": algo},
    }
    if cpu:
        import oracle as orc
        m = dict(t0, hidden=H, n_experts=E, top_k=8, expert_ffn=FF, dense_ffn=FF2)
        h = formats.synth_normal(500, H)
        t1 = time.perf_counter()
        n = 0
        while time.perf_counter() - t1 < 10.0:
            orc.moe_ffn(m, h)
            n += 1
        dt = (time.perf_counter() - t1) / n
        out["cpu_baseline"] = {"value": round(algo / dt / 1e9, 3), "unit": "GB/s", "cores": _cpu_cores(),
                               "kind": "port", "sample": f"{n} oracle MoE layers (~10 s)"}
    return out


def bench_c3p(steps: int, warmup: int, cpu: bool) -> dict:
    """The c3 MoE half-layer over a 512-token prompt chunk (the batched
    prefill: expert-grouped MFMA GEMMs); a step = one layer over 512 tokens."""
    from e4b import formats
    from e4b._lib import check, lib
    from e4b.device import DeviceBuffer, Event
    from e4b.kernels import MoeLayer, _vp

    H, E, FF, FF2, M = 2816, 128, 704, 2112, 512
    q = lambda rows, cols, s: formats.synth_q40(s, rows, cols, 0.02)  # noqa: E731
    ones = np.ones(H, np.float32)
    t = {"ffn_norm": ones, "router_scale": ones, "pre_ffw2": ones, "post_ffw1": ones, "post_ffw2": ones,
         "post_ffw": ones, "router_w": formats.synth_normal(10, E * H, 0.0, 0.02).reshape(E, H),
         "pes": np.ones(E, np.float32), "dense_gate": q(FF2, H, 1), "dense_up": q(FF2, H, 2),
         "dense_down": q(H, FF2, 3), "exp_gate_up": q(E * 2 * FF, H, 4), "exp_down": q(E * H, FF, 5)}
    L = MoeLayer(H, E, FF, FF2, t)
    hd = DeviceBuffer.from_array(formats.synth_normal(77, M * H))
    ho = DeviceBuffer(M * H * 4)

    def run():
        check(lib.e4b_k_moe_prefill(C.byref(L.w), _vp(hd), M, _vp(ho), None, None, None, None, None),
              "e4b_k_moe_prefill")

    for _ in range(warmup):
        run()
    e0, e1 = Event(), Event()
    e0.record()
    for _ in range(steps):
        run()
    e1.record()
    ms = e0.elapsed_ms(e1) / steps
    # algorithmic flops: router (f32) + dense GeGLU and down + 8 expert GeGLU
    # and down per token
    flops = 2 * M * (E * H + 2 * FF2 * H + H * FF2 + 8 * (2 * FF * H + H * FF))
    tf = flops / (ms * 1e-3) / 1e12
    return {
        "metric": "MoE prefill tokens/s per layer (config c3 shapes, 512-token chunk)",
        "value": round(M / (ms * 1e-3), 1), "unit": "tokens/s", "ms_per_step": ms,
        "dtype": "q4_0 x f16 on f16 MFMA (f32 accumulate), f32 router",
        "config": {"workload": "c3 MoE half-layer over 512 tokens: router, top-8, expert-grouped gate/up and down "
                               "GEMMs, dense branch GEMMs, combine, tail", "tokens": M, "flops": flops},
        "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(tf / 2500.0, 4), "traffic": None, "kernel": "whole MoE prefill layer"},
    }


def _time_geglu(cfg, steps: int) -> dict:
    """Dominant kernel of the c4 step: the FFN input GEMV exactly as the step
    launches it -- fused residual + RMSNorm prologue, gate/up q4_0 GEMV
    ([2*ffn][hidden]) and GeGLU epilogue to f16[ffn]
    (e4b_k_q40_geglu_prenorm).  Timed with HIP events on the launch stream
    over `steps` launches that rotate over one weight copy per layer (as in
    the step, so no launch is served from the 256 MB MALL)."""
    from e4b import formats
    from e4b.device import DeviceBuffer, Event
    from e4b.kernels import Q40Matrix

    rows, cols = 2 * cfg.ffn, cfg.hidden
    w = formats.synth_q40(123, rows, cols, 0.02)
    packed = formats.q40_pack(w, rows, cols)
    mats = []
    for _ in range(cfg.layers):
        m = Q40Matrix.__new__(Q40Matrix)
        m.rows, m.cols = rows, cols
        m.buf = DeviceBuffer.from_array(packed)
        mats.append(m)
    h_in = DeviceBuffer.from_array(formats.synth_normal(5, cols))
    resid = DeviceBuffer.from_array(formats.synth_normal(6, cols))
    w_res = DeviceBuffer.from_array(np.ones(cols, np.float32))
    w_in = DeviceBuffer.from_array(np.ones(cols, np.float32))
    h_out = DeviceBuffer(cols * 4)
    out = DeviceBuffer(cfg.ffn * 2)

    def launch(i):
        mats[i % len(mats)].geglu_prenorm_dev(h_in, resid, w_res, w_in, 1.0, cfg.eps, h_out, out)

    for i in range(2 * cfg.layers):
        launch(i)
    e0, e1 = Event(), Event()
    e0.record()
    for i in range(steps):
        launch(i)
    e1.record()
    us = e0.elapsed_ms(e1) * 1e3 / steps
    # weights + 4 f32 prologue vectors in + h out (f32) + f16 GeGLU out
    algo = rows * cols // 32 * 18 + 4 * cols * 4 + cols * 4 + cfg.ffn * 2
    return {"us": us, "algo": algo, "gbs": algo / (us * 1e-6) / 1e9}


def prefill_flops(cfg, n: int) -> dict:
    """Algorithmic flops of a batched prefill of n tokens from position 0:
    2 per weight element per token over every layer GEMM and the PLE model
    projection (counted once, though it runs as two f16 passes), and 4 x
    keys x head_dim per query head of causal attention (q.k and p.v)."""
    H, F, PD, L = cfg.hidden, cfg.ffn, cfg.ple_dim, cfg.layers
    qkv = (cfg.q_heads + 2 * cfg.kv_heads) * cfg.head_dim
    per_layer = qkv * H + H * cfg.q_heads * cfg.head_dim + 2 * F * H + H * F + (2 * PD * H if PD else 0)
    gemm = 2 * n * (L * per_layer + L * PD * H)
    attn = 0
    for g in cfg.layer_global:
        keys = sum(p + 1 if g else min(p + 1, cfg.window) for p in range(n))
        attn += 4 * cfg.q_heads * cfg.head_dim * keys
    return {"gemm": gemm, "attn": attn}


def time_prefill(eng, prompt, reps: int = 3) -> float:
    """Best wall time (s) of `reps` warm batched prefills (e4b_prefill is
    synchronous: it returns after the last token's argmax is read back)."""
    eng.prefill(prompt)
    best = float("inf")
    for _ in range(reps):
        t0 = time.perf_counter()
        eng.prefill(prompt)
        best = min(best, time.perf_counter() - t0)
    return best


def bench_prefill(steps: int, warmup: int, cpu: bool) -> dict:
    """The c4 prompt (512 uniform-random token ids) through the batched
    prefill, `steps` times after `warmup` (for profiling the prefill kernels)."""
    from e4b import formats
    from e4b.engine import Engine
    from e4b.model import E4BConfig, synth_tensors

    prompt_len = 512
    cfg = E4BConfig(max_seq=1024)
    eng = Engine(cfg, synth_tensors(cfg, seed=0))
    prompt = formats.synth_uniform_u32(7, prompt_len, 0, cfg.vocab)
    for _ in range(warmup):
        eng.prefill(prompt)
    t0 = time.perf_counter()
    for _ in range(steps):
        eng.prefill(prompt)
    dt = (time.perf_counter() - t0) / steps
    fl = prefill_flops(cfg, prompt_len)
    tf = (fl["gemm"] + fl["attn"]) / dt / 1e12
    eng.close()
    return {
        "metric": "batched prefill tokens/s (E4B-shape q4_0, 512-token prompt)", "value": round(prompt_len / dt, 1),
        "unit": "tokens/s", "ms_per_step": dt * 1e3,
        "dtype": "q4_0 weights x f16 activations on f16 MFMA, f32 accumulate",
        "config": {"workload": "prefill of the c4 prompt (512 tokens) on the E4B-shaped model",
                   "prompt_tokens": prompt_len, "flops": fl["gemm"] + fl["attn"]},
        "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(tf / 2500.0, 4), "traffic": None,
                     "kernel": "whole prefill (GEMMs + attention + per-token kernels)"},
    }


def _decode_bytes(cfg, sliding_live: int, global_live: int) -> int:
    """Algorithmic bytes of one decode step with the given live K/V rows per
    sliding and per full layer (cfg.bytes_per_token with the KV term replaced)."""
    kv_row = 2 * cfg.kv_heads * cfg.head_dim * 2
    base = cfg.bytes_per_token(0) - len(cfg.layer_global) * kv_row  # position 0: one live row per layer
    return base + sum((global_live if g else sliding_live) * kv_row for g in cfg.layer_global)


def bench_long(steps: int, warmup: int, cpu: bool) -> dict:
    """Long-context decode (src/engine-a4b.js:587-657): an 8192-token prompt
    on the E4B-shaped model with 8320 full-layer slots (KV_PRECAP), decode on
    the whole cache, then after compaction to the 640-entry budget (protect
    64); the full-cache decode is also timed on an engine without scoring."""
    from e4b import formats
    from e4b._lib import FLAG_KV_SCORE
    from e4b.engine import KV_BUDGET, KV_PROTECT, Engine
    from e4b.model import E4BConfig, synth_tensors

    n = 8192
    cfg = E4BConfig(max_seq=8320, max_prompt=n, flags=FLAG_KV_SCORE)
    tensors = synth_tensors(cfg, seed=0)
    prompt = formats.synth_uniform_u32(7, n, 0, cfg.vocab)
    eng = Engine(cfg, tensors)
    t_prefill = time_prefill(eng, prompt, reps=1)
    eng.time_decode(n, warmup)
    ms_full = eng.time_decode(n + warmup, steps) / steps
    pos = n + warmup + steps
    kept = eng.compact(KV_BUDGET, KV_PROTECT)
    eng.time_decode(pos, warmup)
    ms_budget = eng.time_decode(pos + warmup, steps) / steps
    kv_mid = kept + warmup + steps // 2
    eng.close()
    plain = Engine(E4BConfig(max_seq=8320, max_prompt=n), tensors)
    plain.prefill(prompt)
    plain.time_decode(n, warmup)
    ms_plain = plain.time_decode(n + warmup, steps) / steps
    plain.close()
    b_budget = _decode_bytes(cfg, cfg.window, kv_mid)
    b_full = _decode_bytes(cfg, cfg.window, n + warmup + steps // 2)
    gbs = b_budget / (ms_budget * 1e-3) / 1e9
    return {
        "metric": "batch-1 decode tokens/s at 8192-token context, 640-entry full-layer KV budget (E4B-shape q4_0)",
        "value": round(1e3 / ms_budget, 2), "unit": "tokens/s", "ms_per_step": ms_budget,
        "dtype": "q4_0/q6_K weights, f16 activations and KV, f32 accumulate",
        "config": {"workload": "generateLong schedule on the c4 model: 8192-token prompt, full-layer slots 8320, "
                               "compaction to 640 (protect 64); scored decode",
                   "prompt_tokens": n, "prefill_ms": round(t_prefill * 1e3, 1),
                   "decode_ms_full_cache_scored": round(ms_full, 4),
                   "decode_ms_full_cache_unscored": round(ms_plain, 4),
                   "decode_ms_budget_scored": round(ms_budget, 4),
                   "speedup_budget_vs_full_unscored": round(ms_plain / ms_budget, 3),
                   "bytes_per_token_full": b_full, "bytes_per_token_budget": b_budget},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "whole decode step (graph replay) after compaction"},
    }


def bench_a4b(steps: int, warmup: int, cpu: bool, no_graph: bool = False) -> dict:
    """Decode of the reference's live model shape (src/engine-a4b.js:100-116,
    the Gemma-4 26B-A4B MoE its published 95.0 tok/s on an M4 Max is quoted
    on): the A4B recipe at 30 layers, hidden 2816, 16 q heads, sliding layers
    8 KV heads x 256 (window 1024, ring 1536), every sixth layer full with 2
    KV heads x 512 and V = K, dense GeGLU 2112 beside 128 experts of 704
    (top 8), vocab 262144, random-init q4_0 + Q6_K.  The 512-token prompt
    runs through the batched prefill (GEMMs, per-token causal attention, the
    expert-grouped MoE prefill); decode is GPU-fed graph replay.  The roofline is the whole step: algorithmic bytes per token
    (every dense weight, the router, the 8 active experts' blocks, the live
    K/V rows, the lm-head) over the step time."""
    from e4b import formats
    from e4b._lib import FLAG_NO_GRAPH
    from e4b.engine import Engine
    from e4b.model import a4b_config, synth_tensors

    prompt_len = 512
    cfg = a4b_config(max_seq=max(1024, prompt_len + warmup + steps + 8), flags=FLAG_NO_GRAPH if no_graph else 0)
    t0 = time.perf_counter()
    tensors = synth_tensors(cfg, seed=0)
    t_synth = time.perf_counter() - t0
    t0 = time.perf_counter()
    eng = Engine(cfg, tensors)
    t_load = time.perf_counter() - t0
    prompt = formats.synth_uniform_u32(7, prompt_len, 0, cfg.vocab)
    t_prefill = time_prefill(eng, prompt, reps=3)
    eng.time_decode(prompt_len, warmup)
    ms = eng.time_decode(prompt_len + warmup, steps)
    ms_tok = ms / steps
    positions = range(prompt_len + warmup, prompt_len + warmup + steps)
    bytes_tok = sum(cfg.bytes_per_token(p) for p in positions) / steps
    gbs = bytes_tok / (ms_tok * 1e-3) / 1e9
    out = {
        "metric": "batch-1 decode tokens/s (A4B-shape MoE q4_0) + achieved HBM GB/s % of peak",
        "value": round(1e3 / ms_tok, 2), "unit": "tokens/s", "ms_per_step": ms_tok,
        "dtype": "q4_0/q6_K weights, f16 activations and KV, f32 accumulate",
        "config": {"workload": "a4b: Gemma-4-26B-A4B-shaped random-init MoE decoder, 30 layers, hidden 2816, 16q, "
                               "sliding 8kv x 256 (window 1024, ring 1536) : full 2kv x 512 (V = K) 5:1, dense ffn "
                               "2112 + 128 experts x 704 top-8, vocab 262144, q4_0 + Q6_K",
                   "prompt_tokens": prompt_len, "decode_tokens_timed": steps,
                   "decode_positions": [prompt_len + warmup, prompt_len + warmup + steps],
                   "bytes_per_token": int(bytes_tok), "prefill_ms": round(t_prefill * 1e3, 2),
                   "prefill_tokens_per_s": round(prompt_len / t_prefill, 1),
                   "reference_published": "95.0 tok/s, 10.52 ms/token on an M4 Max (546 GB/s) over the real "
                                          "26B-A4B q4_0 GGUF, 2.38 GB/token",
                   "setup_s": {"synth": round(t_synth, 1), "load": round(t_load, 1)}},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": A4B_STEP_TRAFFIC_BYTES,
                     "kernel": "whole decode step (graph replay)"},
    }
    if cpu:
        out["cpu_baseline"] = _cpu_decode_at(eng, cfg, tensors, prompt, prompt_len + warmup, steps)
    eng.close()
    return out


def _cpu_decode_at(eng, cfg, tensors, tokens, p0: int, steps: int, budget_s: float = 15.0) -> dict:
    """The oracle's decode step timed at the GPU's own timed positions: it is
    handed the engine's KV caches (every layer, and the full layers' entry
    count) as they stand at p0, then steps p0, p0 + 1, ... for about
    budget_s seconds (at most `steps` positions), so each oracle step attends
    over as many keys as the GPU step at that position did."""
    import oracle as orc
    om = orc.OracleModel(cfg.as_dict(), {n: t.data for n, t in tensors.items()})
    for layer in range(cfg.layers):
        k, v = eng.read_kv(layer)
        om.set_kv(layer, k.transpose(1, 0, 2), v.transpose(1, 0, 2))
    om.set_kv_count(p0)
    t0 = time.perf_counter()
    n = 0
    while n < steps and (n == 0 or time.perf_counter() - t0 < budget_s):
        om.step(int(tokens[n % len(tokens)]), p0 + n)
        n += 1
    dt = (time.perf_counter() - t0) / n
    return {"value": round(1.0 / dt, 3), "unit": "tokens/s", "cores": _cpu_cores(), "kind": "port",
            "sample": f"{n} oracle decode steps of the same model at positions {p0}..{p0 + n - 1} (the GPU's "
                      f"timed positions), from the GPU's KV caches (~{budget_s:.0f} s)"}


def bench_c4(steps: int, warmup: int, cpu: bool, no_graph: bool = False) -> dict:
    from e4b import formats
    from e4b._lib import FLAG_NO_GRAPH
    from e4b.engine import Engine
    from e4b.model import E4BConfig, synth_tensors

    prompt_len = 512
    flags = FLAG_NO_GRAPH if no_graph else 0
    cfg = E4BConfig(max_seq=max(1024, prompt_len + warmup + steps + 8), flags=flags)
    t0 = time.perf_counter()
    tensors = synth_tensors(cfg, seed=0)
    t_synth = time.perf_counter() - t0
    t0 = time.perf_counter()
    eng = Engine(cfg, tensors)
    t_load = time.perf_counter() - t0
    prompt = formats.synth_uniform_u32(7, prompt_len, 0, cfg.vocab)
    t_prefill = time_prefill(eng, prompt)
    fl = prefill_flops(cfg, prompt_len)
    eng.time_decode(prompt_len, warmup)
    ms = eng.time_decode(prompt_len + warmup, steps)
    ms_tok = ms / steps
    positions = range(prompt_len + warmup, prompt_len + warmup + steps)
    bytes_tok = sum(cfg.bytes_per_token(p) for p in positions) / steps
    step_gbs = bytes_tok / (ms_tok * 1e-3) / 1e9
    dom = _time_geglu(cfg, max(steps, 4 * cfg.layers))
    out = {
        "metric": METRIC, "value": round(1e3 / ms_tok, 2), "unit": "tokens/s", "ms_per_step": ms_tok,
        "dtype": "q4_0/q6_K weights, f16 activations and KV, f32 accumulate",
        "config": {"workload": "c4: E4B-shaped random-init decoder, 35 layers, hidden 2048, ffn 16384, "
                               "8q/2kv x 256, 4 sliding(512):1 global, PLE 256, vocab 262144, q4_0 + Q6_K",
                   "prompt_tokens": prompt_len, "decode_tokens_timed": steps, "decode_positions":
                   [prompt_len + warmup, prompt_len + warmup + steps],
                   "bytes_per_token": int(bytes_tok), "step_hbm_gbs": round(step_gbs, 1),
                   "step_hbm_frac": round(step_gbs / HBM_PEAK_GBS, 4),
                   "prefill_tokens_per_s": round(prompt_len / t_prefill, 1),
                   "prefill_ms": round(t_prefill * 1e3, 3),
                   "layer_loop": "six kernels a layer",
                   "prefill_tflops": round((fl["gemm"] + fl["attn"]) / t_prefill / 1e12, 2),
                   "setup_s": {"synth": round(t_synth, 1), "load": round(t_load, 1)}},
        "roofline": {"bound": "hbm", "achieved": round(dom["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom["gbs"] / HBM_PEAK_GBS, 4), "traffic": GEGLU_TRAFFIC_BYTES,
                     "kernel": "k_q40 gate/up 32768x2048, residual+norm prologue, GeGLU epilogue",
                     "algorithmic_bytes_per_launch": dom["algo"], "avg_launch_us": round(dom["us"], 3)},
    }
    if cpu:
        out["cpu_baseline"] = _cpu_decode_at(eng, cfg, tensors, prompt, prompt_len + warmup, steps)
    eng.close()
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="c4", choices=["c0", "c1", "c2", "c3", "c3p", "c4", "prefill", "long", "a4b"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--kernel-only", action="store_true",
                    help="c4: time only the dominant kernel (for counter runs; prints its own line, not the bench line)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run one 256 MiB device-to-device copy (the byte scale for rocprof FETCH/WRITE_SIZE)")
    ap.add_argument("--no-graph", action="store_true",
                    help="c4, a4b: launch the step kernels directly instead of replaying the hipGraph (for profilers)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for {a.gpus}); "
              "the multi-GPU sharding is a design note, not a measured path.", file=sys.stderr)
        return 2
    fn = {"c0": bench_c0, "c1": bench_c1, "c2": bench_c2, "c3": bench_c3, "c3p": bench_c3p, "c4": bench_c4,
          "prefill": bench_prefill, "long": bench_long, "a4b": bench_a4b}[a.workload]
    steps = a.steps if a.steps is not None else {"c4": 240, "prefill": 10, "long": 64, "a4b": 240}.get(a.workload, 200)
    warmup = a.warmup if a.warmup is not None else {"c4": 16, "prefill": 2, "long": 8, "a4b": 16}.get(a.workload, 20)
    if a.workload == "c4" and a.kernel_only:
        from e4b.model import E4BConfig
        dom = _time_geglu(E4BConfig(), steps)
        print(json.dumps({"kernel": "k_q40 gate/up 32768x2048, residual+norm prologue, GeGLU epilogue",
                          "launches": steps, "avg_launch_us": round(dom["us"], 3),
                          "algorithmic_bytes_per_launch": dom["algo"], "gbs": round(dom["gbs"], 1)}))
        res = None
    elif a.workload == "c4":
        res = bench_c4(steps, warmup, not a.no_cpu, a.no_graph)
    elif a.workload == "a4b":
        res = bench_a4b(steps, warmup, not a.no_cpu, a.no_graph)
    else:
        res = fn(steps, warmup, not a.no_cpu)
    if a.copy_probe:
        from e4b._lib import check, lib
        from e4b.device import DeviceBuffer, sync
        n = 256 << 20
        src, dst = DeviceBuffer(n), DeviceBuffer(n)
        check(lib.e4b_memcpy_d2d(dst.ptr, src.ptr, n, None), "copy probe")
        sync()
    if res is None:
        return 0
    line = {
        "metric": res["metric"], "value": res["value"], "unit": res["unit"], "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(res["ms_per_step"], 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": res["dtype"], "data": "synthetic (seeded)",
        "config": res["config"], "roofline": res["roofline"], "cpu_baseline": res.get("cpu_baseline"),
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
