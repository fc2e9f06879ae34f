"""End-to-end parity of the decode engine (libe4b, HIP) with the CPU oracle.

Tolerances (stated, as the north star asks):
  * greedy tokens: bit-exact, except at a near-tie where the oracle's top-2
    logit margin is below 2e-3 of its logit range (reported, then the oracle's
    choice is fed to both sides so the comparison continues in lock-step);
  * logits: max |gpu - oracle| <= 1e-3 * max |oracle|;
  * hidden state: max |gpu - oracle| <= 1e-3 * max |oracle|;
  * KV caches: the set of written ring slots is identical (bit-exact slot
    indices); values: max error <= 1e-2 * max |value| and mean error <=
    1e-3 * mean |value|.  Later layers' K/V inherit the upstream hidden-state
    differences (f16 rounding points of f32 results that differ in the last
    bits, amplified by scale-1.0 attention), so single entries drift more
    than the hidden state itself.
"""
import numpy as np
import pytest

import oracle as orc
from e4b.engine import Engine
from e4b.model import E4BConfig, norm_weights_random, synth_tensors, tiny_config
from tests.util import top2_margin

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3
TIE_TOL = 2e-3
KV_MAX_TOL = 1e-2
KV_MEAN_TOL = 1e-3


def build(cfg: E4BConfig, seed: int, **synth_kw):
    tensors = norm_weights_random(synth_tensors(cfg, seed, **synth_kw), seed + 1)
    eng = Engine(cfg, tensors)
    om = orc.OracleModel(cfg.as_dict(), {n: t.data for n, t in tensors.items()})
    return eng, om


def lockstep(eng, om, prompt, n_decode, check_logits_every=0):
    """Prefill + GPU-fed decode on the engine; the oracle replays the GPU's
    token stream (each oracle step takes the GPU's previous token), so a
    near-tie that the two sides break differently does not end the
    comparison: every one of the n_decode steps is compared.  Returns
    (tokens, near-tie positions, the oracle's last logits)."""
    g0 = eng.prefill(prompt)
    for i, t in enumerate(prompt):
        o_tok, o_lg, _ = om.step(int(t), i, want_logits=(i == len(prompt) - 1))
    ties = []
    tok = g0
    if tok != o_tok:
        assert top2_margin(o_lg) < TIE_TOL * np.abs(o_lg).max(), f"prefill argmax {tok} vs oracle {o_tok}"
        ties.append(len(prompt) - 1)
    gpu_tokens = eng.decode_chunk(len(prompt), n_decode)
    fed = [tok] + gpu_tokens.tolist()
    compared = 0
    for i in range(n_decode):
        pos = len(prompt) + i
        o_tok, o_lg, _ = om.step(int(fed[i]), pos, want_logits=True)
        compared += 1
        if o_tok != fed[i + 1]:
            margin = top2_margin(o_lg)
            assert margin < TIE_TOL * np.abs(o_lg).max(), (
                f"decode step {i} (pos {pos}): gpu {fed[i + 1]} vs oracle {o_tok}, margin {margin:.3e}")
            ties.append(pos)
    assert compared == n_decode
    return fed, ties, o_lg


def test_tiny_engine_tokens_logits_kv():
    cfg = tiny_config()
    eng, om = build(cfg, 11)
    prompt = np.random.default_rng(0).integers(0, cfg.vocab, 12)
    toks, ties, _ = lockstep(eng, om, prompt, 40)
    print(f"tiny: {len(toks)} tokens, near-ties at {ties}")
    assert len(ties) == 0
    pos = 12 + 40  # next position
    # one more host-fed step with logits and hidden
    lg_tok, lg = eng.step(toks[-1], pos, want_logits=True)
    o_tok, o_lg, o_h = om.step(int(toks[-1]), pos, want_logits=True, want_hidden=True)
    err = float(np.max(np.abs(lg - o_lg)) / np.max(np.abs(o_lg)))
    herr = float(np.max(np.abs(eng.read_hidden() - o_h)) / np.max(np.abs(o_h)))
    print(f"tiny logits err {err:.2e} hidden err {herr:.2e}")
    assert err < LOGIT_TOL and herr < LOGIT_TOL
    assert lg_tok == o_tok or top2_margin(o_lg) < TIE_TOL * np.abs(o_lg).max()
    # KV caches: same written slots, values within tolerance
    for layer in range(cfg.layers):
        k, v = eng.read_kv(layer)  # [kvh][slots][hd]
        slots = k.shape[1]
        ok = om.kcache(layer, slots * cfg.kv_heads * cfg.head_dim).reshape(slots, cfg.kv_heads, cfg.head_dim)
        ov = om.vcache(layer, slots * cfg.kv_heads * cfg.head_dim).reshape(slots, cfg.kv_heads, cfg.head_dim)
        ok, ov = ok.transpose(1, 0, 2), ov.transpose(1, 0, 2)
        written_g = np.any(k != 0, axis=(0, 2))
        written_o = np.any(ok != 0, axis=(0, 2))
        assert np.array_equal(written_g, written_o), f"layer {layer}: written slots differ"
        for a, b in ((k, ok), (v, ov)):
            fa = a.view(np.float16).astype(np.float64)
            fb = b.view(np.float16).astype(np.float64)
            d = np.abs(fa - fb)
            print(f"layer {layer} cache max err {d.max() / np.abs(fb).max():.2e} mean err "
                  f"{d.mean() / max(np.abs(fb).mean(), 1e-30):.2e}")
            assert d.max() <= KV_MAX_TOL * np.abs(fb).max(), f"layer {layer} cache values (max)"
            assert d.mean() <= KV_MEAN_TOL * np.abs(fb).mean(), f"layer {layer} cache values (mean)"
        expect_written = (pos + 1) if cfg.layer_global[layer] else min(pos + 1, slots)
        assert int(written_g.sum()) == expect_written


def test_tiny_engine_step_api_and_reset():
    cfg = tiny_config(layers=5)
    eng, om = build(cfg, 5)
    ids = [3, 17, 999, 0, 42]
    a = [eng.step(t, i) for i, t in enumerate(ids)]
    b = [om.step(t, i)[0] for i, t in enumerate(ids)]
    assert a == b
    eng.reset()
    assert eng.prefill(ids) == b[-1]
    assert eng.argmax_fast() == b[-1]
    with pytest.raises(Exception):
        eng.step(cfg.vocab, 0)  # token out of range
    # the full layers hold max_seq entries: fill them, then one more step
    eng.decode_chunk(len(ids), cfg.max_seq - len(ids))
    with pytest.raises(Exception):
        eng.step(1, cfg.max_seq)


def test_generate_fast_matches_step_loop():
    cfg = tiny_config()
    eng, _ = build(cfg, 21)
    prompt = [5, 6, 7, 8]
    gen = eng.generate_fast(prompt, 20, eos=())
    eng.reset()
    toks = [eng.step(t, i) for i, t in enumerate(prompt)]
    cur = toks[-1]
    ref = [cur]
    for i in range(19):
        cur = eng.step(cur, len(prompt) + i)
        ref.append(cur)
    assert gen == ref


def test_generate_prefill_and_profiles():
    # generatePrefill (batched prefill + GPU-fed decode) and generateFast
    # (prompt through the step) against the oracle's chain fed with the GPU's
    # tokens; profileStep / profilePrefill time every kernel role
    cfg = tiny_config(layers=3, layer_global=[0, 0, 1])
    eng, om = build(cfg, 21)
    prompt = [int(x) for x in np.random.default_rng(21).integers(0, cfg.vocab, 12)]
    gp = eng.generate_prefill(prompt, 12, eos=())
    lg_p = eng.read_logits()
    eng.reset()
    gf = eng.generate_fast(prompt, 12, eos=())
    for i, t in enumerate(prompt):
        o_tok, o_lg, _ = om.step(t, i, want_logits=True)
    ties = []
    for k in range(len(gp)):
        if gp[k] != o_tok:
            assert top2_margin(o_lg) < TIE_TOL * np.abs(o_lg).max(), (k, gp[k], o_tok)
            ties.append(k)
        if k + 1 < len(gp):
            o_tok, o_lg, _ = om.step(gp[k], len(prompt) + k, want_logits=True)
    err = float(np.abs(lg_p - o_lg).max() / np.abs(o_lg).max())
    print(f"generate_prefill {gp}, generate_fast {gf}, near-ties {ties}, logits err {err:.2e}")
    assert err < LOGIT_TOL
    assert gf == gp or ties
    eng.reset()
    ps = eng.profile_step(prompt[0], 0)
    for role, n in (("embed", 1), ("ple_model_proj", 1), ("ple_prep", 1), ("qkv", 3), ("attn_sliding", 2),
                    ("attn_global", 1), ("o_proj", 3), ("gate_up_geglu", 3), ("down", 3), ("ple", 3),
                    ("final_norm", 1), ("lm_head", 1), ("argmax_feedback", 1)):
        assert ps[role]["n"] == n and ps[role]["us"] > 0, (role, ps.get(role))
    # the profiled step is a real step: its argmax is the oracle's at position 0
    om.reset()
    o0, o_lg0, _ = om.step(prompt[0], 0, want_logits=True)
    assert eng.argmax_fast() == o0 or top2_margin(o_lg0) < TIE_TOL * np.abs(o_lg0).max()
    pp = eng.profile_prefill(prompt)
    for role in ("embed_rows", "gemm_ple_model_proj", "ple_prep_rows", "gemm_qkv", "headprep_rows", "attn_prefill",
                 "gemm_o", "gemm_gate_up_geglu", "gemm_down", "gemm_ple_gate", "gelu_mul_rows", "gemm_ple_proj",
                 "resnorm_rows"):
        assert pp[role]["us"] > 0, role
    assert pp["gemm_qkv"]["n"] == 3 and pp["resnorm_rows"]["n"] == 1 + 3 * 3
    print("profile_step:", {k: round(v["us"], 1) for k, v in ps.items()})


def test_c4_width_five_layers():
    cfg = E4BConfig(layers=5, max_seq=256, layer_global=[0, 0, 0, 0, 1])
    eng, om = build(cfg, 3)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab, 6)
    toks, ties, o_lg = lockstep(eng, om, prompt, 6)
    print(f"c4-width 5 layers: near-ties {ties}")
    assert len(ties) == 0
    err = float(np.max(np.abs(eng.read_logits() - o_lg)) / np.max(np.abs(o_lg)))
    print(f"c4-width logits err {err:.2e}")
    assert err < LOGIT_TOL


@pytest.mark.slow
def test_c4_full_model_lockstep():
    cfg = E4BConfig(max_seq=1024)  # benchmark config c4 shapes (35 layers)
    eng, om = build(cfg, 0)
    prompt = np.random.default_rng(2).integers(0, cfg.vocab, 8)
    toks, ties, o_lg = lockstep(eng, om, prompt, 16)
    print(f"c4 full: tokens {toks[:8]}..., near-ties {ties}")
    assert len(ties) == 0
    err = float(np.max(np.abs(eng.read_logits() - o_lg)) / np.max(np.abs(o_lg)))
    print(f"c4 full logits err {err:.2e}")
    assert err < LOGIT_TOL


@pytest.mark.slow
def test_c4_greedy_256_steps():
    # the GPU-fed greedy sequence at the E4B shape equals
    # the oracle's over 256 decode steps (near-ties reported, none expected)
    cfg = E4BConfig(max_seq=1024)
    eng, om = build(cfg, 3)
    prompt = np.random.default_rng(4).integers(0, cfg.vocab, 16)
    toks, ties, o_lg = lockstep(eng, om, prompt, 256)
    print(f"c4 256 steps: {len(toks) - 1} decoded and compared, distinct tokens {len(set(toks))}, near-ties {ties}")
    err = float(np.max(np.abs(eng.read_logits() - o_lg)) / np.max(np.abs(o_lg)))
    print(f"c4 256 steps: final logits err {err:.2e}")
    assert err < LOGIT_TOL


@pytest.mark.slow
@pytest.mark.timeout(900)
def test_c4_stated_workload_teacher_forced(capsys):
    # benchmark config c4 at its stated workload: the 35-layer E4B shape, a
    # 512-token prompt through the batched prefill (e4b_prefill), then 256
    # decode steps fed with seeded random tokens (teacher forcing), so every
    # step's argmax is a decision on a different input and positions 512-767
    # keep the 512-position sliding window full and wrapping its 1024-slot
    # ring.  Two oracles follow the GPU, and every step is compared (no
    # early exit):
    #   * `om` runs free from the prompt on: its caches are its own.  After
    #     the prefill the logits are within 1e-3 of max |logit|; at every
    #     decode step the logits stay within DRIFT_TOL of the oracle's logit
    #     range, and the argmax equals the GPU's unless the oracle's top-2
    #     margin is within twice that step's logit difference.  Over hundreds of positions the two sides'
    #     f16-rounded K/V rows differ by an ulp in 20-40 % of entries (f32 on
    #     the GPU, double in the oracle, straddling a rounding point), and
    #     this random model's scale-1.0 attention (score std ~16) turns an
    #     ulp at a near-tie of two keys into a visible change of that head's
    #     output; the drift is reported, with the end-of-run KV statistics.
    #   * `osync` is handed the GPU's KV caches after each GPU decode step,
    #     the rows the step wrote for its token included (keep_rows: the
    #     oracle attends to the handed-over row of the current token and
    #     keeps its own rows apart), so its step starts from the GPU's
    #     state -- the step's kernels at the full workload shape.  The argmax
    #     must be equal unless a near-tie; the logits within SYNC_TOL = 2e-3
    #     of the oracle's logit range at every step, with the median within
    #     3e-4.  The stated tolerance is not 1e-3: the recipe's f16 rounding
    #     points make the step piecewise constant, and a one-ulp f32 nudge of
    #     a single norm vector already moves the oracle's own logits by
    #     jumps of up to ~7e-4 of max |logit| (~3.5e-4 of range) at some
    #     positions (tests/test_oracle_recipe.py); f32 against double
    #     arithmetic throughout sums several such jumps (worst step measured
    #     1.0e-3 of the range over these 256 positions, median 1.8e-4).  The
    #     GPU's new rows are checked against the oracle's own: layer 0's
    #     within 2^-9 of the row's max |value| (two f16 ulps at its top
    #     binade: nothing upstream of it amplifies), the other layers' within
    #     the KV tolerance of the other engine tests, 1e-2 of max |value| (a
    #     row inherits the step's jumps upstream of its layer); the share of
    #     bit-identical entries is reported.
    #   * KV written-slot sets bit-exact; mean |err| <= 1e-3 of mean |value|.
    import time
    DRIFT_TOL = 1e-2
    SYNC_TOL = 2e-3
    from e4b._lib import FLAG_LAYER_HIDDEN
    cfg = E4BConfig(max_seq=1024, flags=FLAG_LAYER_HIDDEN)
    tensors = norm_weights_random(synth_tensors(cfg, 5), 6)
    eng = Engine(cfg, tensors)
    tens = {n: t.data for n, t in tensors.items()}
    om = orc.OracleModel(cfg.as_dict(), tens)
    osync = orc.OracleModel(cfg.as_dict(), tens)
    rng = np.random.default_rng(12)
    prompt = rng.integers(0, cfg.vocab, 512)
    forced = rng.integers(0, cfg.vocab, 256)
    S = cfg.kv_heads * cfg.head_dim

    def say(msg):
        with capsys.disabled():
            print(msg, flush=True)

    def lerr(a, b):
        d = float(np.max(np.abs(a.astype(np.float64) - b)))
        return d / float(np.max(np.abs(b))), d / float(np.max(b) - np.min(b))

    t0 = time.time()
    g0 = eng.prefill(prompt)
    g_lg = eng.read_logits()
    for i, t in enumerate(prompt):
        o_tok, o_lg, _ = om.step(int(t), i, want_logits=(i == len(prompt) - 1))
        if i % 128 == 127:
            say(f"c4 stated: oracle prompt {i + 1}/512 ({time.time() - t0:.0f} s)")
    err_m, err_r = lerr(g_lg, o_lg)
    print(f"after the batched prefill: logits err {err_m:.2e} of max, {err_r:.2e} of range")
    assert g0 == o_tok or top2_margin(o_lg) < TIE_TOL * np.abs(o_lg).max(), f"prefill argmax {g0} vs {o_tok}"
    assert err_m < LOGIT_TOL
    free, sync, ties, row_same, layer_err, flips = [], [], [], [], [], []
    argmaxes = []
    osync.set_keep_rows(True)
    for k, t in enumerate(forced):
        pos = len(prompt) + k
        g, lg = eng.step(int(t), pos, want_logits=True)
        o_tok, o_lg, _ = om.step(int(t), pos, want_logits=True)
        # the synced oracle starts this step from the GPU's caches, the rows
        # the GPU wrote for this token included
        gpu_rows = []
        for layer in range(cfg.layers):
            kg, vg = eng.read_kv(layer)
            osync.set_kv(layer, kg.transpose(1, 0, 2), vg.transpose(1, 0, 2))
            slot = pos if cfg.layer_global[layer] else pos % kg.shape[1]
            gpu_rows.append((kg[:, slot, :], vg[:, slot, :]))
        osync.set_kv_count(pos)
        s_tok, s_lg, _ = osync.step(int(t), pos, want_logits=True)
        ulp1 = np.zeros(cfg.layers, np.int64)  # new K/V entries one f16 code apart (a rounding point straddled)
        ulpn = np.zeros(cfg.layers, np.int64)  # ... more than one code apart
        for layer, (kg, vg) in enumerate(gpu_rows):
            for a, b in zip((kg, vg), osync.rows(layer)):
                fa, fb = a.view(np.float16).astype(np.float64), b.view(np.float16).astype(np.float64)
                d = np.abs(fa - fb).max() / np.abs(fb).max()
                assert d <= (2.0 ** -9 if layer == 0 else KV_MAX_TOL), f"pos {pos} layer {layer}: new row {d:.2e}"
                row_same.append(float(np.mean(a == b)))
                du = np.abs(a.view(np.int16).astype(np.int32) - b.view(np.int16).astype(np.int32))
                ulp1[layer] += int(np.sum(du == 1))
                ulpn[layer] += int(np.sum(du > 1))
        flips.append((ulp1, ulpn))
        argmaxes.append(g)
        fm, fr = lerr(lg, o_lg)
        sm, sr = lerr(lg, s_lg)
        # attribution: the residual stream after every layer (E4B_FLAG_LAYER_HIDDEN)
        # against the synced oracle's, as a fraction of that layer's range
        layer_err.append([lerr(eng.read_layer_hidden(layer), osync.layer_hidden(layer))[1]
                          for layer in range(cfg.layers)])
        # synced: equal unless a near-tie; free-running: a different argmax
        # only where the oracle's top-2 margin is within twice that step's
        # logit difference (the flip the drift can cause)
        if g != s_tok:
            assert top2_margin(s_lg) < TIE_TOL * np.abs(s_lg).max(), f"pos {pos}: gpu {g} vs synced oracle {s_tok}"
            ties.append((pos, "synced"))
        if g != o_tok:
            assert top2_margin(o_lg) <= 2 * float(np.max(np.abs(lg.astype(np.float64) - o_lg))), (
                f"pos {pos}: gpu {g} vs free oracle {o_tok}")
            ties.append((pos, "free"))
        free.append((pos, fm, fr))
        sync.append((pos, sm, sr))
        assert sr < SYNC_TOL, f"pos {pos}: logits err {sr:.2e} of the logit range from the GPU's own state"
        assert fr < DRIFT_TOL, f"pos {pos}: free-running logits err {fr:.2e} of the logit range"
        if k % 32 == 31:
            say(f"c4 stated: decode {k + 1}/256 pos {pos}: synced err {sm:.2e}, free err {fm:.2e} of max "
                f"({time.time() - t0:.0f} s)")
    fr = np.array([e[2] for e in free])
    sm = np.array([e[1] for e in sync])
    sr = np.array([e[2] for e in sync])
    assert np.median(sr) < 3e-4, f"synced step logits err median {np.median(sr):.2e} of the range"
    print(f"c4 stated workload: 256 steps compared against both oracles, distinct argmax tokens "
          f"{len(set(argmaxes))}, near-ties {ties}; synced step logits err of range median {np.median(sr):.2e} "
          f"max {sr.max():.2e} (of max |logit|: median {np.median(sm):.2e} max {sm.max():.2e}); free-running err (of range) median {np.median(fr):.2e} p90 "
          f"{np.percentile(fr, 90):.2e} max {fr.max():.2e} at pos {free[int(np.argmax(fr))][0]}; new K/V rows "
          f"bit-identical to the synced oracle's in {100 * np.mean(row_same):.1f} % of entries (min row "
          f"{100 * np.min(row_same):.1f} %)")
    # where the worst steps' logit error comes from: the per-layer hidden
    # error from the GPU's own caches, against the median step's profile
    le = np.array(layer_err)
    med = np.median(le, axis=0)
    print("per-layer hidden err of range (median step), layers 0/5/10/.../34: " +
          " ".join(f"{x:.1e}" for x in med[::5]) + f" {med[-1]:.1e}")
    f1 = np.array([f[0].sum() for f in flips])
    fn = np.array([f[1].sum() for f in flips])
    print(f"new K/V entries (35 layers x 2 x 512 a step) one f16 code apart from the synced oracle's: median "
          f"{int(np.median(f1))} a step, more than one code apart: median {int(np.median(fn))}, max {int(fn.max())}")
    for i in np.argsort(-sr)[:6]:
        prof = le[i]
        ratio = prof / np.maximum(med, 1e-12)
        jump = int(np.argmax(np.diff(np.r_[0.0, prof])))
        print(f"  step pos {sync[i][0]}: logits err {sr[i]:.2e} of range; hidden err layer 0 {prof[0]:.1e}, "
              f"largest rise at layer {jump} ({prof[jump - 1] if jump else 0.0:.1e} -> {prof[jump]:.1e}), "
              f"last layer {prof[-1]:.1e} ({ratio[-1]:.1f}x the median step's); layers above 3x the median: "
              f"{[int(x) for x in np.flatnonzero(ratio > 3)]}; K/V entries one code apart {int(f1[i])} "
              f"(layers 0-4: {[int(x) for x in flips[i][0][:5]]}), more than one {int(fn[i])}")
        print("    per-layer hidden err of range: " + " ".join(f"{x:.1e}" for x in prof))
    assert le[:, 0].max() < 1e-3, f"layer 0 hidden err {le[:, 0].max():.2e} of range"
    # KV caches after position 767: written slots identical, values close
    moved = []
    for layer in range(cfg.layers):
        k, v = eng.read_kv(layer)
        slots = k.shape[1]
        ok = om.kcache(layer, slots * S).reshape(slots, cfg.kv_heads, cfg.head_dim).transpose(1, 0, 2)
        ov = om.vcache(layer, slots * S).reshape(slots, cfg.kv_heads, cfg.head_dim).transpose(1, 0, 2)
        live = np.any(ok != 0, axis=(0, 2))
        assert np.array_equal(np.any(k != 0, axis=(0, 2)), live), f"layer {layer} slots"
        for a, b in ((k, ok), (v, ov)):
            fa, fb = a.view(np.float16).astype(np.float64), b.view(np.float16).astype(np.float64)
            d = np.abs(fa - fb)
            assert d.mean() <= KV_MEAN_TOL * np.abs(fb).mean(), f"layer {layer} cache values (mean)"
            rows = np.any(d[:, live] > KV_MAX_TOL * np.abs(fb).max(), axis=(0, 2))
            moved.append((layer, int(rows.sum()), float(d.max() / np.abs(fb).max())))
    print("free-running KV rows moved by more than 1e-2 of max |value| (layer, rows, max rel): "
          + ", ".join(f"({l},{r},{m:.1e})" for l, r, m in moved if r))


def test_c4_width_256_forced_tokens_argmax():
    # 256 decode steps fed with random tokens (teacher forcing): every step's
    # argmax is an independent decision on a different input, compared with
    # the oracle's (near-ties reported); random-init greedy chains collapse to
    # one or two tokens, so this is the varied-input counterpart of the
    # 256-step greedy test above
    cfg = E4BConfig(layers=5, max_seq=512)
    eng, om = build(cfg, 9)
    toks = np.random.default_rng(10).integers(0, cfg.vocab, 256)
    ties = []
    for pos, t in enumerate(toks):
        g = eng.step(int(t), pos)
        o_tok, o_lg, _ = om.step(int(t), pos, want_logits=True)
        if g != o_tok:
            margin = top2_margin(o_lg)
            assert margin < TIE_TOL * np.abs(o_lg).max(), f"pos {pos}: gpu {g} vs oracle {o_tok}, margin {margin:.3e}"
            ties.append(pos)
    err = float(np.max(np.abs(eng.read_logits() - o_lg)) / np.max(np.abs(o_lg)))
    print(f"c4-width forced 256: near-ties {ties}, final logits err {err:.2e}")
    assert err < LOGIT_TOL


def test_unfused_attention_combine_lockstep():
    # 32-position chunks over a 4096-slot global cache = 128 chunks per head,
    # more than the o projection's fused combine prologue merges (64): the
    # global layer takes the separate combine launch + plain o GEMV path
    cfg = tiny_config(attn_chunk=32, max_seq=4096)
    eng, om = build(cfg, 61)
    prompt = np.random.default_rng(61).integers(0, cfg.vocab, 12)
    toks, ties, o_lg = lockstep(eng, om, prompt, 12)
    print(f"unfused combine: near-ties {ties}")
    assert len(ties) == 0
    err = float(np.max(np.abs(eng.read_logits() - o_lg)) / np.max(np.abs(o_lg)))
    assert err < LOGIT_TOL


def test_context_beyond_4096_positions():
    # an 8192-position global cache (128 chunks of 64 per head): a 4300-token
    # prompt through the batched prefill (chunks of 512) against the same
    # prompt through the decode step, then GPU-fed decode past position 4096
    from e4b._lib import FLAG_STEP_PREFILL
    kw = dict(hidden=256, layers=2, ffn=512, vocab=1000, window=512, ring=1024, max_seq=8192, layer_global=[0, 1])
    cfg = tiny_config(**kw)
    tensors = norm_weights_random(synth_tensors(cfg, 71), 72)
    a = Engine(cfg, tensors)
    b = Engine(tiny_config(flags=FLAG_STEP_PREFILL, **kw), tensors)
    prompt = np.random.default_rng(73).integers(0, cfg.vocab, 4300)
    ga, gb = a.prefill(prompt), b.prefill(prompt)
    la, lb = a.read_logits(), b.read_logits()
    err = float(np.max(np.abs(la - lb)) / np.max(np.abs(lb)))
    print(f"4300-token prompt: batched {ga} step {gb}, logits err {err:.2e}")
    assert err < LOGIT_TOL
    assert ga == gb or top2_margin(lb) < TIE_TOL * np.abs(lb).max()
    ta, tb = a.decode_chunk(4300, 16), b.decode_chunk(4300, 16)
    print(f"continuations {ta.tolist()} / {tb.tolist()}")
    assert np.array_equal(ta, tb)
