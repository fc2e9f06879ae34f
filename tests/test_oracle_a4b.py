"""Pins of the oracle's A4B layer (oracle/oracle.c a4b_layer, the reference's
encodeLayer of src/engine-a4b.js:424-463) by branch-isolating closed forms,
in the manner of tests/test_oracle_recipe.py (whose helpers it uses): every
layer matrix is zero or a one-hot q4_0 gather, so each branch can be switched
on alone and written out from the reference kernels in float64.

  * full layers (src/engine-a4b.js:152-156, 330-334; kernels/headprep.wgsl
    :19-87): head dim 512, V is the scale-less head RMS of the raw K
    projection (KEQV, headprep.wgsl:23), q and k rotate only the first
    0.25 * 512 / 2 = 64 pairs (p, p + 256) with theta_global and frequencies
    THETA^(-2p/512); the cache row of k is f16
  * the attention residual h1 = h + rms(o) w_post_attn (rmsacc3), then the MoE
    half on h1 (orc_moe_ffn, pinned by the a4btail closed forms of
    tests/test_oracle_recipe.py); with every down matrix zero the half adds
    rms(0) = 0 and leaves h1 * layer_scale
"""
import math

import numpy as np

import oracle as orc
from e4b.model import synth_tensors, tiny_a4b_config
from tests.test_oracle_recipe import EPS, check, f16, gather, onehot_q40, rms, select, set_scale


def a4b_model(layer_global=(1,), kvh=(2,), seed=3, q_heads=4, n_experts=8):
    """Tiny A4B model, every layer matrix (router included) zero, random norm
    and scale vectors, an O(1) embedding."""
    L = len(layer_global)
    cfg = tiny_a4b_config(layers=L, q_heads=q_heads, layer_global=list(layer_global), layer_kv_heads=list(kvh),
                          vocab=64, eps=EPS, n_experts=n_experts, expert_ffn=32, ffn=32)
    t = synth_tensors(cfg, seed, emb_sigma=2e-4)
    rng = np.random.default_rng(seed + 100)
    tens = {}
    for n, ten in t.items():
        a = ten.data
        if n.startswith("blk.") and (a.dtype == np.uint8 or n.endswith("ffn_gate_inp.weight")):
            a = np.zeros_like(a)
        elif a.dtype == np.float32 and a.size > 1:
            a = rng.uniform(0.5, 1.5, a.size).astype(np.float32)
        tens[n] = a
    return cfg, tens


def emb_row(cfg, tens, token):
    H = cfg.hidden
    return orc.q6k_row(tens["token_embd.weight"], H, token, math.sqrt(H)).astype(np.float64)


def run(cfg, tens, tokens):
    om = orc.OracleModel(cfg.as_dict(), tens)
    hid = None
    for p, t in enumerate(tokens):
        _, _, hid = om.step(int(t), p, want_hidden=True)
    return hid.astype(np.float64)


def rope(x, pos, theta, hd, angles):
    """NeoX-half rotation of the first `angles` pairs (p, p + hd/2), angle
    f32(pos) * f32(theta^(-2p/hd)) in f32, cos/sin in double."""
    x = np.asarray(x, np.float64).copy()
    half = hd // 2
    for p in range(angles):
        inv = np.float32(theta ** (-2.0 * p / hd))
        th = float(np.float32(np.float32(pos) * inv))
        c, s = math.cos(th), math.sin(th)
        a, b = x[p], x[p + half]
        x[p], x[p + half] = a * c - b * s, a * s + b * c
    return x


def test_full_layer_v_is_the_raw_k_slice_at_position_0():
    # one full layer (head dim 512, 2 KV heads for 4 q heads), position 0:
    # the softmax over one key returns v = f16(rms(k_raw)) -- the scale-less
    # RMS of the K projection's output (no k_norm weight, no rotation, no V
    # projection).  Catches V from a V projection (absent: zero), V weighted
    # by k_norm, q head j reading the wrong KV head, the attention residual
    # normed with another weight, the layer scalar on the branch only
    cfg, tens = a4b_model()
    H, QH, (KVH, HD, _, keqv) = cfg.hidden, cfg.q_heads, cfg.layer_shape(0)
    assert keqv and HD == 512
    wk = select(KVH * HD, H, 7)
    wo = select(H, QH * HD, 8)
    tens["blk.0.attn_k.weight"] = onehot_q40(KVH * HD, H, *wk)
    tens["blk.0.attn_output.weight"] = onehot_q40(H, QH * HD, *wo)
    set_scale(tens, 0, 0.75)
    for token in (5, 41):
        h = emb_row(cfg, tens, token)
        x = f16(rms(h, tens["blk.0.attn_norm.weight"]))
        k_raw = gather(x, *wk).reshape(KVH, HD)
        v = np.stack([f16(rms(k_raw[g])) for g in range(KVH)])
        a = np.concatenate([v[j // (QH // KVH)] for j in range(QH)])
        h1 = h + rms(gather(a, *wo), tens["blk.0.post_attention_norm.weight"])
        check(run(cfg, tens, [token]), h1 * 0.75, f"full layer, position 0, token {token}")


def _attn_two_positions(cfg, tens, tokens, wq, wk, wv, wo, l=0):
    """h after the layer at position 1, the first token's K/V rows cached."""
    H, QH = cfg.hidden, cfg.q_heads
    KVH, HD, ANG, keqv = cfg.layer_shape(l)
    glob = bool(cfg.layer_global[l])
    theta = cfg.theta_global if glob else cfg.theta_local
    p = f"blk.{l}."
    ks, vs = [], []
    for pos, token in enumerate(tokens):
        h = emb_row(cfg, tens, token)
        x = f16(rms(h, tens[p + "attn_norm.weight"]))
        q_raw = gather(x, *wq).reshape(QH, HD)
        k_raw = gather(x, *wk).reshape(KVH, HD)
        v_raw = k_raw if keqv else gather(x, *wv).reshape(KVH, HD)
        q = np.stack([rope(rms(q_raw[j], tens[p + "attn_q_norm.weight"]), pos, theta, HD, ANG) for j in range(QH)])
        ks.append(np.stack([f16(rope(rms(k_raw[g], tens[p + "attn_k_norm.weight"]), pos, theta, HD, ANG))
                            for g in range(KVH)]))
        vs.append(np.stack([f16(rms(v_raw[g])) for g in range(KVH)]))
    out = []
    for j in range(QH):
        g = j // (QH // KVH)
        s = np.array([float(q[j] @ ks[t][g]) for t in range(2)])   # scale 1.0
        e = np.exp(s - s.max())
        out.append(f16((e[0] * vs[0][g] + e[1] * vs[1][g]) / e.sum()))
    o = gather(np.concatenate(out), *wo)
    return h + rms(o, tens[p + "post_attention_norm.weight"])


def test_full_layer_rotates_a_quarter_of_the_pairs_at_position_1():
    # position 1 on a full layer: scores q . k with the first 64 of 256 pairs
    # rotated by theta_global and frequencies THETA^(-2p/512).  Catches every
    # pair rotated, the sliding layers' theta or head dim in the frequencies,
    # k cached before its rotation, a 1/sqrt(d) score scale
    cfg, tens = a4b_model(seed=5)
    H, QH, (KVH, HD, ANG, _) = cfg.hidden, cfg.q_heads, cfg.layer_shape(0)
    assert ANG == 64
    wq, wk, wo = select(QH * HD, H, 21), select(KVH * HD, H, 22), select(H, QH * HD, 23)
    tens["blk.0.attn_q.weight"] = onehot_q40(QH * HD, H, *wq)
    tens["blk.0.attn_k.weight"] = onehot_q40(KVH * HD, H, *wk)
    tens["blk.0.attn_output.weight"] = onehot_q40(H, QH * HD, *wo)
    set_scale(tens, 0, 1.0)
    want = _attn_two_positions(cfg, tens, [11, 37], wq, wk, None, wo)
    check(run(cfg, tens, [11, 37]), want, "full layer, position 1")
    # the same layer with every pair rotated is a different function
    alt = dict(tens)
    cfg2, _ = a4b_model(seed=5)
    cfg2.rope_angles_full = 256
    assert np.abs(run(cfg2, alt, [11, 37]) - want).max() > 100 * 2e-6 * np.abs(want).max()


def test_sliding_layer_own_v_projection_at_position_1():
    # a sliding layer (head dim 256, its own V projection, all 128 pairs with
    # theta_local, 4 KV heads for 4 q heads) beside the full layer's recipe
    cfg, tens = a4b_model(layer_global=(0,), kvh=(4,), seed=9)
    H, QH, (KVH, HD, ANG, keqv) = cfg.hidden, cfg.q_heads, cfg.layer_shape(0)
    assert not keqv and HD == 256 and ANG == 128
    wq, wk, wv, wo = (select(QH * HD, H, 31), select(KVH * HD, H, 32), select(KVH * HD, H, 33),
                      select(H, QH * HD, 34))
    tens["blk.0.attn_q.weight"] = onehot_q40(QH * HD, H, *wq)
    tens["blk.0.attn_k.weight"] = onehot_q40(KVH * HD, H, *wk)
    tens["blk.0.attn_v.weight"] = onehot_q40(KVH * HD, H, *wv)
    tens["blk.0.attn_output.weight"] = onehot_q40(H, QH * HD, *wo)
    set_scale(tens, 0, 1.0)
    want = _attn_two_positions(cfg, tens, [3, 60], wq, wk, wv, wo)
    check(run(cfg, tens, [3, 60]), want, "sliding layer, position 1")


def test_moe_half_runs_on_the_attention_residual():
    # attention zero (h1 = h) and a live MoE half: the layer's output equals
    # orc_moe_ffn on h1 with the layer's own weights, once (the MoE input is
    # h1, not a normed h; the layer scalar is applied by the tail alone);
    # over two layers the second layer's MoE half starts from the first's output
    from tests.test_oracle_recipe import onehot_q40 as oh
    cfg, tens = a4b_model(layer_global=(0, 1), kvh=(4, 2), seed=13)
    H, E, FE, FF = cfg.hidden, cfg.n_experts, cfg.expert_ffn, cfg.ffn
    rng = np.random.default_rng(14)
    for l in range(2):
        p = f"blk.{l}."
        tens[p + "ffn_gate_inp.weight"] = rng.normal(0, 0.5, E * H).astype(np.float32)
        tens[p + "ffn_gate.weight"] = oh(FF, H, *select(FF, H, 40 + l))
        tens[p + "ffn_up.weight"] = oh(FF, H, *select(FF, H, 42 + l))
        tens[p + "ffn_down.weight"] = oh(H, FF, *select(H, FF, 44 + l))
        tens[p + "ffn_gate_up_exps.weight"] = oh(E * 2 * FE, H, *select(E * 2 * FE, H, 46 + l))
        tens[p + "ffn_down_exps.weight"] = oh(E * H, FE, *select(E * H, FE, 48 + l))
        set_scale(tens, l, 0.5 + l)
    h = emb_row(cfg, tens, 17)
    for l in range(2):
        p = f"blk.{l}."
        m = dict(hidden=H, n_experts=E, top_k=8, expert_ffn=FE, dense_ffn=FF, eps=EPS, layer_scale=0.5 + l,
                 ffn_norm=tens[p + "ffn_norm.weight"], router_scale=tens[p + "ffn_gate_inp.scale"],
                 pre_ffw2=tens[p + "pre_ffw_norm_2.weight"], router_w=tens[p + "ffn_gate_inp.weight"],
                 pes=tens[p + "ffn_down_exps.scale"], dense_gate=tens[p + "ffn_gate.weight"],
                 dense_up=tens[p + "ffn_up.weight"], dense_down=tens[p + "ffn_down.weight"],
                 exp_gate_up=tens[p + "ffn_gate_up_exps.weight"], exp_down=tens[p + "ffn_down_exps.weight"],
                 post_ffw1=tens[p + "post_ffw_norm_1.weight"], post_ffw2=tens[p + "post_ffw_norm_2.weight"],
                 post_ffw=tens[p + "post_ffw_norm.weight"])
        h = orc.moe_ffn(m, h.astype(np.float32))[4].astype(np.float64)
    check(run(cfg, tens, [17]), h, "MoE halves over two layers")


def test_route_margin_of_the_step():
    # the smallest top-8 decision margin of a step: 0 with a zero router (all
    # scores tie), in (0, 1] with a random one, and equal to the margin of
    # the scores recomputed from the layer's MoE input in numpy (one layer,
    # attention zero so the input is the embedding row itself)
    cfg, tens = a4b_model(layer_global=(0,), kvh=(4,), seed=21, n_experts=16)
    om = orc.OracleModel(cfg.as_dict(), tens)
    om.step(7, 0)
    assert om.route_margin() == 0.0
    rng = np.random.default_rng(22)
    H, E = cfg.hidden, cfg.n_experts
    W = rng.normal(0, 0.5, E * H).astype(np.float32)
    tens["blk.0.ffn_gate_inp.weight"] = W
    om = orc.OracleModel(cfg.as_dict(), tens)
    om.step(7, 0)
    got = om.route_margin()
    h = emb_row(cfg, tens, 7)
    xr = rms(h) * (tens["blk.0.ffn_gate_inp.scale"].astype(np.float64) / math.sqrt(H))
    sc = np.sort(W.reshape(E, H).astype(np.float64) @ xr)[::-1]
    want = (sc[7] - sc[8]) / np.abs(sc).max()
    assert 0.0 < got <= 1.0
    assert abs(got - want) <= 1e-4 * abs(want) + 1e-7, (got, want)


def test_one_ulp_nudge_jumps_in_the_a4b_recipe():
    # the A4B recipe rounds to f16 at the same kinds of points as the E4B one
    # (GEMV inputs, the K/V rows, the GeGLU and attention outputs, the MoE
    # branch inputs): nudging layer 0's input-norm weights by one f32 ulp
    # leaves most steps of the tiny model bit-identical and moves a few by a
    # jump hundreds of times larger.  At this seed the largest reaches ~9e-4
    # of max |h| (~5e-4 of the hidden range); the GPU tests' synced
    # tolerance (2e-3 of the range) is stated against sums of such jumps.
    from e4b.model import norm_weights_random
    cfg = tiny_a4b_config()
    tens = {n: t.data for n, t in norm_weights_random(synth_tensors(cfg, 41), 42).items()}
    pert = dict(tens)
    w = np.asarray(tens["blk.0.attn_norm.weight"], np.float32)
    pert["blk.0.attn_norm.weight"] = np.nextafter(w, np.float32(np.inf)).astype(np.float32)
    a = orc.OracleModel(cfg.as_dict(), tens)
    b = orc.OracleModel(cfg.as_dict(), pert)
    b.set_keep_rows(True)
    rng = np.random.default_rng(41)
    prompt, forced = rng.integers(0, cfg.vocab, 16), rng.integers(0, cfg.vocab, 40)
    for i, t in enumerate(prompt):
        a.step(int(t), i)
    jumps = []
    for k, t in enumerate(forced):
        pos = len(prompt) + k
        _, _, ha = a.step(int(t), pos, want_hidden=True)
        for l in range(cfg.layers):
            kvh, hd = a.layer_shape(l)[:2]
            n = (cfg.max_seq if cfg.layer_global[l] else cfg.ring) * kvh * hd
            b.set_kv(l, a.kcache(l, n), a.vcache(l, n))
        b.set_kv_count(pos)
        _, _, hb = b.step(int(t), pos, want_hidden=True)
        jumps.append(float(np.abs(ha.astype(np.float64) - hb).max() / (ha.max() - ha.min())))
    jumps = np.array(jumps)
    print(f"A4B one-ulp nudge: {int((jumps == 0).sum())} of {jumps.size} steps bit-identical, largest jump "
          f"{jumps.max():.2e} of the hidden range")
    assert (jumps == 0).sum() >= jumps.size // 2
    assert jumps.max() > 100 * 2.0 ** -23


def test_a4b_full_layer_mass_sums_to_the_scored_steps():
    # scoring on the A4B recipe's full layer (head dim 512, V = K): every
    # scored step adds one normalised weight row per q head, so each head's
    # mass sums to the number of scored steps and stays 0 past the entries;
    # the sliding layers keep none
    from e4b.model import norm_weights_random
    cfg = tiny_a4b_config(max_seq=64)
    tens = {n: t.data for n, t in norm_weights_random(synth_tensors(cfg, 61), 62).items()}
    om = orc.OracleModel(cfg.as_dict(), tens)
    rng = np.random.default_rng(63)
    for i, t in enumerate(rng.integers(0, cfg.vocab, 12)):
        om.step(int(t), i)
    om.set_scoring(True)
    for i, t in enumerate(rng.integers(0, cfg.vocab, 7)):
        om.step(int(t), 12 + i)
    full = cfg.layer_global.index(1)
    sc = om.score(full).astype(np.float64)
    np.testing.assert_allclose(sc.sum(axis=1), 7, rtol=1e-5)
    assert np.all(sc[:, 19:] == 0) and np.all(sc[:, :19] > 0)
    # compaction keeps the protected newest entries and the heaviest others
    keep = orc.kv_keep(om.score(full), 19, 10, 3)
    assert len(keep) == 10 and list(keep[-3:]) == [16, 17, 18]
    assert om.compact(10, 3) == 10 == om.kv_count()


def test_layer_hidden_and_forced_routing():
    # the oracle's per-layer readouts: the residual stream after each layer
    # (the last one equals the step's hidden output; with every matrix zero a
    # layer only scales h by its layer scalar, so after layer l it is
    # emb * s_0 ... s_l in f32) and, on random weights, each layer's own
    # top-8; forcing a layer to its own picks reproduces the step bit for
    # bit, forcing another set changes it while layer_topk still reports the
    # oracle's own picks
    from e4b.model import norm_weights_random
    cfg, tens = a4b_model(layer_global=(0, 1, 0), kvh=(2, 1, 2))
    sc = [0.75, 1.25, 0.5]
    for l, s in enumerate(sc):
        set_scale(tens, l, s)
    om = orc.OracleModel(cfg.as_dict(), tens)
    _, _, hid = om.step(5, 0, want_hidden=True)
    h = emb_row(cfg, tens, 5).astype(np.float32)
    for l, s in enumerate(sc):
        h = (h.astype(np.float64) * s).astype(np.float32)
        np.testing.assert_array_equal(om.layer_hidden(l), h)
    np.testing.assert_array_equal(om.layer_hidden(cfg.layers - 1), hid)

    cfg = tiny_a4b_config()
    tensors = norm_weights_random(synth_tensors(cfg, 21), 22)
    tens = {n: t.data for n, t in tensors.items()}
    a, b, c = (orc.OracleModel(cfg.as_dict(), tens) for _ in range(3))
    toks = np.random.default_rng(23).integers(0, cfg.vocab, 6)
    for p, t in enumerate(toks):
        _, lga, _ = a.step(int(t), p, want_logits=True)
        picks = [a.layer_topk(l) for l in range(cfg.layers)]
        for l in range(cfg.layers):
            b.force_topk(l, picks[l])
        _, lgb, _ = b.step(int(t), p, want_logits=True)
        np.testing.assert_array_equal(lgb, lga)
        for l in range(cfg.layers):
            np.testing.assert_array_equal(b.layer_topk(l), picks[l])
        if p == 0:
            # another expert in layer 0's eighth slot
            swapped = picks[0].copy()
            swapped[7] = next(e for e in range(cfg.n_experts) if e not in picks[0])
            c.force_topk(0, swapped)
            _, lgc, _ = c.step(int(t), p, want_logits=True)
            assert np.abs(lgc - lga).max() > 0
            np.testing.assert_array_equal(c.layer_topk(0), picks[0])
