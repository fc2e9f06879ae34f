"""Pins of the oracle's layer recipe (orc_step) and of the A4B MoE tail
(orc_moe_ffn) by branch-isolating closed forms.

Every per-layer matrix is either zero or a one-hot q4_0 selection (d = 1,
nibble 9 or 7 at one column and 8 elsewhere: an exact +-x[c]), so each GEMV
is an exact gather and each branch of a layer can be switched on alone.  A
zero branch adds an exact zero to the residual (rms of a zero vector is 0).
The expected hidden state is then written out from the reference kernels
for that special case, in float64:

  * E4B layer (src/engine.js:292-323):
      h1 = h + rms(o) w_post_attn                      (rmsaccsrq NS=2, kernels/rmsaccsrq.wgsl:31-47, MUL 1)
      x  = f16(rms(h1) w_ffn)                          (same kernel, NORM2 = 1)
      h2 = h1 + rms(down) w_post_ffw; xg = f16(h2)     (rmsaccPle: NORM2 = 0, raw hidden)
      g  = f16(gelu(W_gate xg) ple_l)                  (kernels/plegatemv.wgsl:48-57)
      h3 = (h2 + rms(W_proj g) w_post_norm) scale      (rmsaccNext / rmsacc, kernels/rmsacc.wgsl:10-26)
  * PLE inputs (kernels/pleprep.wgsl:15-46, src/engine.js:132,287-289):
      proj = W_pm h_emb H^-1/2;  ple_b = (rms(proj_b) w_pn + row_b(token) sqrt(PD)) 2^-1/2
  * attention head prep (kernels/headprep.wgsl:19-87): v is a scale-less
    head RMS; at position 0 the softmax has one key, so the output is v
  * A4B tail (kernels/a4btail.wgsl:26-71): comb = rms(t1) w1 + rms(m) w2;
    h = (h + rms(comb) wp) MUL; router input rms(h) scale H^-1/2
    (kernels/rmsacc3.wgsl:44-53, src/engine-a4b.js:174-179)

The eps of these models is large (0.05) on purpose: rms is then not
scale-invariant, so a dropped constant factor (H^-1/2, sqrt(PD), 2^-1/2, a
layer scalar applied to the branch instead of the sum) changes the result.
Norm weights are distinct random vectors, so a norm weight used in the wrong
place fails.  Each test names the mistakes it catches; test_recipe_mutants
checks that the closed forms do reject such variants.
"""
import math

import numpy as np
import pytest

import oracle as orc
from e4b.model import synth_tensors, tiny_config

from closed_form import EPS, SQ12, f16, f32, gather, gelu, onehot_q40, rms, select  # noqa: F401


def base_model(layers=1, ple=True, layer_global=None, emb_sigma=2e-4, seed=3):
    """Tiny E4B-shaped model, every layer matrix zero, random norm weights,
    an embedding of O(1) magnitude after the sqrt(H) scale."""
    cfg = tiny_config(layers=layers, vocab=64, ple_dim=256 if ple else 0, eps=EPS,
                      layer_global=layer_global or [0] * layers)
    t = synth_tensors(cfg, seed, emb_sigma=emb_sigma)
    rng = np.random.default_rng(seed + 100)
    tens = {}
    for n, ten in t.items():
        a = ten.data
        if n.startswith("blk.") and a.dtype == np.uint8:
            a = np.zeros_like(a)
        elif a.dtype == np.float32 and a.size > 1:
            a = rng.uniform(0.5, 1.5, a.size).astype(np.float32)
        tens[n] = a
    if ple:
        tens["per_layer_model_proj.weight"] = np.zeros_like(tens["per_layer_model_proj.weight"])
    return cfg, tens


def emb_row(cfg, tens, token):
    H = cfg.hidden
    return orc.q6k_row(tens["token_embd.weight"], H, token, math.sqrt(H)).astype(np.float64)


def run_step(cfg, tens, tokens):
    om = orc.OracleModel(cfg.as_dict(), tens)
    hid = None
    for p, t in enumerate(tokens):
        _, _, hid = om.step(int(t), p, want_hidden=True)
    return hid.astype(np.float64)


def check(got, want, what):
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6 * np.abs(want).max(), err_msg=what)


def set_scale(tens, layer, s):
    tens[f"blk.{layer}.layer_output_scale.weight"] = np.array([s], np.float32)


# ---------------------------------------------------------------------------
# the attention branch alone (q and k are irrelevant at position 0)
# ---------------------------------------------------------------------------

def attn_branch_pos0(cfg, tens, l, h, wv, wo):
    """h + rms(o) w_post_attn for the attention branch at position 0."""
    H, QH, KVH, HD = cfg.hidden, cfg.q_heads, cfg.kv_heads, cfg.head_dim
    p = f"blk.{l}."
    x = f16(rms(h, tens[p + "attn_norm.weight"]))
    v_raw = gather(x, *wv).reshape(KVH, HD)
    v = np.stack([f16(rms(v_raw[g])) for g in range(KVH)])           # scale-less head RMS, f16 cache
    a = np.concatenate([v[j // (QH // KVH)] for j in range(QH)])       # softmax over one key
    o = gather(a, *wo)
    return h + rms(o, tens[p + "post_attention_norm.weight"])


def with_attention(cfg, tens, l, seed):
    H, QH, KVH, HD = cfg.hidden, cfg.q_heads, cfg.kv_heads, cfg.head_dim
    wv = select(KVH * HD, H, seed)
    wo = select(H, QH * HD, seed + 1)
    tens[f"blk.{l}.attn_v.weight"] = onehot_q40(KVH * HD, H, *wv)
    tens[f"blk.{l}.attn_output.weight"] = onehot_q40(H, QH * HD, *wo)
    return wv, wo


@pytest.mark.parametrize("token", [5, 41])
def test_attention_branch_alone(token):
    # catches: v without its scale-less RMS, post_attention_norm replaced by
    # another norm, the attention residual scaled, the scalar not applied to
    # the whole sum, the attn_norm weight missing from the input
    cfg, tens = base_model()
    wv, wo = with_attention(cfg, tens, 0, 7)
    set_scale(tens, 0, 0.75)
    h0 = emb_row(cfg, tens, token)
    want = attn_branch_pos0(cfg, tens, 0, h0, wv, wo) * 0.75
    check(run_step(cfg, tens, [token]), want, "attention branch")


# ---------------------------------------------------------------------------
# the FFN branch alone
# ---------------------------------------------------------------------------

def ffn_branch(cfg, tens, l, h, wg, wu, wd):
    p = f"blk.{l}."
    x = f16(rms(h, tens[p + "ffn_norm.weight"]))
    gg = f16(gelu(gather(x, *wg)) * gather(x, *wu))
    return h + rms(gather(gg, *wd), tens[p + "post_ffw_norm.weight"])


def with_ffn(cfg, tens, l, seed):
    H, FF = cfg.hidden, cfg.ffn
    wg, wu, wd = select(FF, H, seed), select(FF, H, seed + 1), select(H, FF, seed + 2)
    tens[f"blk.{l}.ffn_gate.weight"] = onehot_q40(FF, H, *wg)
    tens[f"blk.{l}.ffn_up.weight"] = onehot_q40(FF, H, *wu)
    tens[f"blk.{l}.ffn_down.weight"] = onehot_q40(H, FF, *wd)
    return wg, wu, wd


@pytest.mark.parametrize("ple", [True, False])
def test_ffn_branch_alone(ple):
    # catches: gate and up swapped (gelu(u) g), the FFN input normed with
    # attn_norm, post_ffw_norm replaced, the scalar applied to the branch only
    cfg, tens = base_model(ple=ple)
    wg, wu, wd = with_ffn(cfg, tens, 0, 11)
    set_scale(tens, 0, 1.25)
    h0 = emb_row(cfg, tens, 9)
    want = ffn_branch(cfg, tens, 0, h0, wg, wu, wd) * 1.25
    check(run_step(cfg, tens, [9]), want, "ffn branch")


# ---------------------------------------------------------------------------
# the PLE branch alone, and the PLE inputs
# ---------------------------------------------------------------------------

def ple_inputs(cfg, tens, token, h_emb):
    """pleprep: [L][PD] per-layer inputs of `token` (kernels/pleprep.wgsl:15-46)."""
    H, PD, L = cfg.hidden, cfg.ple_dim, cfg.layers
    W = orc.q40_dequant(tens["per_layer_model_proj.weight"]).reshape(L * PD, H).astype(np.float64)
    proj = f32(f32(W @ h_emb) * (1.0 / math.sqrt(H)))
    idv = orc.q6k_row(tens["per_layer_token_embd.weight"], L * PD, token, math.sqrt(PD)).astype(np.float64)
    w_pn = tens["per_layer_proj_norm.weight"]
    return np.stack([(rms(proj[b * PD:(b + 1) * PD], w_pn) + idv[b * PD:(b + 1) * PD]) * SQ12 for b in range(L)])


def ple_branch(cfg, tens, l, h, ple_l, wpg, wpp):
    p = f"blk.{l}."
    xg = f16(h)                                            # raw hidden, no norm
    g = f16(gelu(gather(xg, *wpg)) * ple_l)
    return h + rms(gather(g, *wpp), tens[p + "post_norm.weight"])


def with_ple(cfg, tens, l, seed):
    H, PD = cfg.hidden, cfg.ple_dim
    wpg, wpp = select(PD, H, seed), select(H, PD, seed + 1)
    tens[f"blk.{l}.inp_gate.weight"] = onehot_q40(PD, H, *wpg)
    tens[f"blk.{l}.proj.weight"] = onehot_q40(H, PD, *wpp)
    return wpg, wpp


@pytest.mark.parametrize("token", [3, 60])
def test_ple_branch_table_only(token):
    # model projection zero: ple_l = row_l(token) sqrt(PD) 2^-1/2.  Catches a
    # dropped sqrt(PD) or 2^-1/2, the wrong 256-block of the table row, a
    # normed (instead of raw) gate input, post_norm replaced, the scalar
    # applied to the branch only
    cfg, tens = base_model(layers=2)
    for l in range(2):
        with_ple(cfg, tens, l, 20 + 3 * l)
    set_scale(tens, 0, 0.5)
    set_scale(tens, 1, 1.5)
    h = emb_row(cfg, tens, token)
    ple = ple_inputs(cfg, tens, token, h)
    idv = orc.q6k_row(tens["per_layer_token_embd.weight"], 2 * cfg.ple_dim, token, 16.0).astype(np.float64)
    np.testing.assert_allclose(ple[1], idv[256:] * SQ12, rtol=1e-12)  # the closed form of this case
    for l in range(2):
        wpg, wpp = select(cfg.ple_dim, cfg.hidden, 20 + 3 * l), select(cfg.hidden, cfg.ple_dim, 21 + 3 * l)
        h = ple_branch(cfg, tens, l, h, ple[l], wpg, wpp) * (0.5 if l == 0 else 1.5)
    check(run_step(cfg, tens, [token]), h, "ple branch, table only")


def test_ple_inputs_model_projection():
    # one-hot model projection: proj = +-h_emb[c] H^-1/2, then per 256-block
    # rms with the per_layer_proj_norm weight, plus the table row, times
    # 2^-1/2.  Catches a missing H^-1/2 (eps makes rms scale-sensitive), the
    # norm weight indexed over all L*PD entries, the table row left out
    cfg, tens = base_model(layers=2)
    H, PD = cfg.hidden, cfg.ple_dim
    sel = select(2 * PD, H, 31)
    tens["per_layer_model_proj.weight"] = onehot_q40(2 * PD, H, *sel)
    for l in range(2):
        with_ple(cfg, tens, l, 40 + 3 * l)
    token = 17
    h = emb_row(cfg, tens, token)
    ple = ple_inputs(cfg, tens, token, h)
    proj0 = gather(h, *sel)[:PD] / math.sqrt(H)
    idv0 = orc.q6k_row(tens["per_layer_token_embd.weight"], 2 * PD, token, 16.0)[:PD].astype(np.float64)
    np.testing.assert_allclose(ple[0], (rms(proj0, tens["per_layer_proj_norm.weight"]) + idv0) * SQ12, rtol=1e-6)
    for l in range(2):
        wpg, wpp = select(PD, H, 40 + 3 * l), select(H, PD, 41 + 3 * l)
        h = ple_branch(cfg, tens, l, h, ple[l], wpg, wpp)
    check(run_step(cfg, tens, [token]), h, "ple inputs with the model projection")


# ---------------------------------------------------------------------------
# the whole layer, two layers deep: branch order, residual chain, scalar
# placement before the next layer's input norm
# ---------------------------------------------------------------------------

def test_full_layer_order_two_layers():
    # every branch on in both layers.  Catches any reordering of the
    # branches (FFN before attention, PLE before FFN), the PLE gate fed
    # from h1 instead of h2, the scalar applied before the PLE residual or
    # after the next layer's norm
    cfg, tens = base_model(layers=2)
    H, PD = cfg.hidden, cfg.ple_dim
    sel = select(2 * PD, H, 51)
    tens["per_layer_model_proj.weight"] = onehot_q40(2 * PD, H, *sel)
    ws = []
    for l in range(2):
        ws.append((with_attention(cfg, tens, l, 60 + 10 * l), with_ffn(cfg, tens, l, 63 + 10 * l),
                   with_ple(cfg, tens, l, 66 + 10 * l)))
    set_scale(tens, 0, 0.6)
    set_scale(tens, 1, 1.4)
    token = 29
    h = emb_row(cfg, tens, token)
    ple = ple_inputs(cfg, tens, token, h)
    for l in range(2):
        (wv, wo), (wg, wu, wd), (wpg, wpp) = ws[l]
        h = attn_branch_pos0(cfg, tens, l, h, wv, wo)
        h = ffn_branch(cfg, tens, l, h, wg, wu, wd)
        h = ple_branch(cfg, tens, l, h, ple[l], wpg, wpp) * (0.6 if l == 0 else 1.4)
    check(run_step(cfg, tens, [token]), h, "two full layers")


def test_no_ple_layer_scalar():
    # without per-layer embeddings the scalar multiplies h2 (rmsacc MUL)
    cfg, tens = base_model(layers=2, ple=False)
    ws = [(with_attention(cfg, tens, l, 80 + 5 * l), with_ffn(cfg, tens, l, 82 + 5 * l)) for l in range(2)]
    set_scale(tens, 0, 0.7)
    set_scale(tens, 1, 1.1)
    h = emb_row(cfg, tens, 2)
    for l in range(2):
        (wv, wo), (wg, wu, wd) = ws[l]
        h = attn_branch_pos0(cfg, tens, l, h, wv, wo)
        h = ffn_branch(cfg, tens, l, h, wg, wu, wd) * (0.7 if l == 0 else 1.1)
    check(run_step(cfg, tens, [2]), h, "two layers, no PLE")


# ---------------------------------------------------------------------------
# attention composition at position 1: which rows are q / k / v, which norm
# weight each head uses, the layer type's RoPE theta, scale 1.0
# ---------------------------------------------------------------------------

def rope_neox(x, pos, theta, hd=256, angles=128):
    """NeoX half rotation (kernels/headprep.wgsl:52-61): pairs (p, p + hd/2)."""
    x = np.asarray(x, np.float64).copy()
    half = hd // 2
    for p in range(min(angles, half)):
        th = float(np.float32(pos * float(np.float32(theta ** (-2.0 * p / hd)))))
        c, s = math.cos(th), math.sin(th)
        a, b = x[p], x[p + half]
        x[p], x[p + half] = a * c - b * s, a * s + b * c
    return x


@pytest.mark.parametrize("glob", [0, 1])
def test_attention_two_positions(glob):
    # catches: q/k/v row blocks permuted, q_norm and k_norm swapped, the other
    # layer type's theta, a 1/sqrt(head_dim) score scale, k without RoPE
    cfg, tens = base_model(layer_global=[glob])
    H, QH, KVH, HD = cfg.hidden, cfg.q_heads, cfg.kv_heads, cfg.head_dim
    wq, wk = select(QH * HD, H, 91), select(KVH * HD, H, 92)
    tens["blk.0.attn_q.weight"] = onehot_q40(QH * HD, H, *wq)
    tens["blk.0.attn_k.weight"] = onehot_q40(KVH * HD, H, *wk)
    wv, wo = with_attention(cfg, tens, 0, 93)
    theta = cfg.theta_global if glob else cfg.theta_local
    qn, kn = tens["blk.0.attn_q_norm.weight"], tens["blk.0.attn_k_norm.weight"]
    toks = [12, 50]
    ks, vs = [], []
    for pos, t in enumerate(toks):
        h0 = emb_row(cfg, tens, t)
        x = f16(rms(h0, tens["blk.0.attn_norm.weight"]))
        q = gather(x, *wq).reshape(QH, HD)
        k = gather(x, *wk).reshape(KVH, HD)
        v = gather(x, *wv).reshape(KVH, HD)
        ks.append(np.stack([f16(rope_neox(rms(k[g], kn, cfg.eps), pos, theta)) for g in range(KVH)]))
        vs.append(np.stack([f16(rms(v[g], None, cfg.eps)) for g in range(KVH)]))
    a = np.zeros(QH * HD)
    for j in range(QH):
        g = j // (QH // KVH)
        qj = f32(rope_neox(rms(q[j], qn, cfg.eps), 1, theta))
        s = np.array([qj @ ks[p][g] for p in range(2)])
        w = np.exp(s - s.max())
        w /= w.sum()
        a[j * HD:(j + 1) * HD] = f16(w[0] * vs[0][g] + w[1] * vs[1][g])
    o = gather(a, *wo)
    want = h0 + rms(o, tens["blk.0.post_attention_norm.weight"])
    got = run_step(cfg, tens, toks)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-4 * np.abs(want).max(), err_msg="attention at pos 1")


# ---------------------------------------------------------------------------
# A4B MoE tail (kernels/a4btail.wgsl:26-71) and router input
# ---------------------------------------------------------------------------

def moe_case(H=256, E=16, FF=64, FF2=96, seed=0):
    rng = np.random.default_rng(seed)
    z = lambda rows, cols: np.zeros(rows * cols // 32 * 18, np.uint8)  # noqa: E731
    m = {"hidden": H, "n_experts": E, "top_k": 8, "expert_ffn": FF, "dense_ffn": FF2, "eps": EPS,
         "layer_scale": 0.8,
         "router_w": np.zeros((E, H), np.float32), "pes": np.ones(E, np.float32),
         "dense_gate": z(FF2, H), "dense_up": z(FF2, H), "dense_down": z(H, FF2),
         "exp_gate_up": z(E * 2 * FF, H), "exp_down": z(E * H, FF)}
    for k in ("ffn_norm", "router_scale", "pre_ffw2", "post_ffw1", "post_ffw2", "post_ffw"):
        m[k] = rng.uniform(0.5, 1.5, H).astype(np.float32)
    h = rng.standard_normal(H).astype(np.float32)
    return m, h


def test_moe_tail_dense_branch_alone():
    # experts' down rows zero: comb = rms(dense) w1 (post_ffw_norm_1),
    # h' = (h + rms(comb) wp) MUL.  Catches the dense input normed with
    # pre_ffw_norm_2, w1/w2 swapped, the outer norm or the scalar misplaced
    m, h = moe_case(seed=1)
    H, FF2 = m["hidden"], m["dense_ffn"]
    wg, wu, wd = select(FF2, H, 1), select(FF2, H, 2), select(H, FF2, 3)
    m["dense_gate"], m["dense_up"] = onehot_q40(FF2, H, *wg), onehot_q40(FF2, H, *wu)
    m["dense_down"] = onehot_q40(H, FF2, *wd)
    _, _, dense, moe, hout = orc.moe_ffn(m, h)
    xd = f16(rms(h, m["ffn_norm"]))
    want_dense = gather(f16(gelu(gather(xd, *wg)) * gather(xd, *wu)), *wd)
    check(dense, want_dense, "dense branch")
    assert not np.any(moe)
    comb = rms(want_dense, m["post_ffw1"])
    check(hout, (h + rms(comb, m["post_ffw"])) * 0.8, "tail, dense only")


def test_moe_tail_expert_branch_alone():
    # identical one-hot experts, per-expert scale c: every routing gives
    # moe = c S_d f16(gelu(S_g xm) S_u xm) with xm = f16(rms(h) pre_ffw_norm_2)
    # (the top-8 weights sum to 1 before the scale); dense branch zero.
    m, h = moe_case(seed=2)
    H, E, FF = m["hidden"], m["n_experts"], m["expert_ffn"]
    wg, wu, wd = select(FF, H, 4), select(FF, H, 5), select(H, FF, 6)
    one_gu = np.concatenate([onehot_q40(FF, H, *wg), onehot_q40(FF, H, *wu)])
    m["exp_gate_up"] = np.tile(one_gu, E)
    m["exp_down"] = np.tile(onehot_q40(H, FF, *wd), E)
    m["pes"] = np.full(E, 0.3, np.float32)
    m["router_w"] = np.random.default_rng(9).standard_normal((E, H)).astype(np.float32)
    _, w, dense, moe, hout = orc.moe_ffn(m, h)
    assert not np.any(dense)
    xm = f16(rms(h, m["pre_ffw2"]))
    want_moe = 0.3 * gather(f16(gelu(gather(xm, *wg)) * gather(xm, *wu)), *wd)
    np.testing.assert_allclose(float(np.sum(w, dtype=np.float64)), 0.3, rtol=1e-6)
    np.testing.assert_allclose(moe, want_moe, rtol=0, atol=1e-6 * np.abs(want_moe).max())
    comb = rms(want_moe, m["post_ffw2"])
    check(hout, (h + rms(comb, m["post_ffw"])) * 0.8, "tail, experts only")


def test_moe_tail_both_branches():
    # comb = rms(t1) w1 + rms(m) w2 and ONE outer rms (not rms of each added)
    m, h = moe_case(seed=3)
    H, E, FF, FF2 = m["hidden"], m["n_experts"], m["expert_ffn"], m["dense_ffn"]
    wg, wu, wd = select(FF2, H, 7), select(FF2, H, 8), select(H, FF2, 9)
    m["dense_gate"], m["dense_up"] = onehot_q40(FF2, H, *wg), onehot_q40(FF2, H, *wu)
    m["dense_down"] = onehot_q40(H, FF2, *wd)
    eg, eu, ed = select(FF, H, 10), select(FF, H, 11), select(H, FF, 12)
    m["exp_gate_up"] = np.tile(np.concatenate([onehot_q40(FF, H, *eg), onehot_q40(FF, H, *eu)]), E)
    m["exp_down"] = np.tile(onehot_q40(H, FF, *ed), E)
    _, _, dense, moe, hout = orc.moe_ffn(m, h)
    xd, xm = f16(rms(h, m["ffn_norm"])), f16(rms(h, m["pre_ffw2"]))
    t1 = gather(f16(gelu(gather(xd, *wg)) * gather(xd, *wu)), *wd)
    mo = gather(f16(gelu(gather(xm, *eg)) * gather(xm, *eu)), *ed)
    comb = rms(t1, m["post_ffw1"]) + rms(mo, m["post_ffw2"])
    check(hout, (h + rms(comb, m["post_ffw"])) * 0.8, "tail, both branches")


def test_router_input_scale():
    # router row e = a_e e_e: score_e = a_e x_r[e] with
    # x_r = rms(h) router_scale H^-1/2 (src/engine-a4b.js:174-179); the
    # softmax is not scale-invariant, so a dropped H^-1/2 moves the weights
    m, h = moe_case(seed=4)
    H, E = m["hidden"], m["n_experts"]
    a = np.linspace(40.0, -40.0, E)
    rw = np.zeros((E, H), np.float32)
    rw[np.arange(E), np.arange(E)] = a
    m["router_w"] = rw
    h = np.full(H, 1.3, np.float32)
    idx, w, _, _, _ = orc.moe_ffn(m, h)
    xr = f32(rms(h, None, EPS) * f32(m["router_scale"].astype(np.float64) / math.sqrt(H)))
    s = f32(a * xr[:E])
    p = np.exp(s - s.max())
    p /= p.sum()
    top = np.argsort(-p, kind="stable")[:8]
    np.testing.assert_array_equal(idx, top)
    np.testing.assert_allclose(w, p[top] / p[top].sum(), rtol=1e-5)


# ---------------------------------------------------------------------------
# the closed forms reject plausible mistakes: each mutant of the recipe,
# written against the same special case, is far outside the tolerance
# ---------------------------------------------------------------------------

def test_recipe_mutants():
    cfg, tens = base_model(layers=1)
    H, PD = cfg.hidden, cfg.ple_dim
    sel = select(PD, H, 101)
    tens["per_layer_model_proj.weight"] = onehot_q40(PD, H, *sel)
    (wv, wo), (wg, wu, wd), (wpg, wpp) = (with_attention(cfg, tens, 0, 102), with_ffn(cfg, tens, 0, 104),
                                          with_ple(cfg, tens, 0, 107))
    set_scale(tens, 0, 0.6)
    token = 7
    got = run_step(cfg, tens, [token])
    h0 = emb_row(cfg, tens, token)
    p = "blk.0."

    def recipe(swap_gu=False, ple_gate_normed=False, no_sqrt_half=False, scale_branch_only=False,
               no_h_inv=False, post_attn_w=None):
        hh = h0.copy()
        proj = gather(hh, *sel) / (1.0 if no_h_inv else math.sqrt(H))
        idv = orc.q6k_row(tens["per_layer_token_embd.weight"], PD, token, 16.0).astype(np.float64)
        ple = (rms(proj, tens["per_layer_proj_norm.weight"]) + idv) * (1.0 if no_sqrt_half else SQ12)
        x = f16(rms(hh, tens[p + "attn_norm.weight"]))
        v = f16(rms(gather(x, *wv).reshape(2, 256)[0]))
        v2 = f16(rms(gather(x, *wv).reshape(2, 256)[1]))
        a = np.concatenate([v] * 4 + [v2] * 4)
        hh = hh + rms(gather(a, *wo), post_attn_w if post_attn_w is not None else tens[p + "post_attention_norm.weight"])
        x = f16(rms(hh, tens[p + "ffn_norm.weight"]))
        g, u = gather(x, *wg), gather(x, *wu)
        if swap_gu:
            g, u = u, g
        hh = hh + rms(gather(f16(gelu(g) * u), *wd), tens[p + "post_ffw_norm.weight"])
        xg = f16(rms(hh, tens[p + "ffn_norm.weight"])) if ple_gate_normed else f16(hh)
        br = rms(gather(f16(gelu(gather(xg, *wpg)) * ple), *wpp), tens[p + "post_norm.weight"])
        return hh + 0.6 * br if scale_branch_only else (hh + br) * 0.6

    want = recipe()
    check(got, want, "recipe")
    tol = 2e-6 * np.abs(want).max()
    for kw in ({"swap_gu": True}, {"ple_gate_normed": True}, {"no_sqrt_half": True}, {"scale_branch_only": True},
               {"no_h_inv": True}, {"post_attn_w": tens[p + "ffn_norm.weight"]}):
        err = float(np.max(np.abs(recipe(**kw) - got)))
        assert err > 100 * tol, (kw, err, tol)


def test_one_ulp_perturbation_jumps_at_f16_rounding_points():
    # The recipe rounds to f16 at fixed points (GEMV inputs, the K/V rows,
    # the GeGLU and attention outputs), so the decode step is piecewise
    # constant in tiny input changes: nudging one norm-weight vector by one
    # f32 ulp (relative 2^-23 ~ 1.2e-7) leaves most steps bit-identical and
    # moves others by a jump hundreds of times larger, wherever a rounding
    # it feeds flips and the flip travels through the scale-1.0 attention.
    # Two implementations that differ by f32-vs-double rounding (the GPU and
    # this oracle) therefore differ by sums of such jumps; the engine
    # tests' logit tolerances are stated against this (at the c4 workload a
    # single such nudge of layer 0 moves the oracle's logits by up to
    # ~7e-4 of max |logit| at some positions and by 0 at most).
    from e4b.model import E4BConfig, norm_weights_random, synth_tensors
    cfg = E4BConfig(layers=5, vocab=4096, max_seq=128, layer_global=[0, 0, 0, 0, 1])
    tens = {n: t.data for n, t in norm_weights_random(synth_tensors(cfg, 5), 6).items()}
    pert = dict(tens)
    w = np.asarray(tens["blk.0.attn_norm.weight"], np.float32)
    pert["blk.0.attn_norm.weight"] = np.nextafter(w, np.float32(np.inf)).astype(np.float32)
    a = orc.OracleModel(cfg.as_dict(), tens)
    b = orc.OracleModel(cfg.as_dict(), pert)
    b.set_keep_rows(True)
    rng = np.random.default_rng(12)
    prompt, forced = rng.integers(0, cfg.vocab, 32), rng.integers(0, cfg.vocab, 32)
    for i, t in enumerate(prompt):
        a.step(int(t), i)
    S = cfg.kv_heads * cfg.head_dim
    jumps = []
    for k, t in enumerate(forced):
        pos = len(prompt) + k
        _, la, _ = a.step(int(t), pos, want_logits=True)
        for l in range(cfg.layers):
            n = (cfg.max_seq if cfg.layer_global[l] else cfg.ring) * S
            b.set_kv(l, a.kcache(l, n), a.vcache(l, n))
        b.set_kv_count(pos)
        _, lb, _ = b.step(int(t), pos, want_logits=True)
        jumps.append(float(np.abs(la.astype(np.float64) - lb).max() / np.abs(la).max()))
    jumps = np.array(jumps)
    print(f"one-ulp nudge: {int((jumps == 0).sum())} of {jumps.size} steps bit-identical, largest jump "
          f"{jumps.max():.2e} of max |logit|")
    assert (jumps == 0).sum() >= jumps.size // 2
    assert jumps.max() > 100 * 2.0 ** -23


# ---------------------------------------------------------------------------
# MoE slot pairing (kernels/q40gu.wgsl:84-87, kernels/q40moedown.wgsl:42-75,
# kernels/routertop.wgsl:19-71): router weight k with the gate/up AND the
# down of expert topk[k]
# ---------------------------------------------------------------------------
from closed_form import moe_pairing_case, moe_pairing_expected, moe_pairing_route  # noqa: E402

PAIRING_MUTANTS = ("weights_rolled", "down_by_slot", "down_next")


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_moe_slot_pairing_closed_form(seed):
    # distinct one-hot experts, strict hand-set router order: the top-8, their
    # weights and the mixture are known in closed form; the three mutants
    # (weights paired by the wrong slot, the down of slot k instead of
    # expert topk[k], the down of the next slot's expert) are rejected by
    # more than 100x the tolerance
    m, sels = moe_pairing_case(seed=seed)
    h = np.random.default_rng(50 + seed).standard_normal(m["hidden"]).astype(np.float32)
    top, w, margin = moe_pairing_route(m, h)
    assert margin > 1e-3, f"seed {seed}: top-8 decision margin {margin:.2e}"
    assert not np.array_equal(np.sort(top), np.arange(8)), "the routed set must not be the first 8 experts"
    idx, wo, dense, moe, _ = orc.moe_ffn(m, h)
    np.testing.assert_array_equal(idx, top)
    np.testing.assert_allclose(wo, w, rtol=1e-6)
    assert not np.any(dense)
    want = moe_pairing_expected(m, sels, h, top, w)
    tol = 1e-6 * np.abs(want).max()
    np.testing.assert_allclose(moe, want, rtol=0, atol=tol)
    for mut in PAIRING_MUTANTS:
        bad = moe_pairing_expected(m, sels, h, top, w, mutant=mut)
        dev = float(np.abs(bad - moe).max())
        assert dev > 100 * tol, f"mutant {mut} not rejected ({dev:.2e} vs tolerance {tol:.2e})"


def test_moe_forced_experts_closed_form():
    # orc_moe_ffn with forced experts (the synced A4B oracle routes a layer
    # to the GPU's picks at a near-tie): the slots use the given experts,
    # weighted from the router's own softmax renormalised over them, times
    # pes; the order of the given experts does not change the mixture
    m, sels = moe_pairing_case(seed=4)
    h = np.random.default_rng(54).standard_normal(m["hidden"]).astype(np.float32)
    top, w, _ = moe_pairing_route(m, h)
    _, _, _, moe_own, _ = orc.moe_ffn(m, h)
    idx, wf, _, moe_same, _ = orc.moe_ffn(m, h, force=top[::-1])
    np.testing.assert_array_equal(idx, top[::-1])
    np.testing.assert_allclose(moe_same, moe_own, rtol=0, atol=1e-6 * np.abs(moe_own).max())
    other = np.array([int(top[0]), int(top[1])] + [e for e in range(m["n_experts"]) if e not in top][:6])
    hd = np.asarray(h, np.float64)
    inv = 1.0 / math.sqrt(float(np.mean(hd * hd)) + m["eps"])
    s = 32.0 * f32(hd * inv * f32(np.asarray(m["router_scale"], np.float64) / math.sqrt(m["hidden"])))[:m["n_experts"]]
    p = np.exp(s - s.max())
    p /= p.sum()
    wo = p[other] / p[other].sum() * np.asarray(m["pes"], np.float64)[other]
    idx, wf, _, moe_f, _ = orc.moe_ffn(m, h, force=other)
    np.testing.assert_array_equal(idx, other)
    np.testing.assert_allclose(wf, wo, rtol=1e-6)
    want = moe_pairing_expected(m, sels, h, other, wo)
    np.testing.assert_allclose(moe_f, want, rtol=0, atol=1e-6 * np.abs(want).max())
    assert np.abs(moe_f - moe_own).max() > 0.1 * np.abs(moe_own).max()
