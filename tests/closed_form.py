"""Closed-form building blocks shared by the recipe pins (test_oracle_recipe,
test_oracle_a4b) and the GPU tests that check the kernels against the same
closed forms: f16/f32 rounding in float64, the reference's RMS norm and
tanh GELU, and one-hot q4_0 matrices (d = 1, one nibble 9 or 7 per row, 8
elsewhere), whose GEMV is an exact signed gather.

Also the MoE slot-pairing case (moe_pairing_case): distinct one-hot
experts, a one-hot router whose scores are exact f32 products, and distinct
per-expert scales, so the router weight of slot k, the gate/up of expert
topk[k] and the down of expert topk[k] are each identifiable in the output
(kernels/q40gu.wgsl:84-87, kernels/q40moedown.wgsl:42-75,
kernels/routertop.wgsl:19-71).
"""
import math

import numpy as np

EPS = 0.05
SQ12 = 0.70710678118654752


def f16(a):
    return np.asarray(a, np.float64).astype(np.float32).astype(np.float16).astype(np.float64)


def f32(a):
    return np.asarray(a, np.float64).astype(np.float32).astype(np.float64)


def rms(v, w=None, eps=EPS):
    v = np.asarray(v, np.float64)
    r = v / math.sqrt(float(np.mean(v * v)) + eps)
    return r if w is None else r * np.asarray(w, np.float64)


def gelu(g):
    # kernels/q40gu.wgsl:114 (tanh form, argument clamped to +-20)
    g = np.asarray(g, np.float64)
    return 0.5 * g * (1.0 + np.tanh(np.clip(0.7978845608028654 * (g + 0.044715 * g ** 3), -20.0, 20.0)))


def onehot_q40(rows, cols, sel, sign):
    """q4_0 bytes of a matrix whose row r is sign[r] * e_{sel[r]} (d = 1)."""
    nb = cols // 32
    blk = np.zeros((rows, nb, 18), np.uint8)
    blk[:, :, 1] = 0x3C  # f16 1.0, little endian
    blk[:, :, 2:] = 0x88  # every nibble 8 -> value 0
    for r in range(rows):
        c = int(sel[r])
        b, j = divmod(c, 32)
        n = 9 if sign[r] > 0 else 7
        if j < 16:
            blk[r, b, 2 + j] = (blk[r, b, 2 + j] & 0xF0) | n
        else:
            blk[r, b, 2 + j - 16] = (blk[r, b, 2 + j - 16] & 0x0F) | (n << 4)
    return blk.reshape(-1)


def select(rows, cols, seed):
    rng = np.random.default_rng(seed)
    sel = rng.integers(0, cols, rows)
    sign = np.where(rng.random(rows) < 0.5, -1.0, 1.0)
    return sel, sign


def gather(x, sel, sign):
    return sign * np.asarray(x, np.float64)[sel]




# ---------------------------------------------------------------------------
# MoE slot pairing
# ---------------------------------------------------------------------------
def moe_pairing_case(H=256, E=16, FF=64, FF2=96, seed=0, eps=EPS):
    """An MoE half-layer whose every piece is identifiable: expert e's gate,
    up and down are its own one-hot selections (seeds 1000 + 3e ...), the
    router row e is 32 e_e (a power of two, so score_e = 32 x_r[e] exactly
    in f32), pes[e] = 0.5 + e / E, and the dense branch is zero.  Returns
    the layer dict (orc.moe_ffn / MoeLayer keys) and the per-expert
    selections."""
    rng = np.random.default_rng(seed)
    z = lambda rows, cols: np.zeros(rows * cols // 32 * 18, np.uint8)  # noqa: E731
    m = {"hidden": H, "n_experts": E, "top_k": 8, "expert_ffn": FF, "dense_ffn": FF2, "eps": eps,
         "layer_scale": 1.0, "dense_gate": z(FF2, H), "dense_up": z(FF2, H), "dense_down": z(H, FF2)}
    for k in ("ffn_norm", "router_scale", "pre_ffw2", "post_ffw1", "post_ffw2", "post_ffw"):
        m[k] = rng.uniform(0.5, 1.5, H).astype(np.float32)
    rw = np.zeros((E, H), np.float32)
    rw[np.arange(E), np.arange(E)] = 32.0
    m["router_w"] = rw
    m["pes"] = (0.5 + np.arange(E) / E).astype(np.float32)
    sels = []
    gu, dn = [], []
    for e in range(E):
        g, u, d = select(FF, H, 1000 + 3 * e), select(FF, H, 1001 + 3 * e), select(H, FF, 1002 + 3 * e)
        sels.append((g, u, d))
        gu.append(np.concatenate([onehot_q40(FF, H, *g), onehot_q40(FF, H, *u)]))
        dn.append(onehot_q40(H, FF, *d))
    m["exp_gate_up"] = np.concatenate(gu)
    m["exp_down"] = np.concatenate(dn)
    return m, sels


def moe_pairing_route(m, h):
    """Top-8 ids and weights in closed form: x_r = f32(rms(h) f32(scale
    H^-1/2)) (kernels/rmsacc3.wgsl:44-53, src/engine-a4b.js:174-179); score_e
    = 32 x_r[e]; softmax over the E scores, the 8 largest (ties to the lower
    index), renormalised over the 8, times pes (kernels/routertop.wgsl:19-71).
    Also the decision margin (8th - 9th score) / max |score|."""
    H, E = m["hidden"], m["n_experts"]
    hd = np.asarray(h, np.float64)
    inv = 1.0 / math.sqrt(float(np.mean(hd * hd)) + float(m["eps"]))
    xr = f32(hd * inv * f32(np.asarray(m["router_scale"], np.float64) / math.sqrt(H)))
    s = 32.0 * xr[:E]
    order = np.argsort(-s, kind="stable")
    top = order[:8]
    p = np.exp(s - s.max())
    p /= p.sum()
    w = p[top] / p[top].sum() * np.asarray(m["pes"], np.float64)[top]
    margin = (s[order[7]] - s[order[8]]) / np.abs(s).max()
    return top, w, margin


def moe_pairing_expected(m, sels, h, top, w, mutant=None):
    """moe = sum_k w_k gather(f16(gelu(G_e xm) U_e xm), D_e), e = topk[k],
    xm = f16(rms(h) pre_ffw2); `mutant` replaces the pairing by a plausible
    mistake: "weights_rolled" (w_{k+1} with slot k), "down_by_slot" (the down
    of expert k, not topk[k]), "down_next" (gate/up of topk[k] with the down
    of topk[k+1])."""
    xm = f16(rms(h, m["pre_ffw2"], m["eps"]))
    out = np.zeros(m["hidden"])
    for k in range(8):
        e = int(top[k])
        g, u, _ = sels[e]
        de = {"down_by_slot": k, "down_next": int(top[(k + 1) % 8])}.get(mutant, e)
        wk = w[(k + 1) % 8] if mutant == "weights_rolled" else w[k]
        y = f16(gelu(gather(xm, *g)) * gather(xm, *u))
        out += wk * gather(y, *sels[de][2])
    return out
