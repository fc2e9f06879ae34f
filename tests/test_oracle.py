"""Pins the CPU oracle (oracle/) before anything is compared against it.

Each function of the oracle is checked against something it does not share
code with: the reference's own golden verdicts (KVRing), hand-derived
known-answer blocks, a transliteration of the reference WGSL's indexing,
library routines (numpy float16, torch gelu, scipy softmax), exact rational
arithmetic, or invariants that a plausible mistake (wrong nibble order, wrong
scale group, transposed operand, dropped term, off-by-one window) breaks.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

import oracle as orc
from e4b import formats

# --------------------------------------------------------------------------
# f16 conversion: exhaustive against numpy's IEEE binary16
# --------------------------------------------------------------------------


def test_h2f_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([orc.h2f(int(v)) for v in h[::1]], np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    assert np.array_equal(np.isinf(got), np.isinf(ref))


def test_f2h_matches_numpy_rne():
    rng = np.random.default_rng(0)
    xs = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 100,
        rng.standard_normal(5000).astype(np.float32) * 1e-5,  # subnormal range
        np.array([65504, 65519.99, 65520, 1e9, -1e9, 0.0, -0.0, 2.0 ** -25, 3 * 2.0 ** -26,
                  2.0 ** -24, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], np.float32),
    ])
    ref = xs.astype(np.float16).view(np.uint16)
    got = np.array([orc.f2h(float(v)) for v in xs], np.uint16)
    assert np.array_equal(got, ref)


# --------------------------------------------------------------------------
# q4_0: nibble order known-answer block + exact rational GEMV (mvtest shape)
# --------------------------------------------------------------------------


def _q40_block(d_bits: int, qs) -> bytes:
    return bytes([d_bits & 0xFF, d_bits >> 8]) + bytes(qs)


def test_q40_dequant_known_answer():
    # qs[j] = j | (15-j) << 4: lo nibbles are elements 0..15, hi nibbles 16..31
    # (kernels/q40mv.wgsl:22-29: "lo-plane = elems 0..15, hi-plane = 16..31")
    blk = _q40_block(0x3C00, [j | ((15 - j) << 4) for j in range(16)])  # d = 1.0
    got = orc.q40_dequant(np.frombuffer(blk, np.uint8))
    want = [j - 8 for j in range(16)] + [(15 - j) - 8 for j in range(16)]
    assert got.tolist() == want
    blk = _q40_block(0x3800, [0x0F] * 16)  # d = 0.5, lo = 15, hi = 0
    got = orc.q40_dequant(np.frombuffer(blk, np.uint8))
    assert got.tolist() == [3.5] * 16 + [-4.0] * 16


def test_q40_gemv_exact_rational_mvtest():
    # resident-a4b.html:427-453 structure: x_i = ((i*13+5) % 17 - 8)/8 as f16,
    # one row recomputed exactly from the bytes; here with synthetic weights.
    rows, cols = 4, 2112
    w = formats.synth_q40(11, rows, cols)
    x = np.array([((i * 13 + 5) % 17 - 8) / 8 for i in range(cols)], np.float32)
    y = orc.q40_gemv(w, rows, cols, x)
    for r in range(rows):
        acc = Fraction(0)
        for b in range(cols // 32):
            p = w[(r * (cols // 32) + b) * 18:(r * (cols // 32) + b + 1) * 18]
            d = Fraction(float(np.frombuffer(p[:2].tobytes(), np.float16)[0]))
            s = Fraction(0)
            for j in range(16):
                s += ((int(p[2 + j]) & 15) - 8) * Fraction(float(x[b * 32 + j]))
                s += ((int(p[2 + j]) >> 4) - 8) * Fraction(float(x[b * 32 + 16 + j]))
            acc += d * s
        assert y[r] == np.float32(float(acc)), (r, y[r], float(acc))


def test_q40_gemv_against_dense_matmul():
    rng = np.random.default_rng(1)
    rows, cols = 67, 704
    w = formats.synth_q40(3, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    dense = orc.q40_dequant(w).reshape(rows, cols).astype(np.float64)
    want = dense @ x.astype(np.float64)
    got = orc.q40_gemv(w, rows, cols, x)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6 * np.abs(want).max())


# --------------------------------------------------------------------------
# Q6_K: transliteration of the reference WGSL's u32-unit indexing
# (kernels/q6k.wgsl:44-71 MODE 0 and :89-127 MODE 1) on one superblock
# --------------------------------------------------------------------------


def _wgsl_q6k_mode0(blk: bytes, mult: float, parts: bool = False):
    u = np.frombuffer(blk[:208], np.uint32)  # ql units 0..31, qh 32..47, sc 48..51
    ql, qh, sc = u[0:32], u[32:48], u[48:52]
    d = float(np.frombuffer(blk[208:210], np.float16)[0])

    def i8of(word, k):  # i32(word << ((3-k)*8)) >> 24, 32-bit wraparound
        v = (int(word) << ((3 - k) * 8)) & 0xFFFFFFFF
        v = v - (1 << 32) if v >= (1 << 31) else v
        return float(v >> 24)

    y = np.zeros(256)
    qv = np.zeros(256)
    sv = np.zeros(256)
    for h in range(2):
        scW0, scW1 = sc[h * 2], sc[h * 2 + 1]
        for w in range(8):
            qlA, qlB, qhw = int(ql[h * 16 + w]), int(ql[h * 16 + 8 + w]), int(qh[h * 8 + w])
            is_ = w // 4

            def s(i):
                return i8of(scW1 if i >= 4 else scW0, i % 4)

            s0, s2, s4, s6 = s(is_), s(is_ + 2), s(is_ + 4), s(is_ + 6)
            base = h * 128 + w * 4
            for k in range(4):
                q1 = (((qlA >> (k * 8)) & 0xF) | (((qhw >> (k * 8)) & 3) << 4)) - 32
                q2 = (((qlB >> (k * 8)) & 0xF) | (((qhw >> (k * 8 + 2)) & 3) << 4)) - 32
                q3 = (((qlA >> (k * 8 + 4)) & 0xF) | (((qhw >> (k * 8 + 4)) & 3) << 4)) - 32
                q4 = (((qlB >> (k * 8 + 4)) & 0xF) | (((qhw >> (k * 8 + 6)) & 3) << 4)) - 32
                y[base + k] = d * s0 * q1 * mult
                y[base + k + 32] = d * s2 * q2 * mult
                y[base + k + 64] = d * s4 * q3 * mult
                y[base + k + 96] = d * s6 * q4 * mult
                for o, qq, ss in ((0, q1, s0), (32, q2, s2), (64, q3, s4), (96, q4, s6)):
                    qv[base + k + o], sv[base + k + o] = qq + 32, ss
    return (y, qv, sv) if parts else y


def test_q6k_dequant_matches_wgsl_indexing():
    w = formats.synth_q6k(5, 3, 512)
    for b in range(6):
        blk = w[b * 210:(b + 1) * 210].tobytes()
        want = _wgsl_q6k_mode0(blk, 1.5)
        got = orc.q6k_dequant(np.frombuffer(blk, np.uint8), 1.5)
        np.testing.assert_allclose(got, want, rtol=2e-7, atol=0)


def test_q6k_scale_groups_are_16_contiguous_elements():
    # ql = qh = 0 (every q = 0 -> value -32), distinct scales: element e must
    # carry scale sc[e // 16] (a wrong (half, quad, l) mapping breaks this)
    blk = bytearray(210)
    for j in range(16):
        blk[192 + j] = (j + 1) & 0xFF
    blk[208:210] = np.float16(1.0).tobytes()
    got = orc.q6k_dequant(np.frombuffer(bytes(blk), np.uint8), 1.0)
    assert got.tolist() == [-32.0 * (e // 16 + 1) for e in range(256)]


def test_q6k_gemv_equals_rowwise_mode0_and_refold():
    # invariant: MODE 1 == row-wise MODE 0 . x; plus the reference's
    # 255*bacc - 32*gsum refold (kernels/q6k.wgsl:113-124) evaluated exactly
    rng = np.random.default_rng(2)
    rows, cols = 9, 512
    w = formats.synth_q6k(7, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    got = orc.q6k_gemv(w, rows, cols, x, 0.0)
    dense = np.stack([orc.q6k_row(w, cols, r, 1.0) for r in range(rows)]).astype(np.float64)
    np.testing.assert_allclose(got, dense @ x, rtol=1e-6, atol=1e-7 * np.abs(dense @ x).max())
    for r in range(rows):
        acc = 0.0
        for b in range(cols // 256):
            blk = w[(r * 2 + b) * 210:(r * 2 + b + 1) * 210].tobytes()
            d = float(np.frombuffer(blk[208:210], np.float16)[0])
            _, q, s_el = _wgsl_q6k_mode0(blk, 1.0, parts=True)
            xb = x[b * 256:(b + 1) * 256].astype(np.float64)
            # unorm refold: sum s*(q/255)*x * 255 - 32 * sum s * (group x sums)
            bacc = float(np.sum(s_el * (q / 255.0) * xb))
            gsum = float(np.sum(s_el * xb))
            acc += d * (255.0 * bacc - 32.0 * gsum)
        assert abs(acc - got[r]) <= 1e-5 * max(1.0, abs(acc))


def test_q6k_softcap():
    rng = np.random.default_rng(3)
    rows, cols = 16, 256
    w = formats.synth_q6k(9, rows, cols, sigma=0.05)
    x = rng.standard_normal(cols).astype(np.float32) * 10
    raw = orc.q6k_gemv(w, rows, cols, x, 0.0).astype(np.float64)
    cap = orc.q6k_gemv(w, rows, cols, x, 30.0)
    np.testing.assert_allclose(cap, 30.0 * np.tanh(raw / 30.0), rtol=1e-6, atol=1e-6)


# --------------------------------------------------------------------------
# argmax (kernels/argmax2.wgsl): lowest index among maxima, NaN never wins
# --------------------------------------------------------------------------


def test_argmax_semantics():
    rng = np.random.default_rng(4)
    x = rng.standard_normal(100000).astype(np.float32)
    assert orc.argmax(x)[0] == int(np.argmax(x))
    x[[5, 777, 99999]] = 50.0
    assert orc.argmax(x) == (5, 50.0)
    x[0] = np.nan
    assert orc.argmax(x)[0] == 5
    allneg = np.full(10, -np.inf, np.float32)
    i, v = orc.argmax(allneg)
    assert i == 0 and v == np.float32(-3.0e38)


# --------------------------------------------------------------------------
# norms and activations: textbook / library routines
# --------------------------------------------------------------------------


def test_rmsnorm_textbook_and_invariants():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(2048).astype(np.float32) * 3
    w = rng.standard_normal(2048).astype(np.float32)
    xd = x.astype(np.float64)
    want = xd / np.sqrt(np.mean(xd * xd) + 1e-6) * w
    np.testing.assert_allclose(orc.rmsnorm(x, w), want, rtol=1e-6, atol=1e-6)
    y = orc.rmsnorm(x, None).astype(np.float64)
    assert abs(np.mean(y * y) - 1.0) < 1e-5
    np.testing.assert_allclose(orc.rmsnorm(x * 7.0, None), orc.rmsnorm(x, None), rtol=1e-5, atol=1e-6)


def test_gelu_tanh_matches_torch():
    torch = pytest.importorskip("torch")
    g = np.linspace(-8, 8, 2001, dtype=np.float32)
    want = torch.nn.functional.gelu(torch.from_numpy(g).double(), approximate="tanh").numpy()
    got = np.array([orc.gelu_tanh(float(v)) for v in g])
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)
    # +-20 clamp of the tanh argument (kernels/q40gu.wgsl:114): gelu(40) == 40
    assert orc.gelu_tanh(40.0) == 40.0 and orc.gelu_tanh(-40.0) == 0.0


# --------------------------------------------------------------------------
# router top-k (kernels/routertop.wgsl:19-71)
# --------------------------------------------------------------------------


def test_router_topk_against_softmax_and_stable_sort():
    scipy_special = pytest.importorskip("scipy.special")
    rng = np.random.default_rng(6)
    H, E, K = 256, 128, 8
    for seed in range(5):
        x = rng.standard_normal(H).astype(np.float32)
        W = (rng.standard_normal((E, H)) * 0.5).astype(np.float32)
        pes = rng.uniform(0.5, 2.0, E).astype(np.float32)
        idx, w, scores = orc.router_topk(x, W, pes, K)
        s64 = W.astype(np.float64) @ x.astype(np.float64)
        np.testing.assert_allclose(scores, s64, rtol=1e-6, atol=1e-6)
        p = scipy_special.softmax(scores.astype(np.float64))
        order = np.argsort(-p, kind="stable")[:K]
        assert idx.tolist() == order.tolist()
        want = p[order] / p[order].sum() * pes[order]
        np.testing.assert_allclose(w, want, rtol=1e-6)


def test_router_ties_lowest_index_first():
    H, E, K = 4, 16, 8
    x = np.ones(H, np.float32)
    W = np.zeros((E, H), np.float32)
    W[[3, 9, 12]] = 1.0  # three equal top scores
    idx, w, _ = orc.router_topk(x, W, np.ones(E, np.float32), K)
    assert idx[:3].tolist() == [3, 9, 12]
    assert idx[3:].tolist() == [0, 1, 2, 4, 5]  # remaining zeros, lowest index first
    assert abs(float(w.sum()) - 1.0) < 1e-6


def _router_exact(scores):
    """x = ones, one nonzero per router row: the f32 scores are exactly `scores`."""
    E = len(scores)
    W = np.zeros((E, 4), np.float32)
    W[:, 0] = np.asarray(scores, np.float32)
    return np.ones(4, np.float32), W


def test_router_ranks_on_f32_probabilities():
    # routertop.wgsl:53-64 ranks p = exp(s - max) in f32, so scores whose p
    # round equal go to the lowest index even where the scores differ.
    # (1) f32(s - max) rounds both to -63: 1.0 and the next float 1 + 2^-23
    # (at index 9, the higher score) keep index order 5, 9
    sc = np.full(16, -10.0, np.float32)
    sc[4] = 64.0
    sc[5], sc[9] = 1.0, np.nextafter(np.float32(1.0), np.float32(2.0))
    x, W = _router_exact(sc)
    idx, w, got = orc.router_topk(x, W, np.ones(16, np.float32), 8)
    np.testing.assert_array_equal(got, sc)
    assert idx[:3].tolist() == [4, 5, 9]
    assert w[1] == w[2] and w[1] > 0
    # (2) p underflows to 0 for every score 104 or more below the max: the
    # 8th pick among them is the lowest index, not the highest score
    sc = (0.5 + 0.01 * np.arange(128)).astype(np.float32)
    top = [100, 17, 60, 3, 90, 41, 77]
    sc[top] = [200.0, 199.0, 198.0, 197.0, 196.0, 195.0, 194.0]
    x, W = _router_exact(sc)
    idx, w, _ = orc.router_topk(x, W, np.ones(128, np.float32), 8)
    assert idx[:7].tolist() == top
    assert idx[7] == 0 and w[7] == 0.0  # raw-score order would pick 127
    assert abs(float(w.sum()) - 1.0) < 1e-6


# --------------------------------------------------------------------------
# RoPE / head prep (kernels/headprep.wgsl:19-87)
# --------------------------------------------------------------------------


def _prep(hd=256, angles=128, theta=1e6, pos=0, seed=0):
    rng = np.random.default_rng(seed)
    qh, kvh = 2, 1
    qkv = rng.standard_normal((qh + 2 * kvh) * hd).astype(np.float32)
    qw = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    kw = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    inv = orc.rope_inv_freq(theta, hd, angles)
    q, k, v = orc.headprep(qkv, qh, kvh, hd, angles, inv, qw, kw, 1e-6, pos)
    return qkv, qw, kw, inv, q, k, v


def test_headprep_pos0_is_weighted_rms():
    qkv, qw, _, _, q, _, v = _prep(pos=0)
    hd = 256
    x = qkv[:hd].astype(np.float64)
    np.testing.assert_allclose(q[:hd], x / np.sqrt(np.mean(x * x) + 1e-6) * qw, rtol=1e-6, atol=1e-6)
    vv = qkv[3 * hd:4 * hd].astype(np.float64)
    np.testing.assert_allclose(v.view(np.float16).astype(np.float64), vv / np.sqrt(np.mean(vv * vv) + 1e-6),
                               rtol=1e-3, atol=1e-3)


def test_rope_is_neox_half_rotation():
    # (p, p + hd/2) pairs rotate by pos * theta^(-2p/hd); an interleaved
    # (2i, 2i+1) layout or a wrong frequency fails this
    hd, pos = 256, 37
    qkv, qw, _, inv, q, _, _ = _prep(pos=pos, angles=96)
    x = qkv[:hd].astype(np.float64)
    xn = x / np.sqrt(np.mean(x * x) + 1e-6) * qw
    half = hd // 2
    z = xn[:half] + 1j * xn[half:]
    ang = np.zeros(half)
    ang[:96] = np.float32(pos) * inv.astype(np.float64)
    ang32 = (np.float32(pos) * inv).astype(np.float64)
    ang[:96] = ang32
    r = z * np.exp(1j * ang)
    want = np.concatenate([r.real, r.imag])
    np.testing.assert_allclose(q[:hd], want, rtol=2e-6, atol=2e-6)
    assert abs(float(inv[1]) - 1e6 ** (-2 / 256)) < 1e-7


def test_rope_relative_position_invariance():
    hd = 256
    rng = np.random.default_rng(9)
    qkv = rng.standard_normal(4 * hd).astype(np.float32)
    ones = np.ones(hd, np.float32)
    inv = orc.rope_inv_freq(1e4, hd, 128)

    def rot(pos):
        q, _, _ = orc.headprep(qkv, 2, 1, hd, 128, inv, ones, ones, 1e-6, pos)
        return q[:hd].astype(np.float64), q[hd:2 * hd].astype(np.float64)

    a0, b0 = rot(3)
    a1, b1 = rot(3)
    assert np.dot(a0, b0) == np.dot(a1, b1)
    # q(p).k(p') depends on p - p' only (exact up to f32 angle rounding)
    qa, _ = rot(10)
    _, kb = rot(4)
    qc, _ = rot(16)
    _, kd = rot(10)
    assert abs(np.dot(qa, kb) - np.dot(qc, kd)) < 1e-3 * max(1.0, abs(np.dot(qa, kb)))


# --------------------------------------------------------------------------
# attention: textbook softmax, ring == window, split-K == single pass
# --------------------------------------------------------------------------


def _kv(n, kvh, hd, seed):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((n, kvh, hd)).astype(np.float16)
    v = rng.standard_normal((n, kvh, hd)).astype(np.float16)
    return k, v


def _textbook(q, k, v, qh, kvh, hd, positions):
    out = np.zeros((qh, hd))
    for h in range(qh):
        hk = h // (qh // kvh)
        kk = k[positions, hk].astype(np.float64)
        vv = v[positions, hk].astype(np.float64)
        s = kk @ q[h * hd:(h + 1) * hd].astype(np.float64)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ vv
    return out.reshape(-1)


def test_attn_linear_textbook():
    qh, kvh, hd, n = 8, 2, 64, 300
    k, v = _kv(n, kvh, hd, 1)
    q = np.random.default_rng(2).standard_normal(qh * hd).astype(np.float32) * 0.2
    got = orc.attn_linear(q, k.view(np.uint16), v.view(np.uint16), qh, kvh, hd, n).view(np.float16)
    want = _textbook(q, k, v, qh, kvh, hd, np.arange(n))
    np.testing.assert_allclose(got.astype(np.float64), want, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("pos", [0, 5, 511, 512, 700, 1023, 1024, 4095])
def test_attn_ring_equals_window(pos):
    # ring slot p % RING holds position p; live window = (pos - W, pos]
    qh, kvh, hd, W, RING = 4, 2, 32, 512, 1024
    n = pos + 1
    k, v = _kv(n, kvh, hd, pos)
    kr = np.zeros((RING, kvh, hd), np.float16)
    vr = np.zeros((RING, kvh, hd), np.float16)
    for p in range(n):
        kr[p % RING], vr[p % RING] = k[p], v[p]
    q = np.random.default_rng(pos).standard_normal(qh * hd).astype(np.float32) * 0.3
    got = orc.attn_ring(q, kr.view(np.uint16), vr.view(np.uint16), qh, kvh, hd, RING, W, pos).view(np.float16)
    live = np.arange(max(0, pos - W + 1), pos + 1)
    want = _textbook(q, k, v, qh, kvh, hd, live)
    np.testing.assert_allclose(got.astype(np.float64), want, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("n,window,chunks", [(4096, 0, 16), (1000, 0, 16), (700, 512, 16), (37, 0, 16)])
def test_attn_split_combine_equals_single_pass(n, window, chunks):
    qh, kvh, hd = 4, 2, 64
    k, v = _kv(n, kvh, hd, 3)
    q = np.random.default_rng(4).standard_normal(qh * hd).astype(np.float32) * 0.3
    live = n if not window else min(n, window)
    cs = (live + chunks - 1) // chunks
    po, pme = orc.attn_split(q, k.view(np.uint16), v.view(np.uint16), qh, kvh, hd, n, window, chunks, cs)
    nch = min(chunks, (live + cs - 1) // cs)
    got = orc.attn_combine(po, pme, qh, hd, nch, chunks).view(np.float16)
    positions = np.arange(n - live, n)
    want = _textbook(q, k, v, qh, kvh, hd, positions)
    np.testing.assert_allclose(got.astype(np.float64), want, rtol=2e-3, atol=2e-3)


# --------------------------------------------------------------------------
# KV ring protocol: the reference's own TLC verdicts (DEVPLAN-KV.md:264-276)
# --------------------------------------------------------------------------


@pytest.mark.parametrize("W,Cc,fail_at,pass_at", [(4, 3, 5, 6), (6, 5, 9, 10), (5, 2, 5, 6)])
def test_kvring_small_instance_bounds(W, Cc, fail_at, pass_at):
    # sweep.sh: NCHUNKS=4, GEN=6; boundary exactly RING = W + C - 1, every
    # failure is Complete (SoundRec never violated)
    assert orc.kvring_check(W, Cc, fail_at, 4, 6) == 2
    assert orc.kvring_check(W, Cc, pass_at, 4, 6) == 0
    assert orc.kvring_check(W, Cc, pass_at + 1, 4, 6) == 0
    assert orc.kvring_check(W, Cc, W + Cc - 3, 4, 6) == 2


def test_kvring_production_constants():
    # W=1024 C=512: 1536 PASS, 1535 PASS, 1534 FAIL (NCHUNKS=3, GEN=8)
    assert orc.kvring_check(1024, 512, 1536, 3, 8) == 0
    assert orc.kvring_check(1024, 512, 1535, 3, 8) == 0
    assert orc.kvring_check(1024, 512, 1534, 3, 8) == 2


def test_kvring_soundrec_never_violated_small_sweep():
    # SoundRec holds for every ring size (a clobber only drops context), and
    # RING >= W + C - 1 is sufficient for Complete; tightness is pinned by the
    # reference's own instances above.
    for W in range(1, 8):
        for Cc in range(1, 7):
            for R in range(1, W + Cc + 3):
                rc = orc.kvring_check(W, Cc, R, 3, 4)
                assert rc in (0, 2), (W, Cc, R)
                if R >= W + Cc - 1:
                    assert rc == 0, (W, Cc, R)


def test_kvring_recover_closed_form():
    for ring in (1, 3, 1024):
        for mw in range(0, 3 * ring + 5):
            for t in range(ring):
                if t > mw:
                    continue
                r = orc.kvring_recover(t, mw, ring)
                assert r % ring == t and r <= mw and r + ring > mw


# --------------------------------------------------------------------------
# MoE half-layer (orc_moe_ffn): independent numpy restatement of the A4B
# order (src/engine-a4b.js:438-462) from pinned primitives (q4_0 dequant,
# gelu_tanh, f16 rounding) on a small shape.
# --------------------------------------------------------------------------


def _moe_case(seed, H=256, E=16, FF=64, FF2=96):
    rng = np.random.default_rng(seed)
    q = lambda rows, cols, s: formats.synth_q40(s, rows, cols, 0.02)  # noqa: E731
    m = {"hidden": H, "n_experts": E, "top_k": 8, "expert_ffn": FF, "dense_ffn": FF2, "eps": 1e-6,
         "layer_scale": 0.8,
         "ffn_norm": 1 + 0.1 * rng.standard_normal(H), "router_scale": 1 + 0.1 * rng.standard_normal(H),
         "pre_ffw2": 1 + 0.1 * rng.standard_normal(H), "router_w": 0.02 * rng.standard_normal((E, H)) * 40,
         "pes": 1 + 0.2 * rng.standard_normal(E),
         "dense_gate": q(FF2, H, seed + 1), "dense_up": q(FF2, H, seed + 2), "dense_down": q(H, FF2, seed + 3),
         "exp_gate_up": q(E * 2 * FF, H, seed + 4), "exp_down": q(E * H, FF, seed + 5),
         "post_ffw1": 1 + 0.1 * rng.standard_normal(H), "post_ffw2": 1 + 0.1 * rng.standard_normal(H),
         "post_ffw": 1 + 0.1 * rng.standard_normal(H)}
    for k, v in m.items():
        if isinstance(v, np.ndarray) and v.dtype == np.float64:
            m[k] = v.astype(np.float32)
    h = (2.0 * rng.standard_normal(H)).astype(np.float32)
    return m, h


def _moe_numpy(m, h):
    H, E, FF, FF2 = m["hidden"], m["n_experts"], m["expert_ffn"], m["dense_ffn"]
    f16 = lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float64)  # noqa: E731
    deq = lambda w, rows, cols: orc.q40_dequant(w).reshape(rows, cols).astype(np.float64)  # noqa: E731
    gelu = np.vectorize(lambda g: orc.gelu_tanh(float(g)))
    hd = h.astype(np.float64)
    rinv = 1.0 / np.sqrt(np.mean(hd * hd) + 1e-6)
    xd = f16(hd * rinv * m["ffn_norm"])
    xm = f16(hd * rinv * m["pre_ffw2"])
    rs = (m["router_scale"].astype(np.float64) / np.sqrt(H)).astype(np.float32).astype(np.float64)
    xr = (hd * rinv * rs).astype(np.float32).astype(np.float64)
    s = (m["router_w"].astype(np.float64) @ xr).astype(np.float32).astype(np.float64)
    p = np.exp(s - s.max())
    p /= p.sum()
    idx = np.argsort(-p, kind="stable")[:8]
    w = p[idx] / p[idx].sum() * m["pes"][idx]
    Wg = deq(np.concatenate([m["dense_gate"], m["dense_up"]]), 2 * FF2, H)
    g = Wg @ xd
    gd = f16(gelu(g[:FF2]) * g[FF2:])
    dense = (deq(m["dense_down"], H, FF2) @ gd).astype(np.float32).astype(np.float64)
    Wgu = deq(m["exp_gate_up"], E * 2 * FF, H).reshape(E, 2 * FF, H)
    Wdn = deq(m["exp_down"], E * H, FF).reshape(E, H, FF)
    moe = np.zeros(H)
    for k in range(8):
        e = idx[k]
        gk = Wgu[e] @ xm
        ge = f16(gelu(gk[:FF]) * gk[FF:])
        moe += float(np.float32(w[k])) * (Wdn[e] @ ge).astype(np.float32)
    r = lambda v: v / np.sqrt(np.mean(v * v) + 1e-6)  # noqa: E731
    comb = r(dense) * m["post_ffw1"] + r(moe) * m["post_ffw2"]
    hout = (hd + r(comb) * m["post_ffw"]) * m["layer_scale"]
    return idx, w, dense, moe, hout


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_moe_ffn_matches_numpy_restatement(seed):
    m, h = _moe_case(seed)
    idx, w, dense, moe, hout = orc.moe_ffn(m, h)
    ridx, rw, rdense, rmoe, rhout = _moe_numpy(m, h)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(w, rw, rtol=1e-6)
    for got, want in ((dense, rdense), (moe, rmoe), (hout, rhout)):
        np.testing.assert_allclose(got, want, rtol=0, atol=1e-5 * np.abs(want).max())


# --------------------------------------------------------------------------
# Full step (orc_step): a special case that reduces to a closed form.  With
# every per-layer matrix zero, attention, FFN and the PLE branch add exact
# zeros (rms of a zero vector is 0), so the hidden state is the embedding row
# times the product of the layer scalars, and the logits are
# softcap(E . rms(h) * w_out) with the tied Q6_K embedding E.
# --------------------------------------------------------------------------


@pytest.mark.parametrize("token,pos", [(17, 0), (999, 5)])
def test_step_zero_layers_closed_form(token, pos):
    from e4b.model import norm_weights_random, synth_tensors, tiny_config
    cfg = tiny_config()
    t = norm_weights_random(synth_tensors(cfg, 5), 6)
    for name, ten in t.items():
        if name.startswith("blk.") and ten.data.dtype == np.uint8:
            ten.data = np.zeros_like(ten.data)
        if name.endswith("layer_output_scale.weight"):
            ten.data = np.full_like(ten.data, 0.75)
    om = orc.OracleModel(cfg.as_dict(), {n: x.data for n, x in t.items()})
    for p in range(pos):
        om.step(3, p)
    tok, lg, hid = om.step(token, pos, want_logits=True, want_hidden=True)
    H = cfg.hidden
    emb = orc.q6k_row(t["token_embd.weight"].data, H, token, math.sqrt(H)).astype(np.float64)
    np.testing.assert_allclose(hid, emb * 0.75 ** cfg.layers, rtol=1e-6, atol=1e-9)
    x = emb / np.sqrt(np.mean(emb * emb) + cfg.eps) * t["output_norm.weight"].data
    E = np.stack([orc.q6k_row(t["token_embd.weight"].data, H, r) for r in range(cfg.vocab)]).astype(np.float64)
    want = 30.0 * np.tanh((E @ x.astype(np.float32).astype(np.float64)) / 30.0)
    np.testing.assert_allclose(lg, want, rtol=2e-5, atol=2e-5 * np.abs(want).max())
    assert tok == int(np.argmax(want)) or np.sort(want)[-1] - np.sort(want)[-2] < 1e-5


def test_moe_zero_router_picks_first_eight_uniformly():
    # zero router rows -> equal scores -> ties resolve to experts 0..7 with
    # weight p/sum_top(p) = 1/8, times the per-expert scale
    m, h = _moe_case(7)
    m["router_w"] = np.zeros_like(m["router_w"])
    idx, w, _, _, _ = orc.moe_ffn(m, h)
    np.testing.assert_array_equal(idx, np.arange(8))
    np.testing.assert_allclose(w, m["pes"][:8] / 8.0, rtol=1e-6)


def test_moe_identical_experts_reduce_to_one_expert():
    # every expert identical and pes = 1: the routed mixture equals one
    # expert's output whatever the routing (the weights sum to 1)
    m, h = _moe_case(8)
    E, FF, H = m["n_experts"], m["expert_ffn"], m["hidden"]
    gu1 = np.asarray(m["exp_gate_up"]).reshape(E, -1)[0]
    dn1 = np.asarray(m["exp_down"]).reshape(E, -1)[0]
    m["exp_gate_up"] = np.tile(gu1, E)
    m["exp_down"] = np.tile(dn1, E)
    m["pes"] = np.ones(E, np.float32)
    _, w, _, moe, _ = orc.moe_ffn(m, h)
    np.testing.assert_allclose(w.sum(), 1.0, rtol=1e-6)
    hd = h.astype(np.float64)
    xm = (hd / np.sqrt(np.mean(hd * hd) + 1e-6) * m["pre_ffw2"]).astype(np.float32).astype(np.float16)
    g = orc.q40_gemv(gu1, 2 * FF, H, xm.astype(np.float32)).astype(np.float64)
    ge = np.array([orc.gelu_tanh(float(a)) for a in g[:FF]]) * g[FF:]
    one = orc.q40_gemv(dn1, H, FF, ge.astype(np.float16).astype(np.float32)).astype(np.float64)
    np.testing.assert_allclose(moe, one, rtol=0, atol=2e-6 * np.abs(one).max())


# --------------------------------------------------------------------------
# Full-layer KV budget (src/engine-a4b.js:587-617 compactAll, attnos SCORE)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("masses,budget,protect,want", [
    ([0.1, 0.5, 0.2, 0.5, 0.3, 0.0], 4, 1, [1, 3, 4, 5]),   # tie at 0.5: both fit
    ([0.5, 0.5, 0.5, 0.5, 0.1, 0.2], 3, 2, [0, 4, 5]),      # four-way tie: lowest index first
    ([0.9, 0.1, 0.8], 8, 1, [0, 1, 2]),                     # budget >= n: everything kept
    ([0.9, 0.1, 0.8, 0.7], 1, 2, [2, 3]),                   # budget < protect: only the newest
    ([0.3, 0.2], 2, 5, [0, 1]),                             # protect > n
    ([], 4, 1, []),                                         # empty cache
])
def test_kv_keep_hand_cases(masses, budget, protect, want):
    sc = np.array([masses], np.float32).reshape(1, -1) if masses else np.zeros((1, 1), np.float32)
    got = orc.kv_keep(sc, len(masses), budget, protect)
    assert got.tolist() == want


@pytest.mark.parametrize("seed", range(4))
def test_kv_keep_equals_stable_sort_over_head_sums(seed):
    # an independent route to the same list: Python's stable sort of the
    # candidates by decreasing f64 head-sum, quantised masses so ties occur
    rng = np.random.default_rng(seed)
    qh, scap, n = 8, 300, 257
    sc = (rng.integers(0, 6, (qh, scap)) / 8.0).astype(np.float32)
    budget, protect = 96, 16
    got = orc.kv_keep(sc, n, budget, protect)
    mass = [sum(float(sc[h, t]) for h in range(qh)) for t in range(n)]
    cand = sorted(range(n - protect), key=lambda t: -mass[t])
    want = sorted(cand[:budget - protect] + list(range(n - protect, n)))
    assert got.tolist() == want
    # the invariant a wrong comparator or off-by-one breaks: every kept
    # candidate outweighs every dropped one
    kept = set(got.tolist())
    lo = min(mass[t] for t in kept if t < n - protect)
    hi = max(mass[t] for t in range(n - protect) if t not in kept)
    assert lo >= hi


def _tiny_scored_model(seed, **kw):
    from e4b.model import norm_weights_random, synth_tensors, tiny_config
    cfg = tiny_config(**kw)
    t = norm_weights_random(synth_tensors(cfg, seed), seed + 1)
    om = orc.OracleModel(cfg.as_dict(), {n: x.data for n, x in t.items()})
    return cfg, om


def test_scores_are_attention_weights_summing_to_one_per_step():
    # every scored step adds a probability distribution over slots [0, kv]
    # per head: after k steps each head's row sums to k, slots beyond the
    # live range stay 0, and slot t only gathers mass from steps >= t
    cfg, om = _tiny_scored_model(3, layers=2, layer_global=[0, 1])
    om.set_scoring(True)
    k = 12
    for p in range(k):
        om.step(int(5 + 7 * p) % cfg.vocab, p)
    sc = om.score(1).astype(np.float64)
    np.testing.assert_allclose(sc.sum(axis=1), k, rtol=1e-5)
    assert np.all(sc[:, k:] == 0)
    assert np.all(sc >= 0)
    # slot k-1 is live only in the last step: its mass is below 1 per head
    assert np.all(sc[:, k - 1] <= 1.0 + 1e-6)
    assert om.kv_count() == k


def test_compaction_gathers_rows_and_resets_scores():
    cfg, om = _tiny_scored_model(4, layers=2, layer_global=[0, 1], max_seq=64)
    om.set_scoring(True)
    n = 20
    for p in range(n):
        om.step(int(11 + 3 * p) % cfg.vocab, p)
    row = cfg.kv_heads * cfg.head_dim
    k_before = om.kcache(1, cfg.max_seq * row).reshape(cfg.max_seq, row)
    v_before = om.vcache(1, cfg.max_seq * row).reshape(cfg.max_seq, row)
    want_keep = orc.kv_keep(om.score(1), n, 8, 3)
    assert om.compact(8, 3) == 8 and om.kv_count() == 8
    k_after = om.kcache(1, cfg.max_seq * row).reshape(cfg.max_seq, row)
    v_after = om.vcache(1, cfg.max_seq * row).reshape(cfg.max_seq, row)
    assert np.array_equal(k_after[:8], k_before[want_keep])
    assert np.array_equal(v_after[:8], v_before[want_keep])
    assert np.all(om.score(1) == 0)
    # decoding continues at slot 8 while the position keeps counting
    om.step(7, n)
    assert om.kv_count() == 9
    assert np.any(om.kcache(1, cfg.max_seq * row).reshape(cfg.max_seq, row)[8] != k_after[8])


def test_counted_slots_equal_positions_without_compaction():
    # kv_count restarts with position 0 and tracks the position: the global
    # layer writes slot p at position p, as before counting was introduced
    cfg, om = _tiny_scored_model(5, layers=2, layer_global=[0, 1])
    for p in range(6):
        om.step(9, p)
    assert om.kv_count() == 6
    om.step(9, 0)
    assert om.kv_count() == 1


def test_state_set_kv_reproduces_a_step():
    # handing one oracle state's caches to a fresh one (set_kv + set_kv_count)
    # makes their next step identical: the step depends on the caches, the
    # entry count, the token and the position only
    from e4b.model import synth_tensors, tiny_config
    cfg = tiny_config(layers=2, layer_global=[0, 1])
    t = {n: x.data for n, x in synth_tensors(cfg, 1).items()}
    a, b = orc.OracleModel(cfg.as_dict(), t), orc.OracleModel(cfg.as_dict(), t)
    for p, tok in enumerate([3, 5, 7, 9, 11, 13]):
        a.step(tok, p)
    for l in range(cfg.layers):
        n = (cfg.max_seq if cfg.layer_global[l] else cfg.ring) * cfg.kv_heads * cfg.head_dim
        b.set_kv(l, a.kcache(l, n), a.vcache(l, n))
    b.set_kv_count(a.kv_count())
    ta, la, _ = a.step(17, 6, want_logits=True)
    tb, lb, _ = b.step(17, 6, want_logits=True)
    assert ta == tb and np.array_equal(la, lb)


def test_keep_rows_attends_to_the_handed_over_row():
    # keep_rows: the step leaves the current token's cache slot as handed over
    # and attends to it.  Handed the caches a normal step left behind (its own
    # rows included), a keep_rows step at the same position reproduces that
    # step bit for bit and reports the same rows; a perturbed row in the slot
    # changes the result, in the sliding (ring slot p % ring) and the full
    # (counted slot) layer alike, and the cache keeps the perturbed row.
    from e4b.model import synth_tensors, tiny_config
    cfg = tiny_config(layers=2, layer_global=[0, 1])
    t = {n: x.data for n, x in synth_tensors(cfg, 2).items()}
    a, b = orc.OracleModel(cfg.as_dict(), t), orc.OracleModel(cfg.as_dict(), t)
    for p, tok in enumerate([3, 5, 7, 9, 11, 13]):
        a.step(tok, p)
    pre = {}
    for l in range(cfg.layers):
        n = (cfg.max_seq if cfg.layer_global[l] else cfg.ring) * cfg.kv_heads * cfg.head_dim
        pre[l] = (a.kcache(l, n), a.vcache(l, n))
    ta, la, _ = a.step(17, 6, want_logits=True)
    S = cfg.kv_heads * cfg.head_dim
    b.set_keep_rows(True)
    for l in range(cfg.layers):
        n = pre[l][0].size
        b.set_kv(l, a.kcache(l, n), a.vcache(l, n))
    b.set_kv_count(6)
    tb, lb, _ = b.step(17, 6, want_logits=True)
    assert ta == tb and np.array_equal(la, lb)
    for l in range(cfg.layers):
        slot = 6 if cfg.layer_global[l] else 6 % cfg.ring
        ka, va = a.rows(l)
        kb, vb = b.rows(l)
        n = pre[l][0].size
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)
        assert np.array_equal(ka.reshape(-1), a.kcache(l, n).reshape(-1, S)[slot])
        assert not np.array_equal(ka.reshape(-1), pre[l][0].reshape(-1, S)[slot])  # the step wrote it
    # at position 0 the softmax over one key gives the current row all the
    # weight: a perturbed V row handed over in either layer changes the step,
    # and the cache keeps the perturbed row
    z = orc.OracleModel(cfg.as_dict(), t)
    _, l0, _ = z.step(17, 0, want_logits=True)
    for l in range(cfg.layers):
        n = (cfg.max_seq if cfg.layer_global[l] else cfg.ring) * S
        c = orc.OracleModel(cfg.as_dict(), t)
        c.set_keep_rows(True)
        for j in range(cfg.layers):
            nj = (cfg.max_seq if cfg.layer_global[j] else cfg.ring) * S
            k, v = z.kcache(j, nj), z.vcache(j, nj).reshape(-1, S).copy()
            if j == l:
                v[0, :] = z.vcache(j, nj).reshape(-1, S)[0, ::-1]  # the row reversed
            c.set_kv(j, k, v.reshape(-1))
        c.set_kv_count(0)
        _, lc, _ = c.step(17, 0, want_logits=True)
        assert not np.array_equal(lc, l0), f"layer {l}: the handed-over row is not the one attended to"
        assert np.array_equal(c.vcache(l, n).reshape(-1, S)[0], z.vcache(l, n).reshape(-1, S)[0, ::-1])
        assert np.array_equal(c.rows(l)[1].reshape(-1), z.vcache(l, n).reshape(-1, S)[0])
