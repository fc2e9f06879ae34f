"""GPU parity of the full-layer KV budget (src/engine-a4b.js:587-657:
attnos SCORE mass, compactAll, generateLong) with the CPU oracle.

Tolerances:
  * scores: each head's row sums to the number of scored steps (1e-4
    relative; an invariant of normalised weights, independent of the oracle)
    and stays 0 past the live entries; against the oracle's mass within
    SCORE_TOL of the number of scored steps (the weights inherit the KV-cache
    differences of tests/test_engine_gpu.py, which scale-1.0 attention turns
    into relative weight differences of ~1e-3);
  * compaction: the gather is bit-exact (rows of the engine's own cache at the
    slots that orc.kv_keep picks from the engine's own scores); the oracle's
    selection from its own scores equals the engine's unless the two masses at
    the cut are within 1e-3 of each other (then the oracle is compacted with
    the engine's list, so the continuation is still compared);
  * decode after compaction: tokens, logits and caches as tests/
    test_engine_gpu.py (bit-exact tokens outside near-ties, logits 1e-3).
"""
import numpy as np
import pytest

import oracle as orc
from e4b._lib import FLAG_KV_SCORE
from e4b.engine import Engine
from e4b.model import norm_weights_random, synth_tensors, tiny_config
from tests.test_engine_gpu import LOGIT_TOL, TIE_TOL
from tests.util import top2_margin

pytestmark = pytest.mark.gpu

SCORE_TOL = 2e-2
GLOBAL = 1  # the full layer of the two-layer model below


def _build(seed, max_seq=64, flags=FLAG_KV_SCORE, with_tensors=False):
    cfg = tiny_config(layers=2, layer_global=[0, 1], max_seq=max_seq, flags=flags)
    tensors = norm_weights_random(synth_tensors(cfg, seed), seed + 1)
    eng = Engine(cfg, tensors)
    om = orc.OracleModel(cfg.as_dict(), {n: t.data for n, t in tensors.items()})
    return (cfg, eng, om, tensors) if with_tensors else (cfg, eng, om)


def _oracle_prompt(om, prompt):
    om.set_scoring(False)
    for i, t in enumerate(prompt):
        o_tok, o_lg, _ = om.step(int(t), i, want_logits=(i == len(prompt) - 1))
    om.set_scoring(True)
    return o_tok, o_lg


def _follow(eng, om, fed_tok, pos, n):
    """n GPU-fed decode steps from pos (input fed_tok); the oracle replays
    them with scoring.  Returns (tokens, last oracle logits, tie position or
    None)."""
    toks = eng.decode_chunk(pos, n).tolist()
    fed = [fed_tok] + toks
    o_lg = None
    for i in range(n):
        o_tok, o_lg, _ = om.step(int(fed[i]), pos + i, want_logits=True)
        if o_tok != fed[i + 1]:
            assert top2_margin(o_lg) < TIE_TOL * np.abs(o_lg).max(), f"pos {pos + i}: {fed[i + 1]} vs {o_tok}"
            return toks, o_lg, pos + i
    return toks, o_lg, None


def test_scores_match_oracle_and_sum_to_steps():
    cfg, eng, om = _build(21)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab, 20)
    g0 = eng.prefill(prompt)
    assert eng.kv_count() == 20 and np.all(eng.read_scores(GLOBAL) == 0)
    o_tok, _ = _oracle_prompt(om, prompt)
    k = 9
    toks, _, tie = _follow(eng, om, g0, 20, k)
    assert tie is None
    sc, osc = eng.read_scores(GLOBAL).astype(np.float64), om.score(GLOBAL).astype(np.float64)
    n = 20 + k
    assert eng.kv_count() == n == om.kv_count()
    np.testing.assert_allclose(sc.sum(axis=1), k, rtol=1e-4)
    assert np.all(sc[:, n:] == 0) and np.all(sc >= 0)
    err = float(np.abs(sc - osc).max())
    print(f"scores: {k} steps, max |gpu - oracle| {err:.2e}")
    assert err < SCORE_TOL * k
    # the host-fed step scores too
    eng.step(toks[-1], n)
    assert eng.kv_count() == n + 1
    np.testing.assert_allclose(eng.read_scores(GLOBAL).astype(np.float64).sum(axis=1), k + 1, rtol=1e-4)


def _compact_both(eng, om, budget, protect):
    n = eng.kv_count()
    sc_e, sc_o = eng.read_scores(GLOBAL), om.score(GLOBAL)
    keep_e = orc.kv_keep(sc_e, n, budget, protect)
    keep_o = orc.kv_keep(sc_o, n, budget, protect)
    k_before, v_before = eng.read_kv(GLOBAL)
    cnt = eng.compact(budget, protect)
    assert cnt == len(keep_e) == eng.kv_count()
    k_after, v_after = eng.read_kv(GLOBAL)
    assert np.array_equal(k_after[:, :cnt], k_before[:, keep_e]), "K gather"
    assert np.array_equal(v_after[:, :cnt], v_before[:, keep_e]), "V gather"
    assert np.all(eng.read_scores(GLOBAL) == 0)
    if not np.array_equal(keep_e, keep_o):
        # only a near-tie at the cut may separate the two selections
        mass = sc_o.astype(np.float64).sum(axis=0)
        diff = sorted(set(keep_e.tolist()) ^ set(keep_o.tolist()))
        spread = mass[diff].max() - mass[diff].min()
        assert spread < 1e-3 * max(mass[:n].max(), 1e-30), f"selections differ beyond a near-tie: {diff}"
        print(f"near-tie at the cut: {diff}")
    om.compact_with({GLOBAL: keep_e})
    return cnt


@pytest.mark.parametrize("budget,protect", [(16, 4), (24, 24), (10, 0)])
def test_compaction_gather_and_decode_after(budget, protect):
    cfg, eng, om = _build(33)
    prompt = np.random.default_rng(budget).integers(0, cfg.vocab, 30)
    g0 = eng.prefill(prompt)
    _oracle_prompt(om, prompt)
    toks, _, tie = _follow(eng, om, g0, 30, 8)
    assert tie is None
    cnt = _compact_both(eng, om, budget, protect)
    assert cnt == budget
    # decode continues at position 38, full-layer slot `budget`
    toks2, o_lg, tie = _follow(eng, om, toks[-1], 38, 12)
    print(f"budget {budget}/{protect}: after compaction {toks2}, tie {tie}")
    assert tie is None
    lg = eng.read_logits()
    assert float(np.abs(lg - o_lg).max() / np.abs(o_lg).max()) < LOGIT_TOL
    assert eng.kv_count() == om.kv_count() == budget + 12


def test_generate_long_matches_oracle_schedule():
    # generateLong with a small budget: prompt past decap -> probe step +
    # compaction, then recompactions every (decap - budget) / 8 chunks
    budget, protect, decap = 16, 4, 24
    cfg, eng, om, _ = _build(45, with_tensors=True)
    prompt = np.random.default_rng(7).integers(0, cfg.vocab, 30)
    out = eng.generate_long(prompt, 40, eos=(), budget=budget, protect=protect, decap=decap)
    assert len(out) == 40
    assert eng.kv_count() <= decap
    # the oracle under the same schedule, its selections from its own scores,
    # fed with the GPU's tokens (teacher-forced): a near-tie that picks the
    # other token does not end the comparison
    ref, o_lg = _oracle_generate_long(om, prompt, 40, budget, protect, decap, feed=out)
    assert len(ref) == len(out) == 40
    ties = []
    for i, (g, (o, near)) in enumerate(zip(out, ref)):
        if g != o:
            assert near, f"token {i}: gpu {g} vs oracle {o}"
            ties.append(i)
    # the last step's logits depend on every compacted cache: they match when
    # both sides made the same selections
    err = float(np.abs(eng.read_logits() - o_lg).max() / np.abs(o_lg).max())
    print(f"generate_long: {out}, {len(out)} tokens compared, near-ties {ties}, final logits err {err:.2e}")
    assert err < LOGIT_TOL
    assert eng.kv_count() == om.kv_count()


def _oracle_generate_long(om, prompt, max_new, budget, protect, decap, feed=None):
    """generateLong on the oracle: [(token, near_tie)], prefill unscored,
    decode scored, compaction with orc.kv_keep on the oracle's scores.  With
    `feed` (another run's output tokens) each step's input is feed's previous
    token instead of the oracle's own (teacher forcing)."""
    tok, lg = _oracle_prompt(om, prompt)
    out = [(tok, top2_margin(lg) < TIE_TOL * np.abs(lg).max())]
    pos, done = len(prompt), 1

    last = [lg]

    def step():
        nonlocal pos
        inp = out[-1][0] if feed is None else feed[len(out) - 1]
        t, lg2, _ = om.step(int(inp), pos, want_logits=True)
        pos += 1
        last[0] = lg2
        out.append((t, top2_margin(lg2) < TIE_TOL * np.abs(lg2).max()))

    if om.kv_count() > decap:
        step()
        done = 2
        om.compact(budget, protect)
    while done < max_new:
        if om.kv_count() + 8 > decap:
            om.compact(budget, protect)
        n = min(8, max_new - done)
        for _ in range(n):
            step()
        done += n
    return out[:max_new], last[0]


def test_compact_needs_the_scoring_flag():
    cfg, eng, _ = _build(5, flags=0)
    eng.prefill([1, 2, 3])
    with pytest.raises(Exception):
        eng.compact(2, 1)
    with pytest.raises(Exception):
        eng.read_scores(GLOBAL)


def test_decode_refuses_to_overrun_the_full_layer_cache():
    cfg, eng, _ = _build(6, max_seq=32)
    g0 = eng.prefill(list(range(1, 25)))
    eng.decode_chunk(24, 8)  # fills the 32 entries
    with pytest.raises(Exception):
        eng.decode_chunk(32, 1)
    eng.compact(16, 4)
    assert eng.kv_count() == 16
    assert len(eng.decode_chunk(32, 8)) == 8


def test_position_gap_appends_to_the_next_full_layer_slot():
    # counted full layers (src/engine-a4b.js:695-699): after positions 0..4 a
    # step at position 40 rotates by 40 but writes full-layer slot 5 and
    # attends to slots 0..5; the sliding ring still indexes by position.
    # Host-fed steps on the engine and the oracle agree token by token.
    cfg, eng, om = _build(77, flags=0)
    toks = [11, 22, 33, 44, 55]
    for i, t in enumerate(toks):
        a = eng.step(t, i)
        b, _, _ = om.step(t, i)
        assert a == b
    for pos, t in ((40, 66), (41, 77), (42, 88)):
        a, lg = eng.step(t, pos, want_logits=True)
        b, o_lg, _ = om.step(t, pos, want_logits=True)
        assert a == b or top2_margin(o_lg) < TIE_TOL * np.abs(o_lg).max()
        assert float(np.abs(lg - o_lg).max() / np.abs(o_lg).max()) < LOGIT_TOL
    assert eng.kv_count() == om.kv_count() == 8
    k, _ = eng.read_kv(GLOBAL)
    assert np.any(k[:, 7] != 0) and np.all(k[:, 8:] == 0)


def test_compaction_below_the_budget_keeps_everything():
    # fewer entries than the budget: every entry is kept in place, the
    # scores are zeroed and decoding continues at the same slot
    cfg, eng, om = _build(88)
    prompt = np.random.default_rng(3).integers(0, cfg.vocab, 12)
    g0 = eng.prefill(prompt)
    toks = eng.decode_chunk(12, 6).tolist()
    k_before, v_before = eng.read_kv(GLOBAL)
    assert eng.compact(64, 4) == 18 == eng.kv_count()
    k_after, v_after = eng.read_kv(GLOBAL)
    assert np.array_equal(k_after, k_before) and np.array_equal(v_after, v_before)
    assert np.all(eng.read_scores(GLOBAL) == 0)
    assert len(eng.decode_chunk(18, 4)) == 4 and eng.kv_count() == 22
