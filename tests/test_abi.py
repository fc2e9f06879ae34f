"""C-ABI surface and host-side code of libe4b.so (no GPU needed).

* every function declared in include/e4b.h is exported by the library and
  bound in e4b._lib;
* the seeded generator reproduces the published splitmix64 sequence;
* the packed q4_0 / Q6_K device layouts, decoded here in numpy exactly as
  the kernels decode them, reproduce the oracle's ggml dequantisation.
"""
import os
import re

import numpy as np
import pytest

import oracle as orc
from e4b import _lib, formats

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    txt = open(os.path.join(ROOT, "include", "e4b.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(e4b_[a-z0-9_]+)\s*\(", txt)))


def test_every_declared_symbol_is_exported_and_bound():
    decl = declared_functions()
    assert len(decl) >= 20
    bound = set(_lib.exported_symbols())
    for name in decl:
        assert hasattr(_lib.lib, name), f"{name} declared in e4b.h but not exported"
        assert name in bound, f"{name} declared in e4b.h but not bound in e4b._lib"


def test_version_and_error_channel():
    assert b"gfx950" in _lib.lib.e4b_version()
    rc = _lib.lib.e4b_q40_pack(None, 1, 33, None)
    assert rc == _lib.E4B_EINVAL
    assert "e4b_q40_pack" in _lib.last_error()


def test_splitmix64_known_answers():
    # splitmix64 seeded with 0: 0xe220a8397b1dcdaf, 0x6e789e6aa1b965f4, 0x06c45d188009454f
    assert formats.synth_u64(0, 0) == 0xE220A8397B1DCDAF
    assert formats.synth_u64(0, 1) == 0x6E789E6AA1B965F4
    assert formats.synth_u64(0, 2) == 0x06C45D188009454F


def test_synth_distributions():
    x = formats.synth_normal(1, 200000)
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1.0) < 0.01
    u = formats.synth_uniform_u32(2, 100000, 0, 262144)
    assert u.min() >= 0 and u.max() < 262144
    w = formats.synth_q40(3, 64, 2048, 0.02)
    d = w.reshape(-1, 18)[:, :2].copy().view(np.float16).astype(np.float64).ravel()
    assert np.all(d >= 0) and abs(d.mean() / (0.02 / 8 * np.sqrt(2 / np.pi)) - 1) < 0.05
    q6 = formats.synth_q6k(4, 32, 2048, 1e-3).reshape(-1, 210)
    sc = q6[:, 192:208].view(np.int8)
    assert sc.min() == -32 and sc.max() == 31


def unpack_q40(packed, rows, cols):
    """numpy decode of the packed q4_0 layout, mirroring q40_dot in common.h"""
    nb = cols // 32
    nib = packed[: rows * nb * 16].view(np.uint32).reshape(rows, nb, 4)
    off = (rows * nb * 16 + 255) // 256 * 256
    sc = packed[off: off + rows * nb * 2].view(np.float16).astype(np.float64).reshape(rows, nb)
    out = np.zeros((rows, nb, 32))
    for k in range(4):
        w = nib[:, :, k]
        for i, s in enumerate((0, 8, 4, 12)):
            out[:, :, 8 * k + 2 * i] = (w >> s) & 15
            out[:, :, 8 * k + 2 * i + 1] = (w >> (s + 16)) & 15
    return ((out - 8) * sc[:, :, None]).reshape(rows, cols)


def unpack_q6k(packed, rows, cols):
    """numpy decode of the packed Q6_K layout, mirroring q6_pairs in common.h"""
    nseg, ngrp, nsb = cols // 32, cols // 16, cols // 256
    a256 = lambda n: (n + 255) // 256 * 256  # noqa: E731
    o_qb = a256(rows * nseg * 16)
    o_sc = o_qb + a256(rows * nseg * 8)
    o_d = o_sc + a256(rows * ngrp)
    qa = packed[: rows * nseg * 16].view(np.uint32).reshape(rows, nseg, 4)
    qb = packed[o_qb: o_qb + rows * nseg * 8].view(np.uint32).reshape(rows, nseg, 2)
    sc = packed[o_sc: o_sc + rows * ngrp].view(np.int8).astype(np.float64).reshape(rows, ngrp)
    d = packed[o_d: o_d + rows * nsb * 2].view(np.float16).astype(np.float64).reshape(rows, nsb)
    out = np.zeros((rows, nseg, 32))
    M6, M4, MH = 0x3F003F, 0xF000F, 0x300030
    for g in range(2):
        w0, w1, w2 = qa[:, :, 2 * g], qa[:, :, 2 * g + 1], qb[:, :, g]
        pairs = [w0 & M6, (w0 >> 6) & M6, ((w0 >> 12) & M4) | ((w2 >> 8) & MH), w1 & M6, (w1 >> 6) & M6,
                 ((w1 >> 12) & M4) | ((w2 >> 10) & MH), w2 & M6, (w2 >> 6) & M6]
        for i, p in enumerate(pairs):
            out[:, :, 16 * g + 2 * i] = p & 0x3F
            out[:, :, 16 * g + 2 * i + 1] = (p >> 16) & 0x3F
    out = out.reshape(rows, ngrp, 16) - 32
    dd = np.repeat(d, 16, axis=1)
    return (out * sc[:, :, None] * dd[:, :, None]).reshape(rows, cols)


@pytest.mark.parametrize("rows,cols", [(5, 32), (7, 2048), (3, 704)])
def test_q40_pack_roundtrip(rows, cols):
    w = formats.synth_q40(7, rows, cols)
    packed = formats.q40_pack(w, rows, cols)
    assert packed.nbytes == _lib.lib.e4b_q40_packed_bytes(rows, cols)
    np.testing.assert_array_equal(unpack_q40(packed, rows, cols), orc.q40_dequant(w).reshape(rows, cols))


@pytest.mark.parametrize("rows,cols", [(3, 256), (5, 2048), (2, 2816 // 256 * 256)])
def test_q6k_pack_roundtrip(rows, cols):
    w = formats.synth_q6k(8, rows, cols)
    packed = formats.q6k_pack(w, rows, cols)
    assert packed.nbytes == _lib.lib.e4b_q6k_packed_bytes(rows, cols)
    got = unpack_q6k(packed, rows, cols)
    want = np.stack([orc.q6k_row(w, cols, r) for r in range(rows)])
    np.testing.assert_allclose(got, want, rtol=1e-7, atol=0)


def test_tensor_bytes_matches_gguf_js():
    assert formats.tensor_bytes(_lib.GGML_Q4_0, [2048, 16384]) == 16384 * 64 * 18
    assert formats.tensor_bytes(_lib.GGML_Q6_K, [2048, 262144]) == 262144 * 8 * 210
    assert formats.tensor_bytes(_lib.GGML_F32, [7]) == 28
    with pytest.raises(ValueError):
        formats.tensor_bytes(_lib.GGML_Q4_0, [33])


def _split_hl(x):
    """The f32 -> f16 pair of e4b_split_f32 / k_tail / k_embed: hi = f16(x),
    lo = f16(x - hi), both round-to-nearest-even (numpy's f32 -> f16 cast)."""
    x = np.asarray(x, np.float32)
    hi = x.astype(np.float16)
    lo = (x - hi.astype(np.float32)).astype(np.float16)
    return hi, lo


def test_hilo_split_bound():
    # the bound the header states: |x - (hi + lo)| <= max(2^-22 |x|, 2^-25);
    # x - hi is exact in f32 (Sterbenz), so the error is lo's rounding alone
    rng = np.random.default_rng(0)
    xs = [rng.standard_normal(1_000_000).astype(np.float32)]
    for mag in (1e-4, 1e-3, 1e-2):
        xs.append((mag * rng.uniform(0.5, 2.0, 200_000) * rng.choice([-1, 1], 200_000)).astype(np.float32))
    xs.append(np.float32([0.0, 2.0 ** -25, 2.0 ** -14, 0.125, 65504.0, -3.0e4]))
    for x in xs:
        hi, lo = _split_hl(x)
        r = x.astype(np.float64) - hi.astype(np.float64)
        assert np.array_equal(r, (x - hi.astype(np.float32)).astype(np.float64))  # exact residual
        err = np.abs(x.astype(np.float64) - hi.astype(np.float64) - lo.astype(np.float64))
        bound = np.maximum(2.0 ** -22 * np.abs(x.astype(np.float64)), 2.0 ** -25)
        assert np.all(err <= bound), float(np.max(err / bound))
    # the bound is attained in order of magnitude: the split is not exact
    hi, lo = _split_hl(xs[0])
    exact = np.mean(xs[0].astype(np.float64) == hi.astype(np.float64) + lo.astype(np.float64))
    assert 0.4 < exact < 0.8, exact


def test_rope_table_matches_oracle():
    from e4b.kernels import rope_inv_freq
    for theta in (1e4, 1e6):
        np.testing.assert_array_equal(rope_inv_freq(theta, 256, 128), orc.rope_inv_freq(theta, 256, 128))


def test_native_gguf_config_matches_metadata(tmp_path):
    # e4b_gguf_config (the library's C++ reader) returns the configuration
    # written by config_to_kv; missing, non-GGUF and truncated files fail
    from e4b._lib import E4BError
    from e4b.engine import config_to_kv, gguf_config
    from e4b.gguf import write_gguf
    from e4b.model import synth_tensors, tiny_config
    cfg = tiny_config(layers=3, layer_global=[0, 1, 0], theta_local=12345.0, softcap=25.0)
    path = tmp_path / "m.gguf"
    t = synth_tensors(cfg, 5)
    write_gguf(str(path), config_to_kv(cfg), [(x.name, x.ggml_type, x.dims, x.data) for x in t.values()])
    got = gguf_config(str(path), ring=cfg.ring, max_seq=cfg.max_seq)
    for f in ("hidden", "layers", "q_heads", "kv_heads", "head_dim", "ffn", "ple_dim", "vocab", "window",
              "rope_angles", "ring", "max_seq"):
        assert getattr(got, f) == getattr(cfg, f), f
    for f in ("theta_local", "theta_global", "eps", "softcap"):
        assert abs(getattr(got, f) - getattr(cfg, f)) <= 1e-6 * abs(getattr(cfg, f)), f
    assert got.layer_global == [0, 1, 0]
    with pytest.raises(E4BError):
        gguf_config(str(tmp_path / "absent.gguf"))
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"NOPE" + bytes(60))
    with pytest.raises(E4BError):
        gguf_config(str(bad))
    trunc = tmp_path / "trunc.gguf"
    trunc.write_bytes(path.read_bytes()[:200])
    with pytest.raises(E4BError):
        gguf_config(str(trunc))


def _kv_select(score, n, budget, protect):
    import ctypes as C
    sc = np.ascontiguousarray(score, np.float32)
    keep = np.empty(max(n, 1), np.uint32)
    cnt = _lib.check(_lib.lib.e4b_kv_select(sc.ctypes.data_as(C.c_void_p), sc.shape[0], sc.shape[1], n, budget,
                                            protect, keep.ctypes.data_as(C.c_void_p)), "e4b_kv_select")
    return keep[:cnt]


@pytest.mark.parametrize("seed,n,budget,protect", [(0, 257, 96, 16), (1, 64, 64, 8), (2, 40, 10, 0), (3, 9, 2, 5),
                                                   (4, 0, 4, 1), (5, 300, 640, 64)])
def test_kv_select_matches_oracle(seed, n, budget, protect):
    # the library's host selection (used by e4b_kv_compact) against the
    # oracle's restatement of compactAll, on quantised scores so that equal
    # masses occur and the tie order is exercised
    rng = np.random.default_rng(seed)
    sc = (rng.integers(0, 5, (8, max(n, 1) + 7)) / 4.0).astype(np.float32)
    got = _kv_select(sc, n, budget, protect)
    want = orc.kv_keep(sc, n, budget, protect)
    assert np.array_equal(got, want)
    assert np.all(np.diff(got.astype(np.int64)) > 0)


def test_kv_select_rejects_bad_arguments():
    import ctypes as C
    sc = np.zeros((2, 4), np.float32)
    keep = np.empty(8, np.uint32)
    p = sc.ctypes.data_as(C.c_void_p)
    k = keep.ctypes.data_as(C.c_void_p)
    sel = _lib.lib.e4b_kv_select
    assert sel(p, 2, 4, 8, 2, 1, k) < 0   # n beyond the stride
    assert sel(p, 2, 4, 4, -1, 1, k) < 0  # negative budget
    assert sel(None, 2, 4, 4, 2, 1, k) < 0


def test_native_gguf_config_a4b(tmp_path):
    # a gemma4 MoE key set (src/engine-a4b.js:100-116) selects the A4B recipe
    # in both readers: head dims from key_length(_swa), per-layer KV heads
    # from the head_count_kv array, the recipe's theta and rotated pairs, the
    # ring widened to window + 512, the vocabulary from the embedding's rows
    # when vocab_size is absent; a head_count_kv array of the wrong length
    # and an expert_used_count other than 8 are refused
    from e4b._lib import E4BError
    from e4b.engine import config_from_kv, config_to_kv, gguf_config
    from e4b.gguf import write_gguf
    from e4b.model import synth_tensors, tiny_a4b_config
    cfg = tiny_a4b_config(layer_global=[0, 1, 0, 1], layer_kv_heads=[2, 1, 8, 2], window=8, ring=24)
    t = [(x.name, x.ggml_type, x.dims, x.data) for x in synth_tensors(cfg, 5).values()]
    kv = config_to_kv(cfg)
    assert kv["general.architecture"] == "gemma4" and kv["gemma4.attention.key_length"] == 512
    del kv["gemma4.vocab_size"]
    kv["gemma4.rope.freq_base"] = 5.0  # the recipe fixes theta whatever the file says
    path = tmp_path / "a4b.gguf"
    write_gguf(str(path), kv, t)
    for got in (gguf_config(str(path), ring=cfg.ring, max_seq=cfg.max_seq),
                config_from_kv(kv, vocab=cfg.vocab, ring=cfg.ring, max_seq=cfg.max_seq)):
        for f in ("recipe", "hidden", "layers", "q_heads", "head_dim", "head_dim_full", "rope_angles",
                  "rope_angles_full", "ffn", "n_experts", "expert_ffn", "ple_dim", "vocab", "window", "max_seq"):
            assert getattr(got, f) == getattr(cfg, f), f
        assert got.ring == cfg.window + 512  # the reference's kvSlots (src/engine-a4b.js:198)
        assert (got.theta_local, got.theta_global) == (1e4, 1e6)
        assert got.layer_global == [0, 1, 0, 1] and got.layer_kv_heads == [2, 1, 8, 2]
        assert [got.layer_shape(i) for i in range(4)] == [cfg.layer_shape(i) for i in range(4)]
    assert gguf_config(str(path), ring=4096).ring == 4096  # a larger ring is kept
    bad = dict(kv)
    bad["gemma4.attention.head_count_kv"] = [2, 1, 8]
    write_gguf(str(tmp_path / "kvh.gguf"), bad, t)
    with pytest.raises(E4BError, match="head_count_kv"):
        gguf_config(str(tmp_path / "kvh.gguf"))
    bad = dict(kv)
    bad["gemma4.expert_used_count"] = 4
    write_gguf(str(tmp_path / "topk.gguf"), bad, t)
    with pytest.raises(E4BError, match="expert_used_count"):
        gguf_config(str(tmp_path / "topk.gguf"))
    with pytest.raises(ValueError, match="expert_used_count"):
        config_from_kv(bad)


def test_create_validates_before_any_device_call():
    # e4b_create checks the configuration before its first HIP call: unknown
    # flag bits, and an A4B context longer than the full layers' attention
    # merge holds (256 chunks of 64 positions), are refused with E4B_EINVAL
    from e4b.engine import Engine
    from e4b.model import a4b_config, tiny_config
    with pytest.raises(_lib.E4BError, match="unknown flags 0x400"):
        Engine(tiny_config(flags=1 << 10))
    with pytest.raises(_lib.E4BError, match="max_seq beyond 16384"):
        Engine(a4b_config(max_seq=16385))


def test_trace_entry_points_need_the_trace_build():
    # the product library has no device-side timeline: e4b_trace_start fails
    # (before any device call) and names the build that has one
    assert _lib.lib.e4b_trace_start(1 << 16) == _lib.E4B_EINVAL
    assert "E4B_TRACE" in _lib.last_error()


def test_timeline_splits_launches_and_names_tags():
    # e4b.timeline's host logic on hand-made records: a launch is a maximal
    # run of one tag in entry order; spans, gaps and per-token sums in us at
    # a 100 MHz clock; tag names decode csrc/trace.h's variant bits
    from e4b import timeline as tl
    assert tl.tag_name((1 << 16) | (16 + 8) | (1 << 5) | (4 << 8) | (1 << 14)) == \
        "q40 geglu r16 prologue H=4096 batched"
    assert tl.tag_name((1 << 16) | (-1 + 8) | (1 << 8)) == "q40 f32 r2 attn-combine prologue"
    assert tl.tag_name((2 << 16) | 1) == "attn global" and tl.tag_name(9 << 16 | 512) == "attn_gen hd512"
    rec = np.zeros(7, tl.REC)
    a, b = (1 << 16) | 8, (2 << 16)
    # two tokens of [a x2 WGs, b x1 WG]; ticks of 10 ns
    rows = [(0, 100, a), (5, 120, a), (220, 400, b), (1000, 1100, a), (1002, 1160, a), (1250, 1400, b),
            (1400, 1500, b | 1)]
    for r, (t0, t1, tag) in zip(rec, rows):
        r["t0"], r["t1"], r["tag"] = t0, t1, tag
    ls = tl.launches(rec)
    assert [(l["tag"], l["wgs"], l["t0"], l["t1"]) for l in ls] == \
        [(a, 2, 0, 120), (b, 1, 220, 400), (a, 2, 1000, 1160), (b, 1, 1250, 1400), (b | 1, 1, 1400, 1500)]
    txt = tl.summarize(ls, 100_000, 2)
    row_a = next(ln for ln in txt.splitlines() if ln.startswith("| q40 "))
    # spans 1.2 and 1.6 us, gaps 0 and 6 us; median entry 0.025 / 0.02 us after the first,
    # last exit 0.1 / 0.3 us after the median; per token (2.8 + 6.0) / 2
    assert row_a.split(" | ")[1:8] == ["2", "1", "1.40", "3.00", "0.02", "0.20", "4.4 |"], row_a
    assert "first entry to last exit 7.5 us" in txt
