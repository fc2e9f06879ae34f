"""GPU parity of the one-launch decode attention (config c2) against the CPU oracle.

c2: GQA 8 query / 2 KV heads, head_dim 256, f16 KV; a global layer with a
4096-position cache (RoPE theta 1e6) and a sliding layer with a 512-position
window in a 1024-slot ring (theta 1e4).  The kernel does the head prep, writes
the new K/V row at the slot of `pos`, runs split-K softmax partials over
chunks of 32 or 64 positions and merges them.

Oracle: orc.headprep (kernels/headprep.wgsl) then orc.attn_linear (global) /
orc.attn_ring (sliding ring, slot-scan with position recovery as in
kernels/attnf32.wgsl), both pinned in test_oracle.py against a textbook
softmax.  Tolerances: attention output within ATTN_TOL of max|out| (f16
output: 2 ulp at 1.0); the written K/V row within 1 f16 ulp of the oracle's
(GPU head prep in f32, oracle in double, both rounded to f16); every other
slot bit-identical.
"""
import numpy as np
import pytest

import oracle as orc
from e4b.kernels import AttnLayer

pytestmark = pytest.mark.gpu

ATTN_TOL = 2e-3
QH, KVH, HD = 8, 2, 256


def _case(slots, window, pos, theta, chunk, seed):
    rng = np.random.default_rng(seed)
    qw = (1.0 + 0.1 * rng.standard_normal(HD)).astype(np.float32)
    kw = (0.25 * (1.0 + 0.1 * rng.standard_normal(HD))).astype(np.float32)
    # cache contents at the scale of head-normed keys times kw (score std ~4)
    k = (0.25 * rng.standard_normal((KVH, slots, HD))).astype(np.float16)
    v = rng.standard_normal((KVH, slots, HD)).astype(np.float16)
    qkv = rng.standard_normal((QH + 2 * KVH) * HD).astype(np.float32)
    L = AttnLayer(QH, KVH, HD, slots, window, theta, 128, qw, kw, chunk=chunk)
    L.load_cache(k, v)
    got = L.step(qkv, pos).astype(np.float64)
    kc, vc = L.read_cache()

    inv = orc.rope_inv_freq(theta, HD, 128)
    q, kn, vn = orc.headprep(qkv, QH, KVH, HD, 128, inv, qw, kw, 1e-6, pos)
    slot = pos % slots if window else pos
    ko = np.ascontiguousarray(k.transpose(1, 0, 2))  # oracle layout [slot][kvh][hd]
    vo = np.ascontiguousarray(v.transpose(1, 0, 2))
    ko[slot] = kn.view(np.float16).reshape(KVH, HD)
    vo[slot] = vn.view(np.float16).reshape(KVH, HD)
    if window:
        want = orc.attn_ring(q, ko.view(np.uint16), vo.view(np.uint16), QH, KVH, HD, slots, window, pos)
    else:
        want = orc.attn_linear(q, ko.view(np.uint16), vo.view(np.uint16), QH, KVH, HD, pos + 1)
    want = want.view(np.float16).astype(np.float64)
    return got, want, (k, v), (kc, vc), (kn, vn), slot


def _ulp_diff(a16, b16):
    a = a16.view(np.int16).astype(np.int32)
    b = b16.view(np.int16).astype(np.int32)
    # map sign-magnitude to a monotone integer line
    a = np.where(a < 0, -32768 - a, a)
    b = np.where(b < 0, -32768 - b, b)
    return np.abs(a - b)


CASES = [
    # (name, slots, window, pos, theta, chunk)
    ("global-4095", 4096, 0, 4095, 1e6, 64),
    ("global-4095-cs32", 4096, 0, 4095, 1e6, 32),
    ("global-300", 4096, 0, 300, 1e6, 64),
    ("global-0", 4096, 0, 0, 1e6, 64),
    ("global-63", 4096, 0, 63, 1e6, 64),
    ("global-64", 4096, 0, 64, 1e6, 64),
    ("sliding-4095", 1024, 512, 4095, 1e4, 64),
    ("sliding-4095-cs32", 1024, 512, 4095, 1e4, 32),
    ("sliding-300", 1024, 512, 300, 1e4, 64),
    ("sliding-511", 1024, 512, 511, 1e4, 64),
    ("sliding-512", 1024, 512, 512, 1e4, 64),
    ("sliding-1023", 1024, 512, 1023, 1e4, 64),
    ("sliding-1024", 1024, 512, 1024, 1e4, 64),
    ("sliding-ring=window-1000", 512, 512, 1000, 1e4, 64),
]


@pytest.mark.parametrize("name,slots,window,pos,theta,chunk", CASES, ids=[c[0] for c in CASES])
def test_attn_decode_c2(name, slots, window, pos, theta, chunk):
    got, want, (k0, v0), (kc, vc), (kn, vn), slot = _case(slots, window, pos, theta, chunk, seed=pos + slots)
    scale = max(1.0, np.abs(want).max())
    err = np.abs(got - want).max() / scale
    print(f"{name}: attn max err {err:.3e} (scale {scale:.3f})")
    assert err <= ATTN_TOL
    # the new row at slot(pos), within one f16 ulp of the oracle's rounding
    assert _ulp_diff(kc[:, slot, :].reshape(-1), kn.view(np.float16)).max() <= 1
    assert _ulp_diff(vc[:, slot, :].reshape(-1), vn.view(np.float16)).max() <= 1
    # every other slot untouched
    mask = np.ones(slots, bool)
    mask[slot] = False
    np.testing.assert_array_equal(kc[:, mask, :].view(np.uint16), k0[:, mask, :].view(np.uint16))
    np.testing.assert_array_equal(vc[:, mask, :].view(np.uint16), v0[:, mask, :].view(np.uint16))


def test_attn_decode_sequence_fills_ring():
    # 40 consecutive steps through a 16-slot ring with a window of 12: the
    # kernel's own writes feed the following steps (ring wrap, window edge)
    slots, window, theta = 16, 12, 1e4
    rng = np.random.default_rng(7)
    qw = (1.0 + 0.1 * rng.standard_normal(HD)).astype(np.float32)
    kw = (0.25 * (1.0 + 0.1 * rng.standard_normal(HD))).astype(np.float32)
    L = AttnLayer(QH, KVH, HD, slots, window, theta, 128, qw, kw, chunk=32)
    L.load_cache(np.zeros((KVH, slots, HD), np.float16), np.zeros((KVH, slots, HD), np.float16))
    inv = orc.rope_inv_freq(theta, HD, 128)
    ko = np.zeros((slots, KVH, HD), np.float16)
    vo = np.zeros((slots, KVH, HD), np.float16)
    worst = 0.0
    for pos in range(40):
        qkv = rng.standard_normal((QH + 2 * KVH) * HD).astype(np.float32)
        got = L.step(qkv, pos).astype(np.float64)
        q, kn, vn = orc.headprep(qkv, QH, KVH, HD, 128, inv, qw, kw, 1e-6, pos)
        ko[pos % slots] = kn.view(np.float16).reshape(KVH, HD)
        vo[pos % slots] = vn.view(np.float16).reshape(KVH, HD)
        want = orc.attn_ring(q, ko.view(np.uint16), vo.view(np.uint16), QH, KVH, HD, slots, window, pos)
        want = want.view(np.float16).astype(np.float64)
        err = np.abs(got - want).max() / max(1.0, np.abs(want).max())
        worst = max(worst, err)
        assert err <= ATTN_TOL, (pos, err)
        # the device ring follows the oracle's (up to one f16 ulp per element)
        kc, vc = L.read_cache()
        assert _ulp_diff(kc.transpose(1, 0, 2).reshape(-1), ko.reshape(-1)).max() <= 1
        ko = kc.transpose(1, 0, 2).copy()  # continue from the device's rounding
        vo = vc.transpose(1, 0, 2).copy()
    print(f"ring sequence worst err {worst:.3e}")


def test_attn_decode_rejects_bad_shapes():
    from e4b._lib import E4BError
    L = AttnLayer(QH, KVH, HD, 64, 0, 1e6, 128, np.ones(HD, np.float32), np.ones(HD, np.float32))
    with pytest.raises(E4BError):
        L.step(np.zeros((QH + 2 * KVH) * HD, np.float32), 64)  # beyond the global cache
    L.chunk = 48
    with pytest.raises(E4BError):
        L.step(np.zeros((QH + 2 * KVH) * HD, np.float32), 3)
