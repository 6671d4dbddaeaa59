"""Pins the C attention oracle (cpu.rs:342-387; qwen35/cpu.rs:324-365).

Checks: the independent float64 matrix form, torch's
scaled_dot_product_attention with an explicit boolean mask, closed-form
invariants, the reference's own store-then-attend order in the regime where it
is self-consistent, and planted mistakes that the checks must catch.
"""
import numpy as np
import pytest

import oracle
import oracle.textbook as tb
from tests.helpers import AttnCase

MODES = [(0, False), (4, False), (7, False), (0, True), (4, True), (3, True)]


@pytest.mark.parametrize("window,bidi", MODES)
@pytest.mark.parametrize("H,Hkv,hd", [(4, 2, 16), (6, 2, 8), (8, 8, 8), (4, 1, 16)])
@pytest.mark.parametrize("base,t", [(0, 1), (0, 9), (5, 3), (11, 6)])
def test_oracle_matches_float64_textbook(window, bidi, H, Hkv, hd, base, t):
    c = AttnCase(hash((window, bidi, H, hd, base, t)) % 1000, t=t, H=H, Hkv=Hkv, hd=hd, n_pos=base + t)
    got = c.reference(base_pos=base, window=window, bidi=bidi, threads=1)
    ref = tb.attention(c.q, c.kf, c.vf, n_heads=H, n_kv_heads=Hkv, head_dim=hd, base_pos=base,
                       window=window, bidi=bidi)
    assert np.max(np.abs(got - ref)) < 2e-6


def test_oracle_matches_torch_sdpa_with_mask():
    torch = pytest.importorskip("torch")
    H, Hkv, hd, base, t, w = 8, 2, 32, 20, 12, 9
    c = AttnCase(5, t=t, H=H, Hkv=Hkv, hd=hd, n_pos=base + t)
    got = c.reference(base_pos=base, window=w)
    q = torch.tensor(c.q, dtype=torch.float64).view(t, H, hd).transpose(0, 1)
    k = torch.tensor(c.kf, dtype=torch.float64).view(-1, Hkv, hd).transpose(0, 1)
    v = torch.tensor(c.vf, dtype=torch.float64).view(-1, Hkv, hd).transpose(0, 1)
    k = k.repeat_interleave(H // Hkv, 0)
    v = v.repeat_interleave(H // Hkv, 0)
    mask = torch.tensor(tb.mask_matrix(t, base + t, base, w, False))
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask)
    ref = ref.transpose(0, 1).reshape(t, H * hd).numpy()
    assert np.max(np.abs(got - ref)) < 2e-6


def test_threads_do_not_change_bits():
    c = AttnCase(9, t=7, H=8, Hkv=2, hd=32, n_pos=40)
    a = c.reference(base_pos=33, window=10, threads=1)
    b = c.reference(base_pos=33, window=10, threads=5)
    assert np.array_equal(a, b)


def test_single_visible_key_returns_v():
    c = AttnCase(2, t=1, H=4, Hkv=2, hd=16, n_pos=1)
    out = c.reference(base_pos=0).reshape(4, 16)
    v = c.vf.reshape(2, 16)
    for h in range(4):
        assert np.array_equal(out[h], v[h // 2])


def test_constant_values_pass_through():
    c = AttnCase(3, t=3, H=4, Hkv=2, hd=16, n_pos=30)
    vf = np.tile(np.linspace(-1, 1, 32, dtype=np.float32), (30, 1))
    out = oracle.attention(c.q, c.kf, vf, n_heads=4, n_kv_heads=2, head_dim=16, base_pos=27)
    exp = np.concatenate([vf[0, :16], vf[0, :16], vf[0, 16:], vf[0, 16:]])
    assert np.max(np.abs(out - exp[None])) < 1e-6


def test_gqa_equals_expanded_mha():
    H, Hkv, hd, t, base = 8, 2, 16, 4, 10
    c = AttnCase(4, t=t, H=H, Hkv=Hkv, hd=hd, n_pos=base + t)
    gqa = c.reference(base_pos=base)
    g = H // Hkv
    kx = np.repeat(c.kf.reshape(-1, Hkv, hd), g, axis=1).reshape(-1, H * hd)
    vx = np.repeat(c.vf.reshape(-1, Hkv, hd), g, axis=1).reshape(-1, H * hd)
    mha = oracle.attention(c.q, kx, vx, n_heads=H, n_kv_heads=H, head_dim=hd, base_pos=base)
    assert np.array_equal(gqa, mha)


def test_reference_ring_order_agrees_in_self_consistent_regime():
    """The reference stores the batch into the ring, then attends (cpu.rs:332-339
    before 343-387).  For t == 1 or base+t <= window that equals the documented
    window semantics over positions."""
    H, Hkv, hd, w = 4, 2, 8, 6
    for base, t in [(0, 1), (0, 6), (2, 4), (17, 1), (40, 1)]:
        c = AttnCase(base * 7 + t, t=t, H=H, Hkv=Hkv, hd=hd, n_pos=base + t)
        lin = c.reference(base_pos=base, window=w)
        ring_k, ring_v = c.ring(w, base + t)
        ring = oracle.attention(c.q, oracle.from_f16_bits(ring_k), oracle.from_f16_bits(ring_v),
                                n_heads=H, n_kv_heads=Hkv, head_dim=hd, base_pos=base, window=w,
                                linear=False)
        assert np.array_equal(lin, ring), (base, t)


def test_reference_ring_hazard_outside_the_regime():
    """Outside that regime earlier queries of the batch read overwritten slots:
    all but the last query differ (the ring-hazard count)."""
    H, Hkv, hd, w, base, t = 2, 1, 8, 8, 8, 4
    c = AttnCase(77, t=t, H=H, Hkv=Hkv, hd=hd, n_pos=base + t)
    lin = c.reference(base_pos=base, window=w)
    ring_k, ring_v = c.ring(w, base + t)
    ring = oracle.attention(c.q, oracle.from_f16_bits(ring_k), oracle.from_f16_bits(ring_v),
                            n_heads=H, n_kv_heads=Hkv, head_dim=hd, base_pos=base, window=w,
                            linear=False)
    differs = [not np.array_equal(lin[i], ring[i]) for i in range(t)]
    assert differs == [True, True, True, False]


# ------------------------------------------------ planted mistakes are caught --
def _textbook_variant(c, base, window, *, kv_map=None, scale=None, lo_shift=0):
    """The float64 form with one deliberate mistake, to show the checks bite."""
    q = c.q.reshape(c.t, c.H, c.hd).astype(np.float64)
    k = c.kf.reshape(-1, c.Hkv, c.hd).astype(np.float64)
    v = c.vf.reshape(-1, c.Hkv, c.hd).astype(np.float64)
    kv_map = kv_map or (lambda h: h // (c.H // c.Hkv))
    scale = 1 / np.sqrt(c.hd) if scale is None else scale
    out = np.zeros((c.t, c.H, c.hd))
    for i in range(c.t):
        pos = base + i
        lo = max(0, pos - window + 1 + lo_shift) if window else 0
        for h in range(c.H):
            s = k[lo:pos + 1, kv_map(h)] @ q[i, h] * scale
            p = np.exp(s - s.max())
            out[i, h] = (p / p.sum()) @ v[lo:pos + 1, kv_map(h)]
    return out.reshape(c.t, -1)


@pytest.mark.parametrize("mistake", ["kv_map", "scale", "window"])
def test_planted_mistake_is_detected(mistake):
    c = AttnCase(13, t=4, H=8, Hkv=2, hd=16, n_pos=24)
    base, w = 20, 6
    got = c.reference(base_pos=base, window=w)
    honest = _textbook_variant(c, base, w)
    assert np.max(np.abs(got - honest)) < 2e-6
    bad = {
        "kv_map": dict(kv_map=lambda h: h % 2),
        "scale": dict(scale=1.0),
        "window": dict(lo_shift=-1),
    }[mistake]
    assert np.max(np.abs(got - _textbook_variant(c, base, w, **bad))) > 1e-2
