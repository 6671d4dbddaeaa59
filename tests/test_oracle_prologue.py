"""Oracle for the attention prologue (per-head RMS norm, NeoX RoPE, f16 store):
the reference's known-answer tests, a float64 restatement, and planted mistakes.
Test infrastructure only."""
import numpy as np
import pytest

import oracle
from oracle import textbook

# Shapes of the models whose prologue this covers (q_stride > head_dim is the
# qwen35 [query | gate] head; factors with 1e30 entries are Gemma's partial
# rope on global layers).
CONFIGS = {
    "qwen3": dict(n_heads=8, n_kv_heads=2, head_dim=128, n_rot=128, rope_base=1e6, q_stride=128),
    "qwen35": dict(n_heads=6, n_kv_heads=1, head_dim=256, n_rot=64, rope_base=1e7, q_stride=512),
    "gemma_swa": dict(n_heads=4, n_kv_heads=2, head_dim=256, n_rot=256, rope_base=1e4, q_stride=256,
                      v_norm=True, window=16),
    "gemma_global": dict(n_heads=4, n_kv_heads=1, head_dim=256, n_rot=256, rope_base=1e6, q_stride=256,
                         v_norm=True, factors=True),
    # the smallest and largest head sizes the path takes, with partial rope on the latter
    "hd64": dict(n_heads=4, n_kv_heads=2, head_dim=64, n_rot=64, rope_base=1e4, q_stride=64),
    "hd512_partial": dict(n_heads=2, n_kv_heads=1, head_dim=512, n_rot=128, rope_base=1e6, q_stride=512),
    # more rows a wave than one register batch holds (the GPU kernel loads a
    # wave's rows in batches of 24 / (head_dim / 64)): two or more batches
    "many_heads_hd64": dict(n_heads=64, n_kv_heads=32, head_dim=64, n_rot=64, rope_base=1e4, q_stride=64),
    "many_heads_hd128": dict(n_heads=40, n_kv_heads=8, head_dim=128, n_rot=128, rope_base=1e6, q_stride=128),
    "gemma_c4": dict(n_heads=16, n_kv_heads=8, head_dim=256, n_rot=256, rope_base=1e4, q_stride=256,
                     v_norm=True),
    "gemma4_global": dict(n_heads=16, n_kv_heads=1, head_dim=512, n_rot=128, rope_base=1e6, q_stride=512,
                          v_norm=True),
}


def make(cfg_name, t=5, base_pos=37, seed=3):
    c = dict(CONFIGS[cfg_name])
    factors = None
    if c.pop("factors", False):
        half = c["n_rot"] // 2
        factors = np.ones(half, np.float32)
        factors[half // 2:] = 1e30  # the upper half of the pairs stays unrotated
    window = c.pop("window", 0)
    H, Hkv, hd, qs = c["n_heads"], c["n_kv_heads"], c["head_dim"], c["q_stride"]
    q = oracle.normal(seed * 10 + 1, (t, H * qs)) * np.float32(2.0)
    k = oracle.normal(seed * 10 + 2, (t, Hkv * hd))
    v = oracle.normal(seed * 10 + 3, (t, Hkv * hd)) * np.float32(0.5)
    qg = (1.0 + 0.1 * oracle.normal(seed * 10 + 4, (hd,))).astype(np.float32)
    kg = (1.0 + 0.1 * oracle.normal(seed * 10 + 5, (hd,))).astype(np.float32)
    kw = dict(c, base_pos=base_pos, q_gain=qg, k_gain=kg, rope_factors=factors)
    return q, k, v, kw, window


# ---------------------------------------------------------- reference KATs --
def test_rope_at_position_zero_is_identity():  # ops.rs:226-233
    h = np.array([0.5, -1.5, 2.0, 0.25], np.float32)
    np.testing.assert_allclose(oracle.rope_neox(h, 0, 10_000.0, [1.0, 1.0]), h, atol=1e-6)


def test_rope_sentinel_factor_disables_rotation():  # ops.rs:236-244
    h = np.array([0.5, -1.5, 2.0, 0.25], np.float32)
    np.testing.assert_allclose(oracle.rope_neox(h, 137, 10_000.0, [1e30, 1e30]), h, atol=1e-6)


def test_rope_pairs_across_the_half_boundary():  # ops.rs:247-257
    h = (np.arange(8) - 3.5).astype(np.float32)
    r = oracle.rope_neox(h, 3, 10_000.0, [1.0] * 4)
    for i in range(4):
        assert abs(np.hypot(h[i], h[i + 4]) - np.hypot(r[i], r[i + 4])) < 1e-5


def test_rms_norm_gives_unit_rms():  # ops.rs:218-223
    x = np.array([[1.0, 2.0, 3.0, 4.0]], np.float32)
    oracle.lib().orc_rms_norm_rows(oracle._f32p(x), 1, 4, 0.0)
    assert abs(np.sqrt(np.mean(x.astype(np.float64) ** 2)) - 1.0) < 1e-6


# ------------------------------------------------------- float64 restatement --
@pytest.mark.parametrize("pos", [0, 1, 5, 4095, 32767])
def test_rope_matches_closed_form(pos):
    h = oracle.normal(pos + 11, (128,))
    got = oracle.rope_neox(h, pos, 1e6)
    ref = textbook.rope_neox(h, pos, 1e6)
    np.testing.assert_allclose(got, ref, atol=2e-6 * max(1.0, float(np.abs(h).max())))


@pytest.mark.parametrize("cfg", sorted(CONFIGS))
def test_prologue_matches_float64(cfg):
    q, k, v, kw, window = make(cfg)
    n_slots = window or 64
    qo, kc, vc = oracle.attn_prologue(q, k, v, n_slots=n_slots, window=window, **kw)
    qr, kr, vr = textbook.attn_prologue(q, k, v, **kw)
    np.testing.assert_allclose(qo, qr, rtol=0, atol=2e-5 * float(np.abs(qr).max()))
    t = q.shape[0]
    slots = [oracle.slot(kw["base_pos"] + i, window) for i in range(t)]
    for i, s in enumerate(slots):
        # the f16 rows hold the float64 values to within one f16 rounding
        for got, ref in ((kc[s], kr[i]), (vc[s], vr[i])):
            g = oracle.from_f16_bits(got).astype(np.float64)
            assert np.all(np.abs(g - ref) <= np.abs(ref) * 2.0 ** -10 + 2.0 ** -24)


def test_prologue_leaves_gate_half_untouched():
    q, k, v, kw, window = make("qwen35")
    qo, _, _ = oracle.attn_prologue(q, k, v, n_slots=64, **kw)
    qs, hd = kw["q_stride"], kw["head_dim"]
    np.testing.assert_array_equal(qo.reshape(-1, qs)[:, hd:], q.reshape(-1, qs)[:, hd:])


def test_prologue_rows_have_unit_rms_before_gain_and_rotation():
    q, k, v, kw, _ = make("gemma_swa")
    kw = dict(kw, q_gain=np.ones(kw["head_dim"], np.float32), n_rot=0)
    qo, _, vc = oracle.attn_prologue(q, k, v, n_slots=64, **kw)
    rms = np.sqrt(np.mean(qo.reshape(-1, kw["head_dim"]).astype(np.float64) ** 2, axis=1))
    np.testing.assert_allclose(rms, 1.0, atol=1e-5)


# ------------------------------------------------------------ planted mistakes --
def _neighbour_pair_rope(head, pos, base):
    """A plausible mistake: rotating adjacent pairs (2i, 2i+1) instead of NeoX's (i, i+d/2)."""
    h = np.asarray(head, np.float64).copy()
    d = h.size
    for i in range(d // 2):
        a = pos * base ** (-2.0 * i / d)
        x0, x1 = h[2 * i], h[2 * i + 1]
        h[2 * i], h[2 * i + 1] = x0 * np.cos(a) - x1 * np.sin(a), x0 * np.sin(a) + x1 * np.cos(a)
    return h


def test_planted_pairing_mistake_is_detected():
    h = oracle.normal(5, (128,))
    assert np.abs(_neighbour_pair_rope(h, 17, 1e6) - oracle.rope_neox(h, 17, 1e6)).max() > 1e-2


def test_planted_partial_rope_frequency_mistake_is_detected():
    # qwen35 rotates 64 of 256 dims with theta_scale = base^(-2/64), not base^(-2/256)
    h = oracle.normal(6, (64,))
    wrong = textbook.rope_neox(np.concatenate([h, np.zeros(192, np.float32)]), 9, 1e7)[:64]
    assert np.abs(wrong - oracle.rope_neox(h, 9, 1e7)).max() > 1e-2
