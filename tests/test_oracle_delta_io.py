"""Oracle for the delta-net front (causal conv + SiLU, window shift, q/k L2
norm; qwen35/cpu.rs:193-216) and back (gated RMS norm; qwen35/cpu.rs:250-259):
a float64 restatement, invariants and a planted mistake.  Test infrastructure only."""
import numpy as np
import pytest

import oracle
from oracle import textbook

C5 = dict(conv_dim=8192, key_dim=2048, s_dim=128, kernel=4)
TINY = dict(conv_dim=256, key_dim=64, s_dim=64, kernel=4)


def front_inputs(shape, t, seed):
    cd, k = shape["conv_dim"], shape["kernel"]
    x = oracle.normal(seed * 10 + 1, (t, cd))
    taps = (0.5 * oracle.normal(seed * 10 + 2, (cd, k))).astype(np.float32)
    state = oracle.normal(seed * 10 + 3, (k - 1, cd))
    return x, taps, state


@pytest.mark.parametrize("shape", [TINY, C5], ids=["tiny", "c5"])
@pytest.mark.parametrize("t", [1, 2, 3, 17])
def test_front_matches_float64(shape, t):
    x, taps, state = front_inputs(shape, t, t)
    kw = dict(key_dim=shape["key_dim"], s_dim=shape["s_dim"])
    out, st = oracle.delta_front(x, taps, state, **kw)
    ref, st_ref = textbook.delta_front(x, taps, state, **kw)
    np.testing.assert_allclose(out, ref, rtol=0, atol=2e-6)
    np.testing.assert_array_equal(st, st_ref.astype(np.float32))


def test_front_identity_taps_give_silu_then_norm():
    x, taps, state = front_inputs(TINY, 5, 1)
    taps = np.zeros_like(taps)
    taps[:, -1] = 1.0  # only the current row
    out, _ = oracle.delta_front(x, taps, state, key_dim=TINY["key_dim"], s_dim=TINY["s_dim"])
    silu = x / (1.0 + np.exp(-x.astype(np.float64)))
    np.testing.assert_allclose(out[:, 2 * TINY["key_dim"]:], silu[:, 2 * TINY["key_dim"]:], atol=1e-6)
    qk = out[:, :2 * TINY["key_dim"]].reshape(5, -1, TINY["s_dim"]).astype(np.float64)
    np.testing.assert_allclose(np.sqrt((qk * qk).sum(-1)), 1.0, atol=1e-5)


@pytest.mark.parametrize("split", [1, 2, 3, 6])
def test_front_two_calls_equal_one(split):
    """The conv window carries the state across calls: a batch cut in two
    gives the same output and final window as the whole batch."""
    x, taps, state = front_inputs(TINY, 9, 2)
    kw = dict(key_dim=TINY["key_dim"], s_dim=TINY["s_dim"])
    whole, st_whole = oracle.delta_front(x, taps, state, **kw)
    a, st_a = oracle.delta_front(x[:split], taps, state, **kw)
    b, st_b = oracle.delta_front(x[split:], taps, st_a, **kw)
    np.testing.assert_array_equal(np.concatenate([a, b]), whole)
    np.testing.assert_array_equal(st_b, st_whole)


def test_planted_window_order_mistake_is_detected():
    """Reading the window newest-first (a plausible index slip) changes the output."""
    x, taps, state = front_inputs(TINY, 3, 3)
    kw = dict(key_dim=TINY["key_dim"], s_dim=TINY["s_dim"])
    out, _ = oracle.delta_front(x, taps, state, **kw)
    wrong, _ = textbook.delta_front(x, taps[:, [2, 1, 0, 3]], state, **kw)
    assert np.abs(out - wrong).max() > 1e-3


@pytest.mark.parametrize("s_dim", [64, 128, 256])
def test_back_matches_float64(s_dim):
    n_vh, t = 4, 6
    o = oracle.normal(s_dim + 1, (t, n_vh * s_dim))
    z = oracle.normal(s_dim + 2, (t, n_vh * s_dim))
    w = (1.0 + 0.2 * oracle.normal(s_dim + 3, (s_dim,))).astype(np.float32)
    got = oracle.delta_back(o, z, w, n_vh=n_vh, s_dim=s_dim)
    ref = textbook.delta_back(o, z, w, n_vh=n_vh, s_dim=s_dim)
    np.testing.assert_allclose(got, ref, rtol=0, atol=2e-6 * float(np.abs(ref).max()))


@pytest.mark.parametrize("s_dim", [64, 128, 256])
def test_back_matches_torch_rms_norm_and_silu(s_dim):
    """Library special case: per (token, v-head) row, torch's own
    ``F.rms_norm(o, (s_dim,), w, eps)`` times ``F.silu(z)`` in float64 is
    qwen35/cpu.rs:250-259 with ops.rs:40-47 (eps inside the root)."""
    torch = pytest.importorskip("torch")
    F = torch.nn.functional
    n_vh, t, eps = 3, 5, 1e-6
    o = oracle.normal(s_dim + 11, (t, n_vh * s_dim))
    z = oracle.normal(s_dim + 12, (t, n_vh * s_dim))
    w = (1.0 + 0.3 * oracle.normal(s_dim + 13, (s_dim,))).astype(np.float32)
    got = oracle.delta_back(o, z, w, n_vh=n_vh, s_dim=s_dim, eps=eps)
    to = torch.from_numpy(o.astype(np.float64)).view(t, n_vh, s_dim)
    tz = torch.from_numpy(z.astype(np.float64)).view(t, n_vh, s_dim)
    ref = F.rms_norm(to, (s_dim,), torch.from_numpy(w.astype(np.float64)), eps) * F.silu(tz)
    ref = ref.reshape(t, n_vh * s_dim).numpy()
    np.testing.assert_allclose(got, ref, rtol=0, atol=4e-6 * float(np.abs(ref).max()))


def test_back_invariants():
    """With unit weight and z large (silu(z) = z up to e^-z), each output row
    is o / rms(o) * z: a row of unit RMS comes out unit RMS once z is divided
    out, whatever its scale; a constant row of c gives sign(c) * z."""
    s_dim, n_vh = 128, 2
    rng = np.random.default_rng(5)
    o = rng.standard_normal((1, n_vh * s_dim)).astype(np.float32) * np.float32(37.0)
    z = np.full((1, n_vh * s_dim), 40.0, np.float32)
    w = np.ones(s_dim, np.float32)
    got = oracle.delta_back(o, z, w, n_vh=n_vh, s_dim=s_dim, eps=0.0) / 40.0
    for h in range(n_vh):
        row = got[0, h * s_dim:(h + 1) * s_dim].astype(np.float64)
        assert abs(np.sqrt(np.mean(row * row)) - 1.0) < 1e-6
    c = np.full((1, n_vh * s_dim), -2.5, np.float32)
    got = oracle.delta_back(c, z, w, n_vh=n_vh, s_dim=s_dim, eps=0.0)
    np.testing.assert_allclose(got, -40.0, rtol=1e-6)


def test_back_planted_mistake_is_detected():
    """eps outside the root, or the gate's sigmoid in place of silu: both fail
    the torch special case."""
    torch = pytest.importorskip("torch")
    F = torch.nn.functional
    s_dim, n_vh, t = 64, 2, 3
    o = oracle.normal(91, (t, n_vh * s_dim)) * np.float32(1e-3)
    z = oracle.normal(92, (t, n_vh * s_dim))
    w = np.ones(s_dim, np.float32)
    to = torch.from_numpy(o.astype(np.float64)).view(t, n_vh, s_dim)
    tz = torch.from_numpy(z.astype(np.float64)).view(t, n_vh, s_dim)
    ref = (F.rms_norm(to, (s_dim,), None, 1e-6) * F.silu(tz)).reshape(t, -1).numpy()
    rms = np.sqrt((o.reshape(t, n_vh, s_dim).astype(np.float64) ** 2).mean(-1, keepdims=True))
    eps_outside = (o.reshape(t, n_vh, s_dim) / (rms + 1e-6)).reshape(t, -1) * \
        (z / (1 + np.exp(-z)))
    sig_gate = (o.reshape(t, n_vh, s_dim) / np.sqrt(rms ** 2 + 1e-6)).reshape(t, -1) / (1 + np.exp(-z))
    got = oracle.delta_back(o, z, w, n_vh=n_vh, s_dim=s_dim, eps=1e-6)
    assert np.abs(got - ref).max() < 1e-5 * np.abs(ref).max()
    assert np.abs(eps_outside - ref).max() > 1e-3 * np.abs(ref).max()
    assert np.abs(sig_gate - ref).max() > 1e-2 * np.abs(ref).max()
