"""The oracle against the committed golden fixtures (tests/golden/, written by
tests/golden/make_golden.py from the oracle after a float64 cross-check).

These pin the oracle itself: a change to the generator, the f16 rounding, the
mask or slot rules, or the delta-rule term order shows up here first.  The GPU
path is compared with the same fixtures in test_gpu_golden.py.
"""
import os

import numpy as np
import pytest

import oracle
from tests.golden import make_golden as mg

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(HERE, name), allow_pickle=False)


@pytest.mark.parametrize("hd", [8, 16])
@pytest.mark.parametrize("window,bidi", mg.ATTN_TINY_MODES)
def test_attn_tiny_fixture(hd, window, bidi):
    f = load("attn_tiny.npz")
    key = f"hd{hd}_w{window}_b{int(bidi)}"
    q, k16, v16 = f[key + "_q"], f[key + "_k16"], f[key + "_v16"]
    out = oracle.attention(q, oracle.from_f16_bits(k16), oracle.from_f16_bits(v16), n_heads=4,
                           n_kv_heads=2, head_dim=hd, base_pos=3, window=window, bidi=bidi)
    np.testing.assert_allclose(out, f[key + "_out"], rtol=0, atol=1e-6)


def test_attn_c1_fixture_regenerates_and_matches():
    f = load("attn_c1.npz")
    c = mg.attn_c1_inputs()
    assert mg.digest(c.q, c.k16, c.v16) == str(f["input_sha256"]), "generator changed"
    out = c.reference(base_pos=mg.C1["base_pos"], threads=1)
    np.testing.assert_allclose(out, f["out"], rtol=0, atol=1e-6)


def test_delta_tiny_fixture():
    f = load("delta_tiny.npz")
    T, n_vh, n_kh, sd = (int(x) for x in f["config"])
    o, S = oracle.delta_recur(f["conv"], f["alpha"], f["beta"], f["S0"], n_vh=n_vh, n_kh=n_kh,
                              s_dim=sd, ssm_a=f["ssm_a"], dt_bias=f["dt_bias"])
    np.testing.assert_allclose(o, f["o"], rtol=0, atol=1e-6)
    np.testing.assert_allclose(S, f["S"], rtol=0, atol=1e-6)


def test_delta_c5_slice_fixture_regenerates_and_matches():
    f = load("delta_c5_slice.npz")
    conv, al, be, S0, A, dt = mg.delta_c5_inputs()
    assert mg.digest(conv, al, be, S0) == str(f["input_sha256"]), "generator changed"
    d = mg.DELTA_C5
    o, S = oracle.delta_recur(conv, al, be, S0, n_vh=d["n_vh"], n_kh=d["n_kh"], s_dim=d["sd"])
    np.testing.assert_allclose(o, f["o"], rtol=0, atol=1e-6)
    np.testing.assert_allclose(S, f["S"], rtol=0, atol=1e-6)
