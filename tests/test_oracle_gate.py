"""Oracle for Qwen3.5's attention output gate (qwen35/cpu.rs:359-363 with
ops::sigmoid, ops.rs:181-183): special values, a float64 restatement and a
planted sign mistake.  Test infrastructure only."""
import numpy as np

import oracle
from oracle import textbook


def test_zero_gate_halves_the_output():
    out = oracle.normal(1, (3, 64))
    got = oracle.attn_gate(out, np.zeros(3 * 64, np.float32), dim=64)
    np.testing.assert_array_equal(got, out * np.float32(0.5))


def test_large_gates_pass_or_zero_the_output():
    out = oracle.normal(2, (2, 16))
    g = np.concatenate([np.full(16, 40.0), np.full(16, -200.0)]).astype(np.float32)
    got = oracle.attn_gate(out, g, dim=16)
    np.testing.assert_array_equal(got[0], out[0])       # sigmoid(40) rounds to 1 in f32
    np.testing.assert_array_equal(got[1], np.zeros(16))  # exp(200) overflows: 1/inf = 0


def test_gate_matches_float64_with_a_stride():
    # the fused layout: per head [query | gate], the gate at offset hd, stride 2*hd
    rows, hd = 12, 128
    fused = oracle.normal(3, (rows, 2 * hd))
    out = oracle.normal(4, (rows, hd))
    got = oracle.attn_gate(out, fused.reshape(-1)[hd:], dim=hd, gate_stride=2 * hd)
    ref = textbook.attn_gate(out, fused.reshape(-1)[hd:], dim=hd, gate_stride=2 * hd)
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-6)


def test_planted_sign_mistake_is_detected():
    out = oracle.normal(5, (4, 32))
    g = oracle.normal(6, (4 * 32,))
    wrong = textbook.attn_gate(out, -g, dim=32)
    assert np.abs(oracle.attn_gate(out, g, dim=32) - wrong).max() > 1e-2
