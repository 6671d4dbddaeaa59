"""Pins the C delta-rule oracle (qwen35/cpu.rs:218-245).

Checks: the float64 matrix recurrence S <- g S (I - b k k^T) + b v k^T, the
float64 chunked (WY/UT) form (which the chunked kernel implements), closed-form
invariants, and a planted mistake (k-head mapping) that the checks catch.
"""
import numpy as np
import pytest

import oracle
import oracle.textbook as tb
from tests.helpers import delta_inputs

SHAPES = [(4, 2, 8, 37), (2, 2, 16, 20), (6, 3, 8, 9)]


@pytest.mark.parametrize("n_vh,n_kh,sd,T", SHAPES)
def test_oracle_matches_float64_recurrence(n_vh, n_kh, sd, T):
    conv, al, be, S0, A, dt = delta_inputs(3, T=T, n_vh=n_vh, n_kh=n_kh, sd=sd, s0_scale=0.5)
    o, S = oracle.delta_recur(conv, al, be, S0, n_vh=n_vh, n_kh=n_kh, s_dim=sd)
    o2, S2 = tb.delta_recur(conv, al, be, S0, n_vh=n_vh, n_kh=n_kh, s_dim=sd)
    assert np.max(np.abs(o - o2)) < 1e-5 and np.max(np.abs(S - S2)) < 1e-5


@pytest.mark.parametrize("chunk", [1, 4, 8, 16])
def test_chunked_form_equals_recurrence(chunk):
    conv, al, be, S0, A, dt = delta_inputs(4, T=37, n_vh=4, n_kh=2, sd=8, s0_scale=0.5)
    o2, S2 = tb.delta_recur(conv, al, be, S0, n_vh=4, n_kh=2, s_dim=8)
    o3, S3 = tb.delta_chunked(conv, al, be, S0, n_vh=4, n_kh=2, s_dim=8, chunk=chunk)
    assert np.max(np.abs(o2 - o3)) < 1e-12 and np.max(np.abs(S2 - S3)) < 1e-12


def test_gates_follow_softplus_and_sigmoid():
    # g = exp(a * softplus(alpha + dt)) with the x > 20 shortcut (ops.rs:187-193)
    g, b = tb.gates(np.array([[0.0, 25.0]]), np.array([[0.0, 2.0]]), np.array([-1.0, -1.0]),
                    np.array([0.0, 0.0]))
    assert abs(g[0, 0] - 0.5) < 1e-15 and abs(g[0, 1] - np.exp(-25.0)) < 1e-20
    assert abs(b[0, 0] - 0.5) < 1e-15 and abs(b[0, 1] - 1 / (1 + np.exp(-2.0))) < 1e-15


def _one_token(k, q, v, S0, alpha, beta, sd=8):
    conv = np.concatenate([q, k, v]).astype(np.float32)[None]
    return oracle.delta_recur(conv, np.array([[alpha]], np.float32), np.array([[beta]], np.float32),
                              S0.astype(np.float32), n_vh=1, n_kh=1, s_dim=sd)


def test_exact_write_with_unit_key():
    """g = 1 and b = 1 make the update an exact write: S k = v afterwards."""
    sd = 8
    k = np.zeros(sd, np.float32)
    k[3] = 1.0
    v = np.arange(sd, dtype=np.float32) - 2.5
    S0 = oracle.normal(5, (sd * sd,))
    # alpha = -inf-ish makes softplus -> 0 so g = 1; beta large makes b = 1.
    out, S = _one_token(k, k, v, S0, alpha=-200.0, beta=200.0)
    S = S.reshape(sd, sd)
    assert np.max(np.abs(S @ k - v)) < 1e-6
    assert np.max(np.abs(out[0] - v / np.sqrt(sd))) < 1e-6


def test_beta_zero_is_pure_decay():
    sd = 8
    S0 = oracle.normal(6, (sd * sd,))
    k = oracle.l2_norm_rows(oracle.normal(7, (sd,)), sd)
    v = oracle.normal(8, (sd,))
    _, S = _one_token(k, k, v, S0, alpha=0.3, beta=-200.0)
    g = np.exp(-np.log1p(np.exp(0.3)))
    assert np.max(np.abs(S - g * S0)) < 1e-6


def test_linear_in_values_from_zero_state():
    conv, al, be, S0, A, dt = delta_inputs(9, T=11, n_vh=2, n_kh=1, sd=8)
    key_dim = 8
    o1, S1 = oracle.delta_recur(conv, al, be, S0, n_vh=2, n_kh=1, s_dim=8)
    conv2 = conv.copy()
    conv2[:, 2 * key_dim:] *= 3.0
    o2, S2 = oracle.delta_recur(conv2, al, be, S0, n_vh=2, n_kh=1, s_dim=8)
    assert np.max(np.abs(o2 - 3 * o1)) < 1e-5 and np.max(np.abs(S2 - 3 * S1)) < 1e-5


def test_orthonormal_keys_write_independently():
    sd = 8
    basis = np.eye(sd, dtype=np.float32)
    T = 3
    conv = np.zeros((T, 3 * sd), np.float32)
    vals = oracle.normal(10, (T, sd))
    for t in range(T):
        conv[t, :sd] = basis[t]
        conv[t, sd:2 * sd] = basis[t]
        conv[t, 2 * sd:] = vals[t]
    al = np.full((T, 1), -200.0, np.float32)  # g = 1
    be = np.full((T, 1), 200.0, np.float32)   # b = 1
    _, S = oracle.delta_recur(conv, al, be, np.zeros(sd * sd, np.float32), n_vh=1, n_kh=1, s_dim=sd)
    S = S.reshape(sd, sd)
    for t in range(T):
        assert np.max(np.abs(S @ basis[t] - vals[t])) < 1e-6


def test_planted_khead_mistake_is_detected():
    """Mapping v-heads to k-heads by hv // (n_vh/n_kh) instead of hv % n_kh
    (deltanet.wgsl:200 tiles modulo) must disagree."""
    n_vh, n_kh, sd, T = 4, 2, 8, 6
    conv, al, be, S0, A, dt = delta_inputs(11, T=T, n_vh=n_vh, n_kh=n_kh, sd=sd)
    o, _ = oracle.delta_recur(conv, al, be, S0, n_vh=n_vh, n_kh=n_kh, s_dim=sd)
    key_dim = n_kh * sd
    swapped = conv.copy()
    # reorder v-heads so that the modulo map reads what a contiguous map would
    vh = swapped[:, 2 * key_dim:].reshape(T, n_vh, sd)
    swapped[:, 2 * key_dim:] = vh[:, [0, 2, 1, 3]].reshape(T, -1)
    o_bad, _ = oracle.delta_recur(swapped, al, be, S0, n_vh=n_vh, n_kh=n_kh, s_dim=sd)
    assert np.max(np.abs(o - o_bad)) > 1e-2


def test_threaded_recurrence_is_bit_identical():
    """Splitting the independent v-heads over threads changes no value."""
    from tests.helpers import delta_inputs
    conv, al, be, S0, A, dt = delta_inputs(77, T=23, n_vh=6, n_kh=3, sd=16, s0_scale=0.3)
    o1, s1 = oracle.delta_recur(conv, al, be, S0, n_vh=6, n_kh=3, s_dim=16, n_threads=1)
    for n in (2, 4, 6, 9):
        o2, s2 = oracle.delta_recur(conv, al, be, S0, n_vh=6, n_kh=3, s_dim=16, n_threads=n)
        assert np.array_equal(o1, o2) and np.array_equal(s1, s2)
