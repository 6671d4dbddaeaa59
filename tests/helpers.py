"""Shared input generation and tolerance checks for the parity tests.

Inputs come from the oracle's seeded xorshift64* generator (the reference's
sample.rs:73-92 recipe) so the GPU and the oracle see identical bits.
"""
from __future__ import annotations

import os

import numpy as np

import oracle

# Tolerances from the path's contract: max abs error and max|diff|/max|ref| on
# fp32 outputs (the reference's own relative form, bisect_qwen35.rs:66-88).
ABS_TOL = 2e-3
REL_TOL = 1e-2

CPU_THREADS = min(8, os.cpu_count() or 1)


def compare(got, ref, abs_tol=ABS_TOL, rel_tol=REL_TOL):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), "non-finite output"
    diff = np.abs(got - ref)
    max_abs = float(diff.max()) if diff.size else 0.0
    scale = float(np.abs(ref).max()) if ref.size else 0.0
    rel = max_abs / scale if scale > 0 else max_abs
    return max_abs, rel


def assert_close(got, ref, abs_tol=ABS_TOL, rel_tol=REL_TOL, what=""):
    max_abs, rel = compare(got, ref)
    assert max_abs <= abs_tol and rel <= rel_tol, (
        f"{what}: max_abs={max_abs:.3e} (tol {abs_tol}), rel={rel:.3e} (tol {rel_tol})")
    return max_abs, rel


class AttnCase:
    """Seeded attention inputs.  K/V hold one row per absolute position."""

    def __init__(self, seed, *, t, H, Hkv, hd, n_pos, q_f16=False, qk_norm=False, kv_dim=None):
        self.t, self.H, self.Hkv, self.hd, self.n_pos = t, H, Hkv, hd, n_pos
        self.kv_dim = kv_dim or Hkv * hd
        q = oracle.normal(seed * 10 + 1, (t, H * hd))
        k = oracle.normal(seed * 10 + 2, (n_pos, self.kv_dim))
        v = oracle.normal(seed * 10 + 3, (n_pos, self.kv_dim))
        if qk_norm:  # per-head RMS norm without gain (ops.rs:40-47)
            q = oracle.rms_norm_rows(q, hd).reshape(q.shape)
            k = oracle.rms_norm_rows(k, hd).reshape(k.shape)
        if q_f16:
            q = oracle.round_f16(q)
        self.q = np.ascontiguousarray(q, np.float32)
        self.q_f16 = q_f16
        self.k16 = oracle.to_f16_bits(k)
        self.v16 = oracle.to_f16_bits(v)
        self.kf = oracle.from_f16_bits(self.k16)
        self.vf = oracle.from_f16_bits(self.v16)

    def reference(self, *, base_pos, window=0, bidi=False, scale=None, threads=CPU_THREADS):
        return oracle.attention(self.q, self.kf, self.vf, n_heads=self.H, n_kv_heads=self.Hkv,
                                head_dim=self.hd, base_pos=base_pos, window=window, bidi=bidi,
                                scale=scale, linear=True, n_threads=threads, kv_dim=self.kv_dim)

    def ring(self, window, upto):
        """The ring cache after storing positions [0, upto) in order."""
        cache_k = np.zeros((window, self.kv_dim), np.uint16)
        cache_v = np.zeros((window, self.kv_dim), np.uint16)
        lo = max(0, upto - window)
        for p in range(lo, upto):
            cache_k[p % window] = self.k16[p]
            cache_v[p % window] = self.v16[p]
        return cache_k, cache_v


def delta_inputs(seed, *, T, n_vh, n_kh, sd, s0_scale=0.0, eps=1e-6):
    """Gated delta-net inputs per the C5 recipe: q, k L2-normalized N(0,1),
    v ~ N(0,1), alpha ~ N(0,1) with ssm_a = -1 and dt = 0 (g = exp(-softplus)),
    beta_raw ~ N(0,1)."""
    key_dim = n_kh * sd
    conv = oracle.normal(seed * 10 + 1, (T, 2 * key_dim + n_vh * sd))
    qk = oracle.l2_norm_rows(np.ascontiguousarray(conv[:, :2 * key_dim]), sd, eps)
    conv[:, :2 * key_dim] = qk.reshape(T, 2 * key_dim)
    alpha = oracle.normal(seed * 10 + 2, (T, n_vh))
    beta = oracle.normal(seed * 10 + 3, (T, n_vh))
    S0 = (oracle.normal(seed * 10 + 4, (n_vh * sd * sd,)) * np.float32(s0_scale)).astype(np.float32)
    ssm_a = np.full(n_vh, -1.0, np.float32)
    dt = np.zeros(n_vh, np.float32)
    return np.ascontiguousarray(conv), alpha, beta, S0, ssm_a, dt
