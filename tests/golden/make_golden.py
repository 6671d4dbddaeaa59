#!/usr/bin/env python3
"""Write the golden fixtures under tests/golden/ (run from the repo root).

Every fixture is an output of the C oracle (oracle/lmx_oracle.c) that has first
been checked here against the independent float64 restatement in
oracle/textbook.py, so a fixture is pinned by two implementations of the
reference's loops (cpu.rs:342-387, qwen35/cpu.rs:218-245).

Inputs come from the oracle's seeded xorshift64* generator (sample.rs:73-92).
Small fixtures store their inputs.  The larger ones store the seed, the shape
and a SHA-256 of the generated input bytes, so a test regenerates the inputs,
checks that they are the same bits, and compares against the stored outputs.

  attn_tiny.npz        hd in {8, 16} x {causal, window 4, bidi, window 4 + bidi},
                       t=5 tokens at base_pos 3, H=4, Hkv=2 (inputs stored)
  attn_c1.npz          C1: H=16, Hkv=8, hd=128, query at pos 511 over 512 keys
                       (seed + digest + out [16*128])
  delta_tiny.npz       d=8, Hk=2, Hv=4, T=37, S0 != 0 (inputs stored); also the
                       chunked form at chunk 8 equals the recurrence
  delta_c5_slice.npz   C5 head slice: d=128, Hk=Hv=1, T=256 (seed + digest + o, S)
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

import oracle  # noqa: E402
from oracle import textbook  # noqa: E402
from helpers import AttnCase, delta_inputs  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))

ATTN_TINY_MODES = [(0, False), (4, False), (0, True), (4, True)]  # (window, bidi)
C1 = dict(seed=101, H=16, Hkv=8, hd=128, n_pos=512, base_pos=511)
DELTA_TINY = dict(seed=7, T=37, n_vh=4, n_kh=2, sd=8, s0_scale=0.3)
DELTA_C5 = dict(seed=55, T=256, n_vh=1, n_kh=1, sd=128, s0_scale=0.0)


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def attn_c1_inputs():
    c = AttnCase(C1["seed"], t=1, H=C1["H"], Hkv=C1["Hkv"], hd=C1["hd"], n_pos=C1["n_pos"])
    return c


def delta_c5_inputs():
    d = DELTA_C5
    return delta_inputs(d["seed"], T=d["T"], n_vh=d["n_vh"], n_kh=d["n_kh"], sd=d["sd"],
                        s0_scale=d["s0_scale"])


def _check(got, ref, tol, what):
    err = float(np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64)).max())
    if err > tol:
        raise SystemExit(f"{what}: oracle and float64 textbook differ by {err:.3e} (> {tol})")


def main():
    # ---- attention, tiny shapes, every mask mode
    arrays = {}
    for hd in (8, 16):
        for window, bidi in ATTN_TINY_MODES:
            c = AttnCase(1000 + hd * 10 + window + 2 * bidi, t=5, H=4, Hkv=2, hd=hd, n_pos=8)
            out = c.reference(base_pos=3, window=window, bidi=bidi, threads=1)
            ref = textbook.attention(c.q, c.kf, c.vf, n_heads=4, n_kv_heads=2, head_dim=hd,
                                     base_pos=3, window=window, bidi=bidi)
            _check(out, ref, 1e-5, f"attn hd={hd} w={window} bidi={bidi}")
            key = f"hd{hd}_w{window}_b{int(bidi)}"
            arrays[key + "_q"] = c.q
            arrays[key + "_k16"] = c.k16
            arrays[key + "_v16"] = c.v16
            arrays[key + "_out"] = out
    np.savez_compressed(os.path.join(HERE, "attn_tiny.npz"), **arrays)

    # ---- attention C1
    c = attn_c1_inputs()
    out = c.reference(base_pos=C1["base_pos"], threads=1)
    ref = textbook.attention(c.q, c.kf, c.vf, n_heads=C1["H"], n_kv_heads=C1["Hkv"],
                             head_dim=C1["hd"], base_pos=C1["base_pos"])
    _check(out, ref, 1e-5, "attn C1")
    np.savez_compressed(os.path.join(HERE, "attn_c1.npz"),
                        config=np.array([C1[k] for k in ("seed", "H", "Hkv", "hd", "n_pos", "base_pos")]),
                        input_sha256=np.array(digest(c.q, c.k16, c.v16)), out=out)

    # ---- delta rule, tiny shape (inputs stored)
    d = DELTA_TINY
    conv, al, be, S0, A, dt = delta_inputs(d["seed"], T=d["T"], n_vh=d["n_vh"], n_kh=d["n_kh"],
                                           sd=d["sd"], s0_scale=d["s0_scale"])
    kw = dict(n_vh=d["n_vh"], n_kh=d["n_kh"], s_dim=d["sd"])
    o, S = oracle.delta_recur(conv, al, be, S0, **kw)
    o_ref, S_ref = textbook.delta_recur(conv, al, be, S0, **kw)
    _check(o, o_ref, 1e-5, "delta tiny o")
    _check(S, S_ref, 1e-5, "delta tiny S")
    o_ch, S_ch = textbook.delta_chunked(conv, al, be, S0, chunk=8, **kw)
    _check(o_ch, o, 1e-5, "delta tiny chunked o")
    _check(S_ch, S, 1e-5, "delta tiny chunked S")
    np.savez_compressed(os.path.join(HERE, "delta_tiny.npz"), conv=conv, alpha=al, beta=be,
                        S0=S0, ssm_a=A, dt_bias=dt, o=o, S=S,
                        config=np.array([d["T"], d["n_vh"], d["n_kh"], d["sd"]]))

    # ---- delta rule, C5 head slice
    d = DELTA_C5
    conv, al, be, S0, A, dt = delta_c5_inputs()
    kw = dict(n_vh=d["n_vh"], n_kh=d["n_kh"], s_dim=d["sd"])
    o, S = oracle.delta_recur(conv, al, be, S0, **kw)
    o_ref, S_ref = textbook.delta_recur(conv, al, be, S0, **kw)
    _check(o, o_ref, 1e-5, "delta C5 o")
    _check(S, S_ref, 1e-5, "delta C5 S")
    np.savez_compressed(os.path.join(HERE, "delta_c5_slice.npz"),
                        config=np.array([d["seed"], d["T"], d["n_vh"], d["n_kh"], d["sd"]]),
                        input_sha256=np.array(digest(conv, al, be, S0)), o=o, S=S)
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
