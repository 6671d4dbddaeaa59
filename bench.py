#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path (one JSON line on stdout).

Headline (BASELINE.json metric, config C2): decode attention at Qwen3-8B shape
(H=32, Hkv=8, hd=128, f16 KV, fp32 math), batch 1, 32768-token context.  One
step is one decode-attention call for one layer; the timed steps rotate over
36 distinct layer caches (Qwen3-8B has 36 layers, 4.5 GiB of KV in all) so
the KV bytes come from HBM, not from the 256 MB last-level cache.  Inputs are
synthetic N(0,1), resident in HBM before timing starts.

Timing: HIP events recorded on the stream the kernels are launched on, around
exactly --steps calls after --warmup untimed calls, with device syncs on both
sides.  ``roofline.achieved`` = algorithmic bytes per launch / mean launch time.

Other configs (ragged batches, prefill, Gemma-shape, delta-net) are reported
under ``extra`` with their own roofline fractions; they are not the headline.
The CPU baseline is the C restatement of the reference's scalar loops
(oracle/), timed on a bounded sample on this host, 1 thread.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, 8 TB/s
MFMA_F16_PEAK_TFS = 2500.0  # MI355X dense f16 MFMA, 2.5 PFLOP/s
METRIC = "decode-attn HBM GB/s (% peak) Qwen3-8B 32k ctx; prefill-attn TFLOP/s"

H, HKV, HD = 32, 8, 128
CTX = 32768
N_LAYERS = 36


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def decode_bytes(ctx_lens, H=H, Hkv=HKV, hd=HD, q_bytes=4):
    """Algorithmic bytes of one decode call: K and V rows read once (f16) plus
    q read and out written (fp32)."""
    return sum(2 * c * Hkv * hd * 2 for c in ctx_lens) + len(ctx_lens) * H * hd * (q_bytes + 4)


def prefill_flops(pairs, H=H, hd=HD):
    """4*hd FLOPs per visible (query, key) pair per head (QK^T and PV)."""
    return 4 * hd * H * pairs


def time_calls(fns, steps, warmup, torch):
    """Mean ms per call of fns[i % len(fns)], HIP events on the current stream."""
    for i in range(warmup):
        fns[i % len(fns)]()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for i in range(steps):
        fns[i % len(fns)]()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def read_traffic(name):
    path = os.path.join(ROOT, "profiles", f"{name}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("bytes_per_launch")


# ------------------------------------------------------------------ headline --
def bench_decode_headline(lmx, torch, steps, warmup):
    n_layers = N_LAYERS
    ks = [torch.randn((CTX, HKV * HD), dtype=torch.float16, device="cuda") for _ in range(n_layers)]
    vs = [torch.randn((CTX, HKV * HD), dtype=torch.float16, device="cuda") for _ in range(n_layers)]
    qs = [torch.randn((1, H * HD), dtype=torch.float32, device="cuda") for _ in range(n_layers)]
    out = torch.empty((1, H * HD), dtype=torch.float32, device="cuda")
    ws = lmx.Workspace()
    fns = [
        (lambda i=i: lmx.attention(qs[i], ks[i], vs[i], n_heads=H, n_kv_heads=HKV, head_dim=HD,
                                   base_pos=CTX - 1, out=out, workspace=ws))
        for i in range(n_layers)
    ]
    ms = time_calls(fns, steps, warmup, torch)
    nbytes = decode_bytes([CTX])
    gbs = nbytes / (ms * 1e-3) / 1e9
    del ks, vs
    torch.cuda.empty_cache()
    return ms, gbs, nbytes


def bench_decode_c1(lmx, torch, steps=360, warmup=36):
    """C1: batch 1, H=16, Hkv=8, hd=128, 512 cached f16 tokens, fp32 q, query
    at position 511; 36 rotated layer caches.  Latency-bound: 2.1 MB a call."""
    Hq, n, n_layers = 16, 512, N_LAYERS
    ks = [torch.randn((n, HKV * HD), dtype=torch.float16, device="cuda") for _ in range(n_layers)]
    vs = [torch.randn((n, HKV * HD), dtype=torch.float16, device="cuda") for _ in range(n_layers)]
    q = torch.randn((1, Hq * HD), dtype=torch.float32, device="cuda")
    out = torch.empty((1, Hq * HD), dtype=torch.float32, device="cuda")
    ws = lmx.Workspace()
    fns = [(lambda i=i: lmx.attention(q, ks[i], vs[i], n_heads=Hq, n_kv_heads=HKV, head_dim=HD,
                                      base_pos=n - 1, out=out, workspace=ws)) for i in range(n_layers)]
    ms = time_calls(fns, steps, warmup, torch)
    nbytes = decode_bytes([n], Hq)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"ctx": n, "ms": ms, "GB/s": gbs, "frac_hbm": gbs / HBM_PEAK_GBS}


# -------------------------------------------------------------------- extras --
def bench_decode_batched(lmx, torch, B, seed, steps=20, warmup=3):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(1024, CTX + 1, (B,), generator=g).tolist()
    max_ctx = max(lens)
    sets = []
    for _ in range(2):  # two independent cache sets, alternated
        ks = [torch.randn((n, HKV * HD), dtype=torch.float16, device="cuda") for n in lens]
        vs = [torch.randn((n, HKV * HD), dtype=torch.float16, device="cuda") for n in lens]
        sets.append(lmx.BatchedCaches(ks, vs))
    q = torch.randn((B, H * HD), dtype=torch.float32, device="cuda")
    ctx = torch.tensor(lens, dtype=torch.int32, device="cuda")
    out = torch.empty((B, H * HD), dtype=torch.float32, device="cuda")
    ws = lmx.Workspace()
    fns = [(lambda s=s: lmx.attention_decode_batched(q, s, ctx, max_ctx=max_ctx, n_heads=H, n_kv_heads=HKV,
                                                     head_dim=HD, n_slots=max_ctx, out=out, workspace=ws))
           for s in sets]
    ms = time_calls(fns, steps, warmup, torch)
    nbytes = decode_bytes(lens)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"B": B, "sum_ctx": sum(lens), "ms": ms, "GB/s": gbs, "frac_hbm": gbs / HBM_PEAK_GBS,
            "tokens/s": B / (ms * 1e-3)}


def bench_prefill(lmx, torch, S, base=0, Hq=H, Hkv=HKV, hd=HD, window=0, scale=None, steps=10,
                  warmup=2):
    n_pos = base + S
    k = torch.randn((n_pos, Hkv * hd), dtype=torch.float16, device="cuda")
    v = torch.randn((n_pos, Hkv * hd), dtype=torch.float16, device="cuda")
    q = torch.randn((S, Hq * hd), dtype=torch.float16, device="cuda")
    out = torch.empty((S, Hq * hd), dtype=torch.float32, device="cuda")
    ws = lmx.Workspace()
    kw = {}
    kc, vc = k, v
    if window:
        # ring of `window` slots for positions < base, the batch's rows as k_cur
        kc = torch.randn((window, Hkv * hd), dtype=torch.float16, device="cuda")
        vc = torch.randn((window, Hkv * hd), dtype=torch.float16, device="cuda")
        kw = dict(k_cur=k[base:], v_cur=v[base:])
    fn = lambda: lmx.attention(q, kc, vc, n_heads=Hq, n_kv_heads=Hkv, head_dim=hd, base_pos=base,
                               window=window, scale=scale, out=out, workspace=ws, **kw)
    ms = time_calls([fn], steps, warmup, torch)
    pairs = 0
    for i in range(S):
        pos = base + i
        lo = max(0, pos - window + 1) if window else 0
        pairs += pos - lo + 1
    fl = prefill_flops(pairs, Hq, hd)
    tfs = fl / (ms * 1e-3) / 1e12
    return {"S": S, "base": base, "window": window, "ms": ms, "TFLOP/s": tfs,
            "frac_mfma": tfs / MFMA_F16_PEAK_TFS, "tokens/s": S / (ms * 1e-3)}


def bench_gemma_decode(lmx, torch, window, steps=50, warmup=5):
    Hq, Hkv, hd = 16, 8, 256
    slots = window or CTX
    n_layers = 8
    ks = [torch.randn((slots, Hkv * hd), dtype=torch.float16, device="cuda") for _ in range(n_layers)]
    vs = [torch.randn((slots, Hkv * hd), dtype=torch.float16, device="cuda") for _ in range(n_layers)]
    q = torch.randn((1, Hq * hd), dtype=torch.float32, device="cuda")
    out = torch.empty((1, Hq * hd), dtype=torch.float32, device="cuda")
    ws = lmx.Workspace()
    fns = [(lambda i=i: lmx.attention(q, ks[i], vs[i], n_heads=Hq, n_kv_heads=Hkv, head_dim=hd,
                                      base_pos=CTX - 1, window=window, scale=1 / 16, out=out, workspace=ws))
           for i in range(n_layers)]
    ms = time_calls(fns, steps, warmup, torch)
    nbytes = decode_bytes([min(window or CTX, CTX)], Hq, Hkv, hd)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"window": window, "ms": ms, "GB/s": gbs, "frac_hbm": gbs / HBM_PEAK_GBS}


def bench_prologue(lmx, torch, t, H=H, Hkv=HKV, hd=HD, steps=20, warmup=3):
    """Per-head RMS norm + NeoX RoPE on Q and K, and the f16 KV store, at the
    C2 shape.  Bytes: q read and written (f32), k and v read (f32), k and v
    written (f16)."""
    kv_dim = Hkv * hd
    q = torch.randn((t, H * hd), device="cuda")
    k = torch.randn((t, kv_dim), device="cuda")
    v = torch.randn((t, kv_dim), device="cuda")
    kc = torch.empty((t, kv_dim), dtype=torch.float16, device="cuda")
    vc = torch.empty_like(kc)
    qg = torch.ones(hd, device="cuda")
    kg = torch.ones(hd, device="cuda")
    fn = lambda: lmx.attn_prologue(q, k, v, kc, vc, n_heads=H, n_kv_heads=Hkv, head_dim=hd,
                                   base_pos=0, q_gain=qg, k_gain=kg)
    ms = time_calls([fn], steps, warmup, torch)
    nbytes = t * (H * hd * 8 + 2 * kv_dim * 4 + 2 * kv_dim * 2)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"t": t, "ms": ms, "GB/s": gbs, "frac_hbm": gbs / HBM_PEAK_GBS}


def bench_matvec(lmx, torch, qtype, rows, in_dim, n_mats, steps=50, warmup=5):
    """lmx_matvec at one token: y = W x over n_mats distinct weight matrices in
    turn (so W comes from HBM, as a decode step's projections do).  Bytes are
    the weight bytes (x and y are 4 * (in_dim + rows))."""
    bb, be = {"q4_k": (144, 256), "q6_k": (210, 256), "q8_0": (34, 32), "bf16": (2, 1)}[qtype]
    nbytes = rows * (in_dim // be) * bb
    ws = [torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda") for _ in range(n_mats)]
    x = torch.randn((1, in_dim), device="cuda")
    y = torch.empty((1, rows), device="cuda")
    fns = [(lambda w=w: lmx.matvec(w, x, qtype=qtype, rows=rows, in_dim=in_dim, y=y)) for w in ws]
    ms = time_calls(fns, steps, warmup, torch)
    total = nbytes + 4 * (in_dim + rows)
    gbs = total / (ms * 1e-3) / 1e9
    del ws
    return {"type": qtype, "rows": rows, "in_dim": in_dim, "weight_bytes": nbytes, "ms": ms,
            "GB/s": gbs, "frac_hbm": gbs / HBM_PEAK_GBS}


def bench_kvm(lmx, torch, which, steps=20, warmup=3):
    """KV manager.  "wipe": zeroing one Qwen3-8B sequence slab (36 layers of
    f16 K and V at 32k positions, 4.83 GB) with lmx_kvm_wipe, an HBM write.
    "batch": host time of lmx_kvm_batch for a ragged batch of 32 sequences."""
    layers = [(0, HKV * HD, -1)] * N_LAYERS
    if which == "wipe":
        m = lmx.KvManager(layers, n_ctx=CTX, max_seqs=1)
        s = m.open()
        ms = time_calls([lambda: m.wipe(s)], steps, warmup, torch)
        nbytes = m.arena_bytes
        del m
        return {"bytes": nbytes, "ms": ms, "GB/s": nbytes / (ms * 1e-3) / 1e9,
                "frac_hbm": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
    m = lmx.KvManager(layers, n_ctx=CTX, max_seqs=32, arena=(1 << 20, 1 << 48))
    seqs = [m.open() for _ in range(32)]
    for i, s in enumerate(seqs):
        m.commit(s, list(range(100 + 900 * i)))
    for _ in range(warmup):
        m.batch(0, seqs)
    t0 = time.perf_counter()
    for _ in range(steps * 50):
        m.batch(0, seqs)
    us = (time.perf_counter() - t0) / (steps * 50) * 1e6
    return {"B": 32, "host_us_per_batch_table": us}


def bench_delta_io(lmx, torch, T, which, steps=20, warmup=3):
    """Delta-net front (conv + SiLU + window + q/k L2 norm) or back (gated RMS
    norm) at C5.  Bytes: front reads x and writes conv_out (f32 [T, 8192]),
    plus taps and window; back reads o and z and writes o (f32 [T, 4096])."""
    n_vh, n_kh, sd, K = 32, 16, 128, 4
    key_dim, d_inner = n_kh * sd, n_vh * sd
    conv_dim = 2 * key_dim + d_inner
    if which == "front":
        x = torch.randn((T, conv_dim), device="cuda")
        taps = torch.randn((conv_dim, K), device="cuda")
        st = torch.zeros((K - 1, conv_dim), device="cuda")
        out = torch.empty_like(x)
        fn = lambda: lmx.delta_front(x, taps, st, out, key_dim=key_dim, s_dim=sd)
        nbytes = 2 * T * conv_dim * 4 + conv_dim * K * 4 + 2 * (K - 1) * conv_dim * 4
    else:
        o = torch.randn((T, d_inner), device="cuda")
        z = torch.randn((T, d_inner), device="cuda")
        w = torch.ones(sd, device="cuda")
        fn = lambda: lmx.delta_back(o, z, w, n_vh=n_vh, s_dim=sd)
        nbytes = 3 * T * d_inner * 4 + sd * 4
    ms = time_calls([fn], steps, warmup, torch)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"T": T, "ms": ms, "GB/s": gbs, "frac_hbm": gbs / HBM_PEAK_GBS}


def bench_delta(lmx, torch, T, chunked, steps=5, warmup=1):
    n_vh, n_kh, sd = 32, 16, 128
    conv_dim = 2 * n_kh * sd + n_vh * sd
    conv = torch.randn((T, conv_dim), dtype=torch.float32, device="cuda")
    qk = conv[:, :2 * n_kh * sd].view(T, 2 * n_kh, sd)
    qk /= qk.norm(dim=-1, keepdim=True)
    al = torch.randn((T, n_vh), device="cuda")
    be = torch.randn((T, n_vh), device="cuda")
    A = torch.full((n_vh,), -1.0, device="cuda")
    dt = torch.zeros(n_vh, device="cuda")
    state = torch.zeros((n_vh, sd, sd), device="cuda")
    out = torch.empty((T, n_vh * sd), device="cuda")
    ws = lmx.Workspace()
    if chunked:
        fn = lambda: lmx.delta_chunked(conv, al, be, state, A, dt, n_vh=n_vh, n_kh=n_kh, s_dim=sd,
                                       chunk=64, out=out, workspace=ws)
    else:
        fn = lambda: lmx.delta_recur(conv, al, be, state, A, dt, n_vh=n_vh, n_kh=n_kh, s_dim=sd, out=out)
    ms = time_calls([fn], steps, warmup, torch)
    nbytes = (conv_dim + 2 * n_vh + n_vh * sd) * 4 * T + 2 * n_vh * sd * sd * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"T": T, "chunked": chunked, "ms": ms, "GB/s": gbs, "frac_hbm": gbs / HBM_PEAK_GBS,
            "tokens/s": T / (ms * 1e-3)}


# -------------------------------------------------------------- CPU baseline --
def cpu_baseline(budget_s=12.0):
    """The C restatement of the reference's scalar attention loop (cpu.rs:342-387;
    qwen35/cpu.rs:324-365) on the headline shape, 1 thread, bounded sample."""
    import numpy as np
    import oracle

    rng = np.random.default_rng(0)
    k = rng.standard_normal((CTX, HKV * HD), dtype=np.float32).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((CTX, HKV * HD), dtype=np.float32).astype(np.float16).astype(np.float32)
    q = rng.standard_normal((1, H * HD), dtype=np.float32)
    calls, t0 = 0, time.perf_counter()
    while True:
        oracle.attention(q, k, v, n_heads=H, n_kv_heads=HKV, head_dim=HD, base_pos=CTX - 1, n_threads=1)
        calls += 1
        el = time.perf_counter() - t0
        if el >= budget_s or calls >= 50:
            break
    per = el / calls
    gbs = decode_bytes([CTX]) / per / 1e9
    return {"value": gbs, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{calls} decode-attention calls at the headline shape (B=1, ctx {CTX}, "
                      f"H={H}, Hkv={HKV}, hd={HD}), {per * 1e3:.1f} ms each, C oracle -O2, 1 thread"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--only", choices=["headline", "all"], default="all")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--extras", default="",
                    help="comma-separated names of the extra configs to run (default: all)")
    ap.add_argument("--pmc-calibration", action="store_true",
                    help="after the timed runs, copy a 256 MiB fp32 buffer 3 times: the known-size "
                         "reference that FETCH_SIZE / WRITE_SIZE counter readings are scaled by")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}): this build has no "
              "multi-GPU path; see DESIGN.md for how it would shard.", file=sys.stderr)
        sys.exit(2)

    import torch
    import llmoxide_amd as lmx

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    lmx.lib()  # fail loudly if the HIP library is missing

    log(f"headline: decode B=1 ctx {CTX}, {args.steps} steps, {args.warmup} warmup")
    ms, gbs, nbytes = bench_decode_headline(lmx, torch, args.steps, args.warmup)
    log(f"headline: {ms * 1e3:.2f} us/call, {gbs:.1f} GB/s")

    extra = {}
    if args.only == "all":
        for name, fn in [
            ("decode_c1_ctx512", lambda: bench_decode_c1(lmx, torch)),
            ("decode_b8", lambda: bench_decode_batched(lmx, torch, 8, 8)),
            ("decode_b32", lambda: bench_decode_batched(lmx, torch, 32, 32)),
            ("gemma_decode_swa_w1024", lambda: bench_gemma_decode(lmx, torch, 1024)),
            ("gemma_decode_global", lambda: bench_gemma_decode(lmx, torch, 0)),
            ("prefill_s512", lambda: bench_prefill(lmx, torch, 512, steps=50, warmup=5)),
            ("prefill_s2048", lambda: bench_prefill(lmx, torch, 2048)),
            ("prefill_s8192", lambda: bench_prefill(lmx, torch, 8192, steps=5, warmup=1)),
            ("prefill_chunk512_on_4k", lambda: bench_prefill(lmx, torch, 512, base=4096, steps=50, warmup=5)),
            ("gemma_prefill_swa_4k", lambda: bench_prefill(lmx, torch, 4096, Hq=16, Hkv=8, hd=256,
                                                           window=1024, scale=1 / 16, steps=5, warmup=1)),
            ("gemma_prefill_global_4k", lambda: bench_prefill(lmx, torch, 4096, Hq=16, Hkv=8, hd=256,
                                                              scale=1 / 16, steps=5, warmup=1)),
            ("prologue_prefill_t4096", lambda: bench_prologue(lmx, torch, 4096)),
            ("prologue_decode_t1", lambda: bench_prologue(lmx, torch, 1, steps=50, warmup=5)),
            ("delta_prefill_T4096_chunked", lambda: bench_delta(lmx, torch, 4096, True)),
            ("delta_prefill_T4096_sequential", lambda: bench_delta(lmx, torch, 4096, False)),
            ("delta_decode_1tok", lambda: bench_delta(lmx, torch, 1, False, steps=50, warmup=5)),
            ("delta_front_T4096", lambda: bench_delta_io(lmx, torch, 4096, "front")),
            ("delta_back_T4096", lambda: bench_delta_io(lmx, torch, 4096, "back")),
            ("matvec_q4k_attn_output_4096", lambda: bench_matvec(lmx, torch, "q4_k", 4096, 4096, 36)),
            ("matvec_q6k_lm_head_151936", lambda: bench_matvec(lmx, torch, "q6_k", 151936, 4096, 2, steps=20)),
            ("matvec_q4k_ffn_up_12288", lambda: bench_matvec(lmx, torch, "q4_k", 12288, 4096, 36)),
            ("matvec_q8_0_attn_output_4096", lambda: bench_matvec(lmx, torch, "q8_0", 4096, 4096, 36)),
            ("kvm_wipe_qwen3_8b_32k", lambda: bench_kvm(lmx, torch, "wipe")),
            ("kvm_batch_tables_b32", lambda: bench_kvm(lmx, torch, "batch")),
        ]:
            if args.extras and name not in args.extras.split(","):
                continue
            t0 = time.perf_counter()
            try:
                extra[name] = fn()
            except Exception as e:  # an extra failing must not hide the headline
                extra[name] = {"error": repr(e)}
            log(f"{name}: {extra[name]} ({time.perf_counter() - t0:.1f}s)")
            torch.cuda.empty_cache()

    if args.pmc_calibration:
        a = torch.empty(64 << 20, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        del a, b

    cpu = None if args.skip_cpu else cpu_baseline()
    if cpu:
        log(f"cpu baseline: {cpu}")

    line = {
        "metric": METRIC,
        "value": gbs,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic N(0,1), resident in HBM",
        "config": {
            "workload": "decode attention, Qwen3-8B shape, B=1, 32768-token context, one layer per "
                        "step over 36 rotated layer caches",
            "n_heads": H, "n_kv_heads": HKV, "head_dim": HD, "context": CTX, "batch": 1,
            "kv_dtype": "f16", "q_dtype": "f32", "parallelism": "none (1 GPU)",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": gbs,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": gbs / HBM_PEAK_GBS,
            "traffic": read_traffic("decode_c2"),
        },
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
