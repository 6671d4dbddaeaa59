#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path (one JSON line on stdout).

Headline (BASELINE.json metric, config C2): decode attention at Qwen3-8B shape
(H=32, Hkv=8, hd=128, f16 KV, fp32 math), batch 1, 32768-token context.  One
step is one decode-attention call for one layer; the timed steps rotate over
36 distinct layer caches (Qwen3-8B has 36 layers, 4.5 GiB of KV in all) so
the KV bytes come from HBM, not from the 256 MB last-level cache.  Inputs are
synthetic N(0,1), resident in HBM before timing starts.

Timing (every config):
  * warm-up: at least --warmup calls and at least 0.3 s of them;
  * timed region: HIP events recorded on the stream the kernels run on,
    around exactly --steps calls, with device syncs on both sides.  A spin
    kernel (torch.cuda._sleep) is queued just before the first event so the
    host enqueues the calls while it runs: the events then time the GPU
    executing the calls back to back, not the 8-10 us ctypes launch of each
    call.  ``ms_per_step`` is the mean over the timed region;
  * median: the median over 10 blocks of a second pass of the same calls
    (events between blocks only).
``roofline.achieved`` = algorithmic bytes per call / mean time per call.

Other configs (C1, ragged batches, prefill, Gemma shape, delta-net, the f-row
kernels) are reported under ``extra`` with their own roofline fractions and
medians.  Prefill (C3) inputs follow the config recipe: N(0,1), per-head
RMS norm of Q and K, then f16.

CPU baseline: the C restatement of the reference's scalar loops (oracle/,
cpu.rs:342-387 for attention, qwen35/cpu.rs:188-246 for the delta rule),
compiled -O2 without fast-math, timed on this host on a bounded sample of
each config, on one core (the reference's attention loop is serial) and on
all the cores this process may use (threads over heads), up to 16 (one GPU's
share of the host); the host's own CPU count and model are printed beside.
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
WARM_S = 0.3


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def decode_bytes(ctx_lens, H=H, Hkv=HKV, hd=HD, q_bytes=4):
    """Algorithmic bytes of one decode call: K and V rows read once (f16) plus
    q read and out written (fp32)."""
    return sum(2 * c * Hkv * hd * 2 for c in ctx_lens) + len(ctx_lens) * H * hd * (q_bytes + 4)


def prefill_flops(pairs, H=H, hd=HD):
    """4*hd FLOPs per visible (query, key) pair per head (QK^T and PV)."""
    return 4 * hd * H * pairs


def visible_pairs(S, base=0, window=0):
    pairs = 0
    for i in range(S):
        pos = base + i
        lo = max(0, pos - window + 1) if window else 0
        pairs += pos - lo + 1
    return pairs


DELTA_BYTES_PER_TOKEN = (8192 + 2 * 32 + 4096) * 4  # conv row, alpha, beta in; out row
DELTA_STATE_BYTES = 2 * 32 * 128 * 128 * 4          # S read and written


def delta_bytes(T):
    return DELTA_BYTES_PER_TOKEN * T + DELTA_STATE_BYTES


# -------------------------------------------------------------------- timing --
def _sleep_ahead(torch, n_calls):
    """Queue a spin kernel long enough for the host to enqueue n_calls calls
    (about 15 us each through ctypes) behind it."""
    us = 2000 + 15 * n_calls
    torch.cuda._sleep(int(us * 2400))  # cycles at up to 2.4 GHz


def time_calls(fns, steps, warmup, torch):
    """Mean and median ms per call of fns[i % len(fns)] (see the module doc)."""
    n = len(fns)
    i, t0 = 0, time.perf_counter()
    while i < warmup or time.perf_counter() - t0 < WARM_S:
        fns[i % n]()
        i += 1
        if i % 32 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _sleep_ahead(torch, steps)
    e0.record(st)
    for i in range(steps):
        fns[i % n]()
    e1.record(st)
    torch.cuda.synchronize()
    mean = e0.elapsed_time(e1) / steps
    # median: a second pass in blocks of calls, events only between blocks
    # (an event between every two calls adds ~2 us to short calls)
    nb = max(1, min(10, steps))
    per_block = max(1, steps // nb)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(nb + 1)]
    _sleep_ahead(torch, nb * per_block)
    ev[0].record(st)
    for b in range(nb):
        for i in range(per_block):
            fns[(b * per_block + i) % n]()
        ev[b + 1].record(st)
    torch.cuda.synchronize()
    per = sorted(ev[b].elapsed_time(ev[b + 1]) / per_block for b in range(nb))
    return mean, per[nb // 2]


def read_traffic(name):
    path = os.path.join(ROOT, "profiles", f"{name}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("bytes_per_launch")


def hbm_entry(nbytes, ms, med, **kw):
    gbs = nbytes / (ms * 1e-3) / 1e9
    return dict(kw, ms=ms, median_ms=med, bytes=nbytes, **{"GB/s": gbs}, frac_hbm=gbs / HBM_PEAK_GBS)


def mfma_entry(flops, ms, med, **kw):
    tfs = flops / (ms * 1e-3) / 1e12
    return dict(kw, ms=ms, median_ms=med, flops=flops, **{"TFLOP/s": tfs}, frac_mfma=tfs / MFMA_F16_PEAK_TFS)


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
    ms, med = time_calls(fns, steps, warmup, torch)
    nbytes = decode_bytes([CTX])
    del ks, vs
    torch.cuda.empty_cache()
    return ms, med, nbytes


# -------------------------------------------------------------------- extras --
def bench_decode_c1(lmx, torch, steps=360, warmup=36):
    """C1: batch 1, H=16, Hkv=8, hd=128, 512 cached f16 tokens, fp32 q, query
    at position 511; 36 rotated layer caches.  2.1 MB a call."""
    Hq, n, n_layers = 16, 512, N_LAYERS
    ks = [torch.randn((n, HKV * HD), dtype=torch.float16, device="cuda") for _ in range(n_layers)]
    vs = [torch.randn((n, HKV * HD), dtype=torch.float16, device="cuda") for _ in range(n_layers)]
    q = torch.randn((1, Hq * HD), dtype=torch.float32, device="cuda")
    out = torch.empty((1, Hq * HD), dtype=torch.float32, device="cuda")
    ws = lmx.Workspace()
    fns = [(lambda i=i: lmx.attention(q, ks[i], vs[i], n_heads=Hq, n_kv_heads=HKV, head_dim=HD,
                                      base_pos=n - 1, out=out, workspace=ws)) for i in range(n_layers)]
    ms, med = time_calls(fns, steps, warmup, torch)
    return hbm_entry(decode_bytes([n], Hq), ms, med, ctx=n)


def ragged_lens(B, seed):
    import torch
    g = torch.Generator().manual_seed(seed)
    return torch.randint(1024, CTX + 1, (B,), generator=g).tolist()


def bench_decode_batched(lmx, torch, B, seed, steps=20, warmup=3):
    lens = ragged_lens(B, seed)
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
    ms, med = time_calls(fns, steps, warmup, torch)
    e = hbm_entry(decode_bytes(lens), ms, med, B=B, sum_ctx=sum(lens))
    e["tokens/s"] = B / (ms * 1e-3)
    return e


def qk_normed_f16(torch, rows, heads, hd, eps=1e-6):
    """C3 recipe: N(0,1), per-head RMS norm without gain (ops.rs:40-47), f16."""
    x = torch.randn((rows, heads, hd), dtype=torch.float32, device="cuda")
    x = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps)
    return x.reshape(rows, heads * hd).to(torch.float16)


def bench_prefill(lmx, torch, S, base=0, Hq=H, Hkv=HKV, hd=HD, window=0, scale=None, qk_norm=True,
                  steps=10, warmup=2):
    n_pos = base + S
    if qk_norm:
        k = qk_normed_f16(torch, n_pos, Hkv, hd)
        q = qk_normed_f16(torch, S, Hq, hd)
    else:
        k = torch.randn((n_pos, Hkv * hd), dtype=torch.float16, device="cuda")
        q = torch.randn((S, Hq * hd), dtype=torch.float16, device="cuda")
    v = torch.randn((n_pos, Hkv * hd), dtype=torch.float16, device="cuda")
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
    ms, med = time_calls([fn], steps, warmup, torch)
    e = mfma_entry(prefill_flops(visible_pairs(S, base, window), Hq, hd), ms, med, S=S, base=base,
                   window=window, inputs="QK-normed" if qk_norm else "N(0,1)")
    e["tokens/s"] = S / (ms * 1e-3)
    return e


def bench_gemma_decode(lmx, torch, window, steps=50, warmup=5, Hkv=8, hd=256, scale=1 / 16):
    """Gemma-shape decode at 32k context.  Defaults: C4 (H 16, Hkv 8, hd 256,
    scale 1/16); Gemma 4's real global layers are Hkv 1, hd 512, scale 1.0
    (ARCHITECTURE.md:25-28).  8 rotated layer caches."""
    Hq = 16
    slots = window or CTX
    n_layers = 8
    ks = [torch.randn((slots, Hkv * hd), dtype=torch.float16, device="cuda") for _ in range(n_layers)]
    vs = [torch.randn((slots, Hkv * hd), dtype=torch.float16, device="cuda") for _ in range(n_layers)]
    q = torch.randn((1, Hq * hd), dtype=torch.float32, device="cuda")
    out = torch.empty((1, Hq * hd), dtype=torch.float32, device="cuda")
    ws = lmx.Workspace()
    fns = [(lambda i=i: lmx.attention(q, ks[i], vs[i], n_heads=Hq, n_kv_heads=Hkv, head_dim=hd,
                                      base_pos=CTX - 1, window=window, scale=scale, out=out, workspace=ws))
           for i in range(n_layers)]
    ms, med = time_calls(fns, steps, warmup, torch)
    return hbm_entry(decode_bytes([min(window or CTX, CTX)], Hq, Hkv, hd), ms, med, window=window,
                     n_kv_heads=Hkv, head_dim=hd, scale=scale)


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
    ms, med = time_calls([fn], steps, warmup, torch)
    return hbm_entry(t * (H * hd * 8 + 2 * kv_dim * 4 + 2 * kv_dim * 2), ms, med, t=t)


def bench_matvec(lmx, torch, qtype, rows, in_dim, n_mats, n_tok=1, steps=50, warmup=5):
    """lmx_matvec: y = W x over n_mats distinct weight matrices in turn (so W
    comes from HBM, as a decode step's projections do).  Bytes are the weight
    bytes plus x and y."""
    bb, be = {"q4_k": (144, 256), "q6_k": (210, 256), "q8_0": (34, 32), "bf16": (2, 1)}[qtype]
    nbytes = rows * (in_dim // be) * bb
    ws = [torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda") for _ in range(n_mats)]
    x = torch.randn((n_tok, in_dim), device="cuda")
    y = torch.empty((n_tok, rows), device="cuda")
    fns = [(lambda w=w: lmx.matvec(w, x, qtype=qtype, rows=rows, in_dim=in_dim, y=y)) for w in ws]
    ms, med = time_calls(fns, steps, warmup, torch)
    del ws
    e = hbm_entry(nbytes + 4 * n_tok * (in_dim + rows), ms, med, type=qtype, rows=rows, in_dim=in_dim,
                  n_tok=n_tok, weight_bytes=nbytes)
    e["TFLOP/s"] = 2.0 * rows * in_dim * n_tok / (ms * 1e-3) / 1e12
    return e


def bench_kvm(lmx, torch, which, steps=20, warmup=3):
    """KV manager.  "wipe": zeroing one Qwen3-8B sequence slab (36 layers of
    f16 K and V at 32k positions, 4.83 GB) with lmx_kvm_wipe, an HBM write.
    "batch": host time of lmx_kvm_batch for a ragged batch of 32 sequences."""
    layers = [(0, HKV * HD, -1)] * N_LAYERS
    if which == "wipe":
        m = lmx.KvManager(layers, n_ctx=CTX, max_seqs=1)
        s = m.open()
        ms, med = time_calls([lambda: m.wipe(s)], steps, warmup, torch)
        nbytes = m.arena_bytes
        del m
        return hbm_entry(nbytes, ms, med)
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
    ms, med = time_calls([fn], steps, warmup, torch)
    return hbm_entry(nbytes, ms, med, T=T)


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
    ms, med = time_calls([fn], steps, warmup, torch)
    e = hbm_entry(delta_bytes(T), ms, med, T=T, chunked=chunked)
    e["tokens/s"] = T / (ms * 1e-3)
    return e


# -------------------------------------------------------------- CPU baseline --
def cpu_cores_all():
    """Cores this process may use, at most 16 (one GPU's share of the box)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def host_cpu_info():
    """The host's logical CPU count, the count this process may run on, and
    the CPU model (from /proc/cpuinfo), reported beside the CPU baselines."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = None
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"logical_cpus": os.cpu_count(), "cpus_allowed": affinity, "model": model,
            "threads_used_all_cores": cpu_cores_all()}


_KV_CACHE = {}


def _cpu_kv(n_pos, kv_dim, seed):
    """f16-representable K/V rows for the oracle, generated once per shape."""
    key = (kv_dim, seed)
    if key in _KV_CACHE and _KV_CACHE[key][0].shape[0] >= n_pos:
        k, v = _KV_CACHE[key]
        return k[:n_pos], v[:n_pos]
    import numpy as np
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((n_pos, kv_dim), dtype=np.float32).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((n_pos, kv_dim), dtype=np.float32).astype(np.float16).astype(np.float32)
    _KV_CACHE[key] = (k, v)
    return k, v


def cpu_attention_rows(rows, *, Hq, Hkv, hd, n_pos, window=0, scale=None, unit, threads, budget_s,
                       what):
    """Time the C oracle's attention (cpu.rs:342-387) on sampled query rows:
    each row is a one-token call at its position (the same computation as
    that row of a prefill or decode batch).  rows are visited in the given
    order until budget_s is spent; unit "GB/s" counts decode bytes (f16 K/V
    read once, q and out), "TFLOP/s" 4*hd*H per visible pair."""
    import numpy as np
    import oracle
    k, v = _cpu_kv(n_pos, Hkv * hd, 11)
    q = np.random.default_rng(12).standard_normal((1, Hq * hd), dtype=np.float32)
    done, work, t0 = 0, 0.0, time.perf_counter()
    for pos in rows:
        oracle.attention(q, k, v, n_heads=Hq, n_kv_heads=Hkv, head_dim=hd, base_pos=int(pos),
                         window=window, scale=scale, n_threads=threads)
        lo = max(0, pos - window + 1) if window else 0
        n_vis = pos - lo + 1
        work += (2 * n_vis * Hkv * hd * 2 + Hq * hd * 8) if unit == "GB/s" else 4 * hd * Hq * n_vis
        done += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    el = time.perf_counter() - t0
    val = work / el / (1e9 if unit == "GB/s" else 1e12)
    return {"value": val, "unit": unit, "cores": threads, "kind": "port",
            "sample": f"{what}: {done} query rows, {el:.2f} s, C oracle -O2, {threads} thread(s)"}


def cpu_delta(T_sample, threads, budget_s):
    """The C oracle's delta rule (qwen35/cpu.rs:188-246) at the C5 shape over
    T_sample tokens (threads over v-heads), scaled to C5's bytes per token."""
    import numpy as np
    import oracle
    n_vh, n_kh, sd = 32, 16, 128
    rng = np.random.default_rng(5)
    conv = rng.standard_normal((T_sample, 2 * n_kh * sd + n_vh * sd), dtype=np.float32)
    qk = conv[:, :2 * n_kh * sd].reshape(T_sample, 2 * n_kh, sd)
    qk /= np.linalg.norm(qk, axis=-1, keepdims=True)
    al = rng.standard_normal((T_sample, n_vh), dtype=np.float32)
    be = rng.standard_normal((T_sample, n_vh), dtype=np.float32)
    S0 = np.zeros((n_vh, sd, sd), np.float32)
    t0 = time.perf_counter()
    n_done = 0
    while True:
        oracle.delta_recur(conv, al, be, S0, n_vh=n_vh, n_kh=n_kh, s_dim=sd, n_threads=threads)
        n_done += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    per_tok = (time.perf_counter() - t0) / (n_done * T_sample)
    return per_tok


def cpu_baselines(budget_s):
    """One-core and all-core CPU figures per config, keyed like ``extra``."""
    import numpy as np
    allc = cpu_cores_all()
    out = {}
    _cpu_kv(CTX, HKV * HD, 11)
    _cpu_kv(CTX, 8 * 256, 11)

    def both(name, fn):
        t0 = time.perf_counter()
        out[name] = {"1core": fn(1), "all_cores": fn(allc)}
        log(f"cpu {name}: 1 core {out[name]['1core']['value']:.4g}, {allc} cores "
            f"{out[name]['all_cores']['value']:.4g} {out[name]['1core']['unit']} "
            f"({time.perf_counter() - t0:.1f}s)")

    def spread(S, base, n):  # n positions evenly over the batch
        return [base + int(x) for x in np.linspace(0, S - 1, n)]

    both("headline", lambda th: cpu_attention_rows([CTX - 1] * 50, Hq=H, Hkv=HKV, hd=HD, n_pos=CTX,
                                                   unit="GB/s", threads=th, budget_s=budget_s,
                                                   what="C2 B=1 ctx 32768 decode"))
    both("decode_c1_ctx512", lambda th: cpu_attention_rows([511] * 20000, Hq=16, Hkv=HKV, hd=HD, n_pos=512,
                                                           unit="GB/s", threads=th, budget_s=budget_s,
                                                           what="C1 decode"))
    for B, seed in ((8, 8), (32, 32)):
        lens = ragged_lens(B, seed)
        both(f"decode_b{B}", lambda th, lens=lens, B=B: cpu_attention_rows(
            [n - 1 for n in lens], Hq=H, Hkv=HKV, hd=HD, n_pos=CTX, unit="GB/s", threads=th,
            budget_s=budget_s, what=f"C2 B={B} ragged decode, sequences in order"))
    for S, base in ((512, 0), (2048, 0), (8192, 0), (512, 4096)):
        name = f"prefill_s{S}" if base == 0 else "prefill_chunk512_on_4k"
        both(name, lambda th, S=S, base=base: cpu_attention_rows(
            spread(S, base, 64), Hq=H, Hkv=HKV, hd=HD, n_pos=base + S, unit="TFLOP/s", threads=th,
            budget_s=budget_s, what=f"C3 prefill S={S} base={base}, rows spread over the batch"))
    for w, name in ((1024, "gemma_prefill_swa_4k"), (0, "gemma_prefill_global_4k")):
        both(name, lambda th, w=w: cpu_attention_rows(
            spread(4096, 0, 64), Hq=16, Hkv=8, hd=256, n_pos=4096, window=w, scale=1 / 16,
            unit="TFLOP/s", threads=th, budget_s=budget_s, what=f"C4 prefill 4k window={w}"))
    both("gemma_decode_swa_w1024", lambda th: cpu_attention_rows(
        [CTX - 1] * 500, Hq=16, Hkv=8, hd=256, n_pos=CTX, window=1024, scale=1 / 16, unit="GB/s",
        threads=th, budget_s=budget_s, what="C4 SWA decode at 32k"))
    both("gemma_decode_global", lambda th: cpu_attention_rows(
        [CTX - 1] * 50, Hq=16, Hkv=8, hd=256, n_pos=CTX, scale=1 / 16, unit="GB/s", threads=th,
        budget_s=budget_s, what="C4 global decode at 32k"))
    _cpu_kv(CTX, 512, 11)
    both("gemma4_global_prefill_4k_hd512", lambda th: cpu_attention_rows(
        spread(4096, 0, 64), Hq=16, Hkv=1, hd=512, n_pos=4096, scale=1.0, unit="TFLOP/s", threads=th,
        budget_s=budget_s, what="Gemma 4 global layer prefill 4k (hd 512, one kv head)"))
    both("gemma4_global_decode_32k_hd512", lambda th: cpu_attention_rows(
        [CTX - 1] * 50, Hq=16, Hkv=1, hd=512, n_pos=CTX, scale=1.0, unit="GB/s", threads=th,
        budget_s=budget_s, what="Gemma 4 global layer decode at 32k (hd 512, one kv head)"))

    def delta(th, T, name):
        per_tok = cpu_delta(64, th, budget_s)
        gbs = delta_bytes(T) / (per_tok * T) / 1e9
        return {"value": gbs, "unit": "GB/s", "cores": th, "kind": "port",
                "tokens/s": 1.0 / per_tok,
                "sample": f"{name}: 64-token runs of the recurrence, {per_tok * 1e3:.3f} ms/token, "
                          f"C oracle -O2, {th} thread(s)"}
    both("delta_prefill_T4096_chunked", lambda th: delta(th, 4096, "C5 prefill"))
    both("delta_decode_1tok", lambda th: delta(th, 1, "C5 decode"))
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--only", choices=["headline", "all"], default="all")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=1.0,
                    help="seconds of CPU timing per config and mode (the headline's 1-core figure "
                         "gets 10x)")
    ap.add_argument("--extras", default="",
                    help="comma-separated names of the extra configs to run (default: all)")
    ap.add_argument("--pmc-calibration", action="store_true",
                    help="after the timed runs, copy a 256 MiB fp32 buffer 3 times: the known-size "
                         "reference that FETCH_SIZE / WRITE_SIZE counter readings are scaled by")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}): this build has no "
              "multi-GPU path (each GPU would run these kernels on its own heads' share).",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import llmoxide_amd as lmx

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    lmx.lib()  # fail loudly if the HIP library is missing

    log(f"headline: decode B=1 ctx {CTX}, {args.steps} steps, {args.warmup} warmup")
    ms, med, nbytes = bench_decode_headline(lmx, torch, args.steps, args.warmup)
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"headline: {ms * 1e3:.2f} us/call (median {med * 1e3:.2f}), {gbs:.1f} GB/s")

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
                                                           window=1024, scale=1 / 16, qk_norm=False,
                                                           steps=5, warmup=1)),
            ("gemma_prefill_global_4k", lambda: bench_prefill(lmx, torch, 4096, Hq=16, Hkv=8, hd=256,
                                                              scale=1 / 16, qk_norm=False, steps=5,
                                                              warmup=1)),
            # Gemma 4's real global layers: hd 512, one kv head, scale 1.0 on
            # RMS-normed q and k (ARCHITECTURE.md:25-28, 54-62); FLOPs are the
            # algorithmic 4*hd*H per visible pair
            ("gemma4_global_prefill_4k_hd512", lambda: bench_prefill(lmx, torch, 4096, Hq=16, Hkv=1, hd=512,
                                                                     scale=1.0, qk_norm=True, steps=5,
                                                                     warmup=1)),
            ("gemma4_global_decode_32k_hd512", lambda: bench_gemma_decode(lmx, torch, 0, Hkv=1, hd=512,
                                                                          scale=1.0)),
            ("prologue_prefill_t4096", lambda: bench_prologue(lmx, torch, 4096)),
            ("prologue_decode_t1", lambda: bench_prologue(lmx, torch, 1, steps=50, warmup=5)),
            ("delta_prefill_T4096_chunked", lambda: bench_delta(lmx, torch, 4096, True)),
            ("delta_prefill_T4096_sequential", lambda: bench_delta(lmx, torch, 4096, False)),
            ("delta_decode_1tok", lambda: bench_delta(lmx, torch, 1, False, steps=50, warmup=5)),
            ("delta_front_T4096", lambda: bench_delta_io(lmx, torch, 4096, "front")),
            ("delta_back_T4096", lambda: bench_delta_io(lmx, torch, 4096, "back")),
            ("matvec_q4k_attn_output_4096", lambda: bench_matvec(lmx, torch, "q4_k", 4096, 4096, 36)),
            ("matvec_q8_0_attn_output_4096", lambda: bench_matvec(lmx, torch, "q8_0", 4096, 4096, 36)),
            ("matvec_q6k_attn_output_4096", lambda: bench_matvec(lmx, torch, "q6_k", 4096, 4096, 36)),
            ("gemm_q4k_attn_output_4096_t512", lambda: bench_matvec(lmx, torch, "q4_k", 4096, 4096, 8,
                                                                    n_tok=512, steps=20)),
            ("gemm_q6k_attn_output_4096_t512", lambda: bench_matvec(lmx, torch, "q6_k", 4096, 4096, 8,
                                                                    n_tok=512, steps=20)),
            ("gemm_q8_0_attn_output_4096_t512", lambda: bench_matvec(lmx, torch, "q8_0", 4096, 4096, 8,
                                                                     n_tok=512, steps=20)),
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

    cpu = None
    if not args.skip_cpu:
        cpus = cpu_baselines(args.cpu_budget)
        for name, v in cpus.items():
            if name != "headline" and name in extra:
                extra[name]["cpu"] = v
        # the headline's one-core figure on a longer sample (about 10 s)
        cpu = cpu_attention_rows([CTX - 1] * 50, Hq=H, Hkv=HKV, hd=HD, n_pos=CTX, unit="GB/s",
                                 threads=1, budget_s=10 * args.cpu_budget,
                                 what="C2 B=1 ctx 32768 decode (the headline shape)")
        cpu["all_cores"] = cpus["headline"]["all_cores"]
        cpu["host"] = host_cpu_info()
        log(f"cpu baseline: {cpu}")

    line = {
        "metric": METRIC,
        "value": gbs,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "median_ms_per_step": med,
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
