"""GPU parity at every configured size, exact masks, and the reference's real
attention scale.

1. Full-size configs against the C oracle:
   * C4 Gemma prefill at 4096 tokens, SWA (w 1024) and global, hd 256 (seeded
     sample rows: a causal row depends only on its own position and keys);
   * C4 global decode at a 32768-token context, hd 256;
   * C2 ragged decode, B = 32 with context lengths drawn from [1k, 32k];
   * C5 chunked delta rule at T = 4096, all 32 v-heads (oracle threaded over
     heads, same arithmetic per head).
2. Exact visible ranges.  With q = 0 every visible key gets weight exactly 1
   (score 0, exp2(0) = 1 in every path), so out[d] = sum_{p in [lo, hi]}
   V[p, d] / n.  V rows carry +-1 bits of their position (dims 0..15) and of
   their kv head (dims 16..19), so the output is an exact integer ratio
   (sums of +-1 are exact in fp32; only the final division rounds).  Each
   row must match its closed-form range [lo, hi] (attn.wgsl:52-66,
   cache.rs:30-38) to 2e-6, and must differ by more than 1e-5 from every
   off-by-one range [lo+-1, hi] and [lo, hi+-1]: an off-by-one changes the
   bit-0 average by ~1/n >= 2.4e-5 at n <= 32768 (the bound the test uses).
   The kv-head dims pin the GQA map h / G (attn.wgsl:78-80), the position
   bits the ring slot map p % w (cache.rs:21-28).
3. Gemma's real scale, 1.0 (config.rs:264-270), with QK-normed heads: the
   scores q.k of unit-RMS heads have a standard deviation of sqrt(hd) (16 at
   hd 256), so the softmax is peaked and the lazy rescale and the f16 P are
   exercised far from N(0,1) scores.

Tolerance for 1 and 3: max abs error <= 2e-3 and max|diff|/max|ref| <= 1e-2
(tests/helpers.py).
"""
import os
import sys

import numpy as np
import pytest

import oracle
from tests.helpers import CPU_THREADS, AttnCase, assert_close, delta_inputs

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import llmoxide_amd as lmx  # noqa: E402

ORACLE_THREADS = max(CPU_THREADS, min(16, os.cpu_count() or 1))


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.cuda()


@pytest.fixture(params=["tile", "pp"])
def prefill_kernel(request, tuning_env):
    """Prefill cases run on both prefill kernels (the ping-pong kernel exists
    for head_dim 128; other head sizes take the tile kernel either way)."""
    tuning_env("LMX_PREFILL_KERNEL", request.param)
    return request.param


# --------------------------------------------------------------- 1. sizes --
def sampled_rows(S, seed, n=45):
    return np.unique(np.concatenate([[0, S - 1, S // 2, 1023, 1024, 1025],
                                     np.random.default_rng(seed).integers(0, S, n)]))


@pytest.mark.parametrize("window", [1024, 0])
def test_c4_gemma_prefill_4096_sampled_rows(window):
    """C4: H=16, Hkv=8, hd 256, scale 1/16, N(0,1) inputs, 4096 tokens at base
    0.  SWA layers read the batch's own rows (k_cur) over an empty ring."""
    S, H, Hkv, hd = 4096, 16, 8, 256
    say(f"C4 prefill S={S} window={window}")
    c = AttnCase(4096 + window, t=S, H=H, Hkv=Hkv, hd=hd, n_pos=S, q_f16=True)
    q = dev(c.q.astype(np.float16))
    if window:
        ring = np.zeros((window, c.kv_dim), np.uint16)
        out = lmx.attention(q, dev(ring, torch.float16), dev(ring, torch.float16), n_heads=H,
                            n_kv_heads=Hkv, head_dim=hd, base_pos=0, window=window, scale=1 / 16,
                            k_cur=dev(c.k16, torch.float16), v_cur=dev(c.v16, torch.float16))
    else:
        out = lmx.attention(q, dev(c.k16, torch.float16), dev(c.v16, torch.float16), n_heads=H,
                            n_kv_heads=Hkv, head_dim=hd, base_pos=0, scale=1 / 16)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for i in sampled_rows(S, window + 7):
        ref = oracle.attention(c.q[i:i + 1], c.kf, c.vf, n_heads=H, n_kv_heads=Hkv, head_dim=hd,
                               base_pos=int(i), window=window, scale=1 / 16, n_threads=ORACLE_THREADS)
        assert_close(got[i:i + 1], ref, what=f"row {i}")


def test_c4_global_decode_32k_hd256():
    """C4 global layer decode: query at 32767 over 32768 keys, hd 256."""
    say("C4 global decode ctx=32768 hd=256")
    c = AttnCase(32768 + 256, t=1, H=16, Hkv=8, hd=256, n_pos=32768)
    out = lmx.attention(dev(c.q), dev(c.k16, torch.float16), dev(c.v16, torch.float16), n_heads=16,
                        n_kv_heads=8, head_dim=256, base_pos=32767, scale=1 / 16)
    torch.cuda.synchronize()
    ref = c.reference(base_pos=32767, scale=1 / 16, threads=ORACLE_THREADS)
    assert_close(out.cpu().numpy(), ref, what="C4 global decode")


def test_c2_batched_b32_ctx_1k_to_32k():
    """C2 at B = 32 with ragged contexts ~ U[1k, 32k] (the configured range):
    every sequence against the oracle at its own length."""
    H, Hkv, hd, B = 32, 8, 128, 32
    lens = np.random.default_rng(3232).integers(1024, 32769, B).tolist()
    max_ctx = int(max(lens))
    say(f"C2 batched B={B} lens in [{min(lens)}, {max_ctx}] sum={sum(lens)}")
    ks, vs, qs, refs = [], [], [], []
    for i, n in enumerate(lens):
        c = AttnCase(5000 + i, t=1, H=H, Hkv=Hkv, hd=hd, n_pos=n)
        refs.append(c.reference(base_pos=n - 1, threads=ORACLE_THREADS))
        qs.append(c.q)
        ks.append(dev(c.k16, torch.float16))
        vs.append(dev(c.v16, torch.float16))
        del c
    out = lmx.attention_decode_batched(dev(np.concatenate(qs)), lmx.BatchedCaches(ks, vs),
                                       dev(np.array(lens, np.int32)), max_ctx=max_ctx, n_heads=H,
                                       n_kv_heads=Hkv, head_dim=hd, n_slots=max_ctx)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for i in range(B):
        assert_close(got[i:i + 1], refs[i], what=f"seq {i} ctx {lens[i]}")


def test_c5_chunked_4096_all_heads_vs_oracle():
    """C5 at full size against the oracle itself (not the HIP sequential
    kernel): T = 4096, Hv = 32, Hk = 16, d = 128, chunk 64; o and the final S."""
    n_vh, n_kh, sd, T = 32, 16, 128, 4096
    say(f"C5 chunked T={T} vs oracle ({ORACLE_THREADS} threads)")
    conv, al, be, S0, A, dt = delta_inputs(4096, T=T, n_vh=n_vh, n_kh=n_kh, sd=sd)
    o_ref, S_ref = oracle.delta_recur(conv, al, be, S0, n_vh=n_vh, n_kh=n_kh, s_dim=sd,
                                      n_threads=ORACLE_THREADS)
    state = dev(S0.reshape(n_vh, sd, sd).copy())
    o = lmx.delta_chunked(dev(conv), dev(al), dev(be), state, dev(A), dev(dt), n_vh=n_vh, n_kh=n_kh,
                          s_dim=sd, chunk=64)
    torch.cuda.synchronize()
    e_o = assert_close(o.cpu().numpy(), o_ref, what="o")
    e_s = assert_close(state.cpu().numpy().ravel(), S_ref, what="S")
    say(f"  o max_abs={e_o[0]:.2e}; S max_abs={e_s[0]:.2e}")


# ---------------------------------------------------------- 2. exact masks --
NBITS = 16


def position_values(n_pos, Hkv, hd):
    """f16 bits of V rows [n_pos, Hkv*hd]: dims 0..15 of head h are +-1 bits of
    the row's position, dims 16..19 +-1 bits of h, the rest 0."""
    v = np.zeros((n_pos, Hkv, hd), np.float32)
    p = np.arange(n_pos)[:, None]
    v[:, :, :NBITS] = np.where((p[:, :, None] >> np.arange(NBITS)) & 1, 1.0, -1.0)[:, 0:1, :]
    for h in range(Hkv):
        v[:, h, NBITS:NBITS + 4] = np.where((h >> np.arange(4)) & 1, 1.0, -1.0)
    return oracle.to_f16_bits(v.reshape(n_pos, Hkv * hd))


def range_average(lo, hi):
    """Exact mean over p in [lo, hi] of the +-1 bit planes of p."""
    n = hi - lo + 1
    e = np.empty(NBITS)
    for d in range(NBITS):
        c = ones_below(hi + 1, d) - ones_below(lo, d)
        e[d] = (2.0 * c - n) / n
    return e


def ones_below(x, d):
    """How many p in [0, x) have bit d set: 2^d per whole period of 2^(d+1),
    plus the part of the last period past its first 2^d."""
    return ((x >> (d + 1)) << d) + max(0, (x & ((2 << d) - 1)) - (1 << d))


def check_exact(out, *, t, H, Hkv, hd, ranges):
    """out [t, H*hd]; ranges[i] = (lo, hi) of token i (all heads)."""
    out = out.reshape(t, H, hd).astype(np.float64)
    G = H // Hkv
    for i in range(t):
        lo, hi = ranges[i]
        want = range_average(lo, hi)
        for h in range(H):
            kvh = h // G
            got = out[i, h]
            err = np.abs(got[:NBITS] - want).max()
            assert err <= 2e-6, f"token {i} head {h}: [{lo}, {hi}] off by {err:.2e}"
            bits = np.where((kvh >> np.arange(4)) & 1, 1.0, -1.0)
            # +-n * fl(1/n): +-1 within an ulp or two
            assert np.abs(got[NBITS:NBITS + 4] - bits).max() <= 2e-6, f"token {i} head {h}: kv head"
            assert np.all(got[NBITS + 4:] == 0.0)
            for (a, b) in ((lo - 1, hi), (lo + 1, hi), (lo, hi - 1), (lo, hi + 1)):
                if 0 <= a <= b:
                    assert np.abs(got[:NBITS] - range_average(a, b)).max() > 1e-5, \
                        f"token {i}: [{a}, {b}] indistinguishable from [{lo}, {hi}]"


def closed_ranges(base, t, window, bidi):
    return [oracle.visible(base + i, window, base, t, bidi) for i in range(t)]


def exact_case(*, t, H, Hkv, hd, base, window=0, bidi=False, ring=False, k_cur=False, q_f16=False):
    say(f"exact mask t={t} H={H} Hkv={Hkv} hd={hd} base={base} w={window} bidi={bidi} "
        f"ring={ring} k_cur={k_cur}")
    end = base + t
    v16 = position_values(end, Hkv, hd)
    k16 = oracle.to_f16_bits(oracle.normal(t + base + hd, (end, Hkv * hd)))
    if ring:
        upto = base if k_cur else end
        kc = np.zeros((window, Hkv * hd), np.uint16)
        vc = np.zeros((window, Hkv * hd), np.uint16)
        for p in range(max(0, upto - window), upto):
            kc[p % window], vc[p % window] = k16[p], v16[p]
    else:
        kc, vc = k16, v16
    q = np.zeros((t, H * hd), np.float32)
    qd = dev(q.astype(np.float16)) if q_f16 else dev(q)
    kw = {}
    if k_cur:
        kw = dict(k_cur=dev(k16[base:end], torch.float16), v_cur=dev(v16[base:end], torch.float16))
    out = lmx.attention(qd, dev(kc, torch.float16), dev(vc, torch.float16), n_heads=H, n_kv_heads=Hkv,
                        head_dim=hd, base_pos=base, window=window, bidi=bidi, **kw)
    torch.cuda.synchronize()
    check_exact(out.cpu().numpy(), t=t, H=H, Hkv=Hkv, hd=hd,
                ranges=closed_ranges(base, t, window, bidi))


@pytest.mark.parametrize("kw", [
    dict(t=1, H=32, Hkv=8, hd=128, base=32767),                                    # C2 headline
    dict(t=1, H=16, Hkv=8, hd=256, base=32767, window=1024, ring=True),            # C4 SWA decode
    dict(t=1, H=16, Hkv=8, hd=256, base=1000, window=1024, ring=True),             # before the wrap
    dict(t=5, H=32, Hkv=8, hd=128, base=4091),                                     # few tokens
    dict(t=6, H=8, Hkv=2, hd=64, base=44, window=16, bidi=True, ring=True, k_cur=True),
    dict(t=7, H=8, Hkv=4, hd=128, base=53, window=16, ring=True, k_cur=True),
])
def test_exact_visible_range_decode(kw):
    exact_case(**kw)


@pytest.mark.parametrize("kw", [
    dict(t=4096, H=16, Hkv=8, hd=256, base=0, window=1024, ring=True, k_cur=True),  # C4 SWA 4k
    dict(t=4096, H=8, Hkv=2, hd=128, base=0, window=1024, ring=True, k_cur=True),
    dict(t=2048, H=8, Hkv=2, hd=128, base=0),                                       # causal
    dict(t=512, H=8, Hkv=2, hd=128, base=4096),                                     # chunk, key splits
    dict(t=256, H=8, Hkv=2, hd=128, base=1044, window=300, ring=True, k_cur=True),  # chunk on a ring
    dict(t=300, H=8, Hkv=4, hd=128, base=100, window=64, bidi=True, ring=True, k_cur=True),
    dict(t=300, H=8, Hkv=4, hd=64, base=100, bidi=True),
    dict(t=600, H=4, Hkv=1, hd=512, base=0, window=256, ring=True, k_cur=True),  # hd 512, dim slices
    dict(t=96, H=4, Hkv=1, hd=512, base=3000),                                    # hd 512, key splits
])
def test_exact_visible_range_prefill(kw, prefill_kernel):
    exact_case(q_f16=True, **kw)


def test_exact_visible_range_batched_decode():
    """Ragged batch: each sequence sees exactly [0, ctx_b - 1] of its cache."""
    H, Hkv, hd = 32, 8, 128
    lens = [1, 17, 1000, 1024, 4097, 30000, 32768, 12345]
    max_ctx = max(lens)
    say(f"exact mask batched lens={lens}")
    v16 = position_values(max_ctx, Hkv, hd)
    k16 = oracle.to_f16_bits(oracle.normal(99, (max_ctx, Hkv * hd)))
    ks = [dev(k16[:n], torch.float16) for n in lens]
    vs = [dev(v16[:n], torch.float16) for n in lens]
    q = torch.zeros((len(lens), H * hd), dtype=torch.float32, device="cuda")
    out = lmx.attention_decode_batched(q, lmx.BatchedCaches(ks, vs), dev(np.array(lens, np.int32)),
                                       max_ctx=max_ctx, n_heads=H, n_kv_heads=Hkv, head_dim=hd,
                                       n_slots=max_ctx)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for b, n in enumerate(lens):
        check_exact(out[b:b + 1], t=1, H=H, Hkv=Hkv, hd=hd, ranges=[(0, n - 1)])


def test_exact_check_rejects_a_planted_off_by_one():
    """The check itself: the average of [lo, hi] passes, the average of a
    window one key too wide (a plausible mask slip) does not."""
    lo, hi = 31744, 32767
    good = np.zeros((1, 1, 32))
    good[0, 0, :NBITS] = range_average(lo, hi)
    good[0, 0, NBITS:NBITS + 4] = -1.0
    check_exact(good.reshape(1, 32), t=1, H=1, Hkv=1, hd=32, ranges=[(lo, hi)])
    bad = good.copy()
    bad[0, 0, :NBITS] = range_average(lo - 1, hi)
    with pytest.raises(AssertionError):
        check_exact(bad.reshape(1, 32), t=1, H=1, Hkv=1, hd=32, ranges=[(lo, hi)])


# ------------------------------------------------- 3. scale 1.0, QK-normed --
@pytest.mark.parametrize("hd,H,Hkv,t,base,window", [
    (256, 16, 8, 1024, 0, 0),       # Gemma global, first chunk
    (256, 16, 8, 2048, 0, 1024),    # Gemma SWA, past the window (k_cur)
    (256, 16, 8, 256, 7000, 0),     # a chunk on a long cache (key splits)
    (128, 32, 8, 1024, 0, 0),       # both kernels at hd 128
    (512, 16, 1, 1024, 0, 0),       # Gemma 4 global layer shape
])
@pytest.mark.parametrize("q_f16", [True, False])
def test_scale_one_qk_normed_prefill(hd, H, Hkv, t, base, window, q_f16, prefill_kernel):
    # f16 queries enter the MFMA as given; fp32 queries as their f16 rounding
    # plus its f16 residual (one rounding alone moves scale-1.0 scores by
    # ~1e-2 in log2 units, past the tolerance)
    say(f"scale 1.0 prefill[{prefill_kernel}] hd={hd} t={t} base={base} w={window} q_f16={q_f16}")
    c = AttnCase(hd + t + base + window, t=t, H=H, Hkv=Hkv, hd=hd, n_pos=base + t, q_f16=q_f16,
                 qk_norm=True)
    q = dev(c.q.astype(np.float16)) if q_f16 else dev(c.q)
    if window:
        ring = np.zeros((window, c.kv_dim), np.uint16)
        for p in range(max(0, base - window), base):
            ring[p % window] = c.k16[p]
        vring = np.zeros_like(ring)
        for p in range(max(0, base - window), base):
            vring[p % window] = c.v16[p]
        out = lmx.attention(q, dev(ring, torch.float16), dev(vring, torch.float16), n_heads=H,
                            n_kv_heads=Hkv, head_dim=hd, base_pos=base, window=window, scale=1.0,
                            k_cur=dev(c.k16[base:], torch.float16), v_cur=dev(c.v16[base:], torch.float16))
    else:
        out = lmx.attention(q, dev(c.k16, torch.float16), dev(c.v16, torch.float16), n_heads=H,
                            n_kv_heads=Hkv, head_dim=hd, base_pos=base, scale=1.0)
    torch.cuda.synchronize()
    ref = c.reference(base_pos=base, window=window, scale=1.0, threads=ORACLE_THREADS)
    # fp32 queries at a tighter bound: their error is the f16 P rounding
    # alone (about 5e-4 here, as for f16 queries against their own oracle);
    # a residual taken against a differently rounded hi showed as 2.6e-3
    e = assert_close(out.cpu().numpy(), ref, abs_tol=2e-3 if q_f16 else 1.5e-3, what="scale 1.0 prefill")
    say(f"  max_abs={e[0]:.2e} rel={e[1]:.2e}")


@pytest.mark.parametrize("hd,H,Hkv,ctx,window", [
    (256, 16, 8, 8192, 0),
    (256, 16, 8, 32768, 1024),
    (128, 32, 8, 32768, 0),
    (512, 16, 1, 4096, 0),          # Gemma 4 global layers: hd 512, one kv head
])
def test_scale_one_qk_normed_decode(hd, H, Hkv, ctx, window):
    say(f"scale 1.0 decode hd={hd} ctx={ctx} w={window}")
    c = AttnCase(hd + ctx, t=1, H=H, Hkv=Hkv, hd=hd, n_pos=ctx, qk_norm=True)
    if window:
        kc, vc = c.ring(window, ctx)
    else:
        kc, vc = c.k16, c.v16
    out = lmx.attention(dev(c.q), dev(kc, torch.float16), dev(vc, torch.float16), n_heads=H,
                        n_kv_heads=Hkv, head_dim=hd, base_pos=ctx - 1, window=window, scale=1.0)
    torch.cuda.synchronize()
    ref = c.reference(base_pos=ctx - 1, window=window, scale=1.0, threads=ORACLE_THREADS)
    e = assert_close(out.cpu().numpy(), ref, what="scale 1.0 decode")
    say(f"  max_abs={e[0]:.2e} rel={e[1]:.2e}")
