"""GPU parity: MFMA tiled attention (prefill, chunked prefill, sliding window,
bidirectional) vs the C oracle.

Full-size cases (S=8192) are checked on a seeded sample of query rows: a
query's causal output depends only on its own position and the keys it sees,
so the oracle run at t=1 for that position is the same computation.
"""
import sys

import numpy as np
import pytest

import oracle
from tests.helpers import CPU_THREADS, AttnCase, assert_close

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import llmoxide_amd as lmx  # noqa: E402


@pytest.fixture(autouse=True, params=["tile", "pp"])
def prefill_kernel(request, tuning_env):
    """Every case on both prefill kernels: the 128-row tile kernel and the
    ping-pong kernel (head_dim 128 only; other head sizes use the tile kernel
    under either setting)."""
    tuning_env("LMX_PREFILL_KERNEL", request.param)
    return request.param


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.cuda()


def lmx_kernel():
    import os
    return os.environ.get("LMX_PREFILL_KERNEL", "auto")


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def gpu_attn(c: AttnCase, *, base, window=0, bidi=False, scale=None, ring=False, k_cur=False):
    end = base + c.t
    if ring:
        kc, vc = c.ring(window, base) if k_cur else c.ring(window, end)
        if base == 0 and k_cur:
            kc = np.zeros((window, c.kv_dim), np.uint16)
            vc = np.zeros((window, c.kv_dim), np.uint16)
    else:
        kc, vc = c.k16[:end], c.v16[:end]
    q = dev(c.q.astype(np.float16)) if c.q_f16 else dev(c.q)
    kw = {}
    if k_cur:
        kw = dict(k_cur=dev(c.k16[base:end], torch.float16), v_cur=dev(c.v16[base:end], torch.float16))
    out = lmx.attention(q, dev(kc, torch.float16), dev(vc, torch.float16), n_heads=c.H,
                        n_kv_heads=c.Hkv, head_dim=c.hd, base_pos=base, window=window, bidi=bidi,
                        scale=scale, kv_dim=c.kv_dim, **kw)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def check(c, *, base, window=0, bidi=False, scale=None, ring=False, k_cur=False):
    say(f"prefill[{lmx_kernel()}] t={c.t} H={c.H} Hkv={c.Hkv} hd={c.hd} base={base} w={window} bidi={bidi} "
        f"ring={ring} k_cur={k_cur} q_f16={c.q_f16}")
    got = gpu_attn(c, base=base, window=window, bidi=bidi, scale=scale, ring=ring, k_cur=k_cur)
    ref = c.reference(base_pos=base, window=window, bidi=bidi, scale=scale)
    return assert_close(got, ref, what="prefill")


@pytest.mark.parametrize("S", [9, 128, 200, 512])
def test_causal_prefill_qwen3_shape(S):
    """C3 recipe: QK-normed N(0,1) inputs, f16 Q/K/V, causal."""
    c = AttnCase(S, t=S, H=32, Hkv=8, hd=128, n_pos=S, q_f16=True, qk_norm=True)
    check(c, base=0)


def test_causal_prefill_2048():
    c = AttnCase(2048, t=2048, H=32, Hkv=8, hd=128, n_pos=2048, q_f16=True, qk_norm=True)
    check(c, base=0)


def test_chunked_prefill_512_onto_4096():
    """C3 chunked: a 512-token chunk appended onto a 4096-token cache."""
    c = AttnCase(4608, t=512, H=32, Hkv=8, hd=128, n_pos=4608, q_f16=True, qk_norm=True)
    check(c, base=4096)


def test_f32_query_prefill():
    c = AttnCase(77, t=300, H=16, Hkv=4, hd=128, n_pos=700)
    check(c, base=400)


@pytest.mark.parametrize("H,Hkv,hd", [(8, 8, 64), (16, 2, 64), (16, 8, 256), (24, 4, 128)])
def test_prefill_head_geometries(H, Hkv, hd):
    c = AttnCase(H + hd, t=333, H=H, Hkv=Hkv, hd=hd, n_pos=333 + 50, q_f16=True)
    check(c, base=50, scale=1.0 / np.sqrt(hd))


@pytest.mark.parametrize("gp,H,Hkv,hd,window", [
    (gp, H, Hkv, hd, w) for (H, Hkv, hd, w) in [(16, 4, 128, 0), (16, 4, 128, 150), (8, 2, 256, 0), (16, 8, 256, 300)]
    for gp in (1, 2, 4) if (H // Hkv) % gp == 0])
def test_prefill_heads_per_workgroup(gp, H, Hkv, hd, window, tuning_env):
    """Query heads of one kv group packed into a workgroup (128 / gp rows
    each): ragged t, a window, and a ring with k_cur rows, against the oracle.
    gp takes every value in {1, 2, 4} that divides the group size."""
    tuning_env("LMX_PREFILL_GP", str(gp))
    c = AttnCase(gp * 1000 + H + hd + window, t=333, H=H, Hkv=Hkv, hd=hd, n_pos=333 + 400, q_f16=True)
    say(f"heads per workgroup gp={gp}")
    if window:
        check(c, base=400, window=window, ring=True, k_cur=True, scale=1.0 / np.sqrt(hd))
    else:
        check(c, base=400, scale=1.0 / np.sqrt(hd))


def test_gemma_swa_prefill_first_window():
    """Gemma-shape SWA layer (hd 256, w 1024, scale 1/16) in the reference's
    self-consistent regime (base + t <= window): reads the ring."""
    c = AttnCase(1024, t=1000, H=16, Hkv=8, hd=256, n_pos=1000, q_f16=True)
    check(c, base=0, window=1024, scale=1.0 / 16, ring=True)


def test_gemma_swa_prefill_4k_with_k_cur():
    """C4 SWA prefill at 4k: the batch reads its own rows via k_cur."""
    c = AttnCase(4096, t=2048, H=16, Hkv=8, hd=256, n_pos=2048, q_f16=True)
    check(c, base=0, window=1024, scale=1.0 / 16, ring=True, k_cur=True)


def test_swa_chunk_onto_ring():
    c = AttnCase(3001, t=256, H=8, Hkv=2, hd=128, n_pos=1300, q_f16=True)
    check(c, base=1044, window=300, ring=True, k_cur=True)


def test_gemma_global_prefill():
    c = AttnCase(1536, t=1536, H=16, Hkv=8, hd=256, n_pos=1536, q_f16=True)
    check(c, base=0, scale=1.0 / 16)


@pytest.mark.parametrize("window", [0, 64, 200])
@pytest.mark.parametrize("hd", [64, 128])
def test_bidirectional_prefill(window, hd):
    c = AttnCase(900 + window + hd, t=300, H=8, Hkv=4, hd=hd, n_pos=400, q_f16=True)
    check(c, base=100, window=window, bidi=True, ring=bool(window), k_cur=bool(window))


@pytest.mark.parametrize("S,base", [(8192, 0), (4096, 4096)])
def test_full_size_sampled_rows(S, base):
    """C3 at full size; 48 seeded query rows checked against the oracle."""
    say(f"full-size S={S} base={base}")
    c = AttnCase(S + base + 1, t=S, H=32, Hkv=8, hd=128, n_pos=base + S, q_f16=True, qk_norm=True)
    got = gpu_attn(c, base=base)
    rows = np.unique(np.concatenate([[0, S - 1, S // 2],
                                     np.random.default_rng(S + base).integers(0, S, 45)]))
    for i in rows:
        ref = oracle.attention(c.q[i:i + 1], c.kf, c.vf, n_heads=32, n_kv_heads=8, head_dim=128,
                               base_pos=base + int(i), n_threads=CPU_THREADS)
        assert_close(got[i:i + 1], ref, what=f"row {i}")
    # every row is a convex combination of V rows: finite and bounded by max|V|
    assert np.all(np.isfinite(got))
    assert np.abs(got).max() <= np.abs(c.vf).max() + 1e-3


@pytest.mark.parametrize("t,base", [(300, 0), (2048, 0), (64, 6000), (333, 50)])
def test_head_dim_512_prefill(t, base):
    """Gemma 4 global layers: head_dim 512, one kv head (ARCHITECTURE.md:25-28;
    attn.wgsl:44-46 takes hd <= 512).  Two waves share each 32-row block, one
    per half of the head's dims, and sum their partial scores through LDS; a
    short chunk on a long cache also takes key splits."""
    c = AttnCase(512 + t + base, t=t, H=16, Hkv=1, hd=512, n_pos=base + t, q_f16=True, qk_norm=True)
    check(c, base=base, scale=1.0 / np.sqrt(512))


def test_head_dim_512_sliding_window_with_k_cur():
    c = AttnCase(5120, t=700, H=8, Hkv=2, hd=512, n_pos=1700, q_f16=True)
    check(c, base=1000, window=512, ring=True, k_cur=True, scale=1.0 / np.sqrt(512))


@pytest.mark.parametrize("gp", [1, 2])
@pytest.mark.parametrize("mode", ["causal", "ring", "bidi"])
def test_head_dim_512_wave_pairs_heads_per_workgroup(gp, mode, tuning_env):
    """The head_dim-512 wave pairs with one or two query heads a workgroup
    (two 32-row blocks of one head, or one block of each of two heads):
    ragged t, rows before the batch, a ring read with k_cur rows, and a
    bidirectional batch (every wave meets the partial-score barrier, also on
    tiles outside its own rows' range)."""
    tuning_env("LMX_PREFILL_GP", str(gp))
    say(f"hd 512 wave pairs gp={gp} {mode}")
    c = AttnCase(700 + 10 * gp + len(mode), t=197, H=8, Hkv=2, hd=512, n_pos=197 + 300, q_f16=True,
                 qk_norm=True)
    if mode == "ring":
        check(c, base=300, window=256, ring=True, k_cur=True, scale=1.0)
    elif mode == "bidi":
        check(c, base=0, bidi=True, scale=1.0 / np.sqrt(512))
    else:
        check(c, base=300, scale=1.0 / np.sqrt(512))


@pytest.mark.parametrize("kh", ["1", "0"])
@pytest.mark.parametrize("H,Hkv,hd,t,base,window,bidi,kcur,qf16", [
    (32, 8, 128, 512, 0, 0, False, False, True),   # C3 S = 512
    (16, 4, 64, 200, 0, 0, False, False, True),
    (8, 2, 128, 333, 100, 0, False, False, False),  # a linear cache with rows before the batch
    (8, 4, 128, 300, 0, 256, False, True, True),    # a windowed first chunk, keys from k_cur
    (8, 4, 64, 250, 0, 0, True, False, True),       # bidirectional
    (16, 4, 128, 9, 0, 0, False, False, True),      # fewer rows than a tile
])
def test_key_halves_prefill(kh, H, Hkv, hd, t, base, window, bidi, kcur, qf16, tuning_env):
    """Short batches: each workgroup's two wave pairs walk the two halves of
    its key tiles and merge through LDS (kh=1), against the oracle; kh=0 is
    the one-chain kernel on the same inputs."""
    tuning_env("LMX_PREFILL_KH", kh)
    c = AttnCase(t + base + hd + window, t=t, H=H, Hkv=Hkv, hd=hd, n_pos=base + t, q_f16=qf16,
                 qk_norm=True)
    check(c, base=base, window=window, bidi=bidi, ring=kcur, k_cur=kcur)
