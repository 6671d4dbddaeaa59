"""GPU parity: split-K decode attention (few query tokens) vs the C oracle.

Tolerance: max abs error <= 2e-3 and max|diff|/max|ref| <= 1e-2 on the fp32
outputs (tests/helpers.py), with f16 K/V and the oracle reading the identical
f16 values upcast to f32.
"""
import sys

import numpy as np
import pytest

from tests.helpers import AttnCase, assert_close

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import llmoxide_amd as lmx  # noqa: E402


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.cuda()


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def run_case(c: AttnCase, *, base, window=0, bidi=False, scale=None, ring=False, k_cur=False):
    say(f"case t={c.t} H={c.H} Hkv={c.Hkv} hd={c.hd} base={base} w={window} bidi={bidi} "
        f"ring={ring} k_cur={k_cur} q_f16={c.q_f16}")
    end = base + c.t
    if ring:
        kc, vc = c.ring(window, end if not k_cur else base)
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
    ref = c.reference(base_pos=base, window=window, bidi=bidi, scale=scale)
    return assert_close(out.cpu().numpy(), ref, what="decode")


def test_c1_config():
    """C1: H=16, Hkv=8, hd=128, 512 cached tokens, query at pos 511, f32 Q."""
    c = AttnCase(1, t=1, H=16, Hkv=8, hd=128, n_pos=512)
    run_case(c, base=511)


@pytest.mark.parametrize("ctx", [1, 2, 63, 64, 65, 257, 1000, 4097, 12345, 32768])
def test_qwen3_8b_shape_decode(ctx):
    c = AttnCase(ctx, t=1, H=32, Hkv=8, hd=128, n_pos=ctx)
    run_case(c, base=ctx - 1)


def test_f16_query():
    c = AttnCase(3, t=1, H=32, Hkv=8, hd=128, n_pos=3000, q_f16=True)
    run_case(c, base=2999)


@pytest.mark.parametrize("H,Hkv,hd", [(8, 8, 128), (16, 2, 128), (24, 4, 128), (16, 1, 64),
                                      (8, 2, 64), (16, 8, 256), (4, 1, 512), (16, 1, 512)])
def test_head_geometries(H, Hkv, hd):
    c = AttnCase(H * 7 + hd, t=1, H=H, Hkv=Hkv, hd=hd, n_pos=2500)
    run_case(c, base=2499, scale=1.0 / np.sqrt(hd))


def test_padded_kv_rows():
    c = AttnCase(8, t=1, H=8, Hkv=2, hd=128, n_pos=700, kv_dim=2 * 128 + 64)
    run_case(c, base=699)


@pytest.mark.parametrize("window,ctx", [(4, 37), (7, 1000), (1024, 1500), (1024, 32768), (100, 100)])
def test_ring_window_decode(window, ctx):
    """Sliding-window decode from a ring cache (Gemma SWA layers, scale 1/16)."""
    c = AttnCase(window + ctx, t=1, H=16, Hkv=8, hd=256, n_pos=ctx)
    run_case(c, base=ctx - 1, window=window, scale=1.0 / 16, ring=True)


@pytest.mark.parametrize("t,base", [(2, 0), (5, 300), (8, 4095)])
def test_few_tokens_causal(t, base):
    c = AttnCase(t + base, t=t, H=32, Hkv=8, hd=128, n_pos=base + t)
    run_case(c, base=base)


@pytest.mark.parametrize("window", [0, 3, 16])
def test_few_tokens_bidi(window):
    c = AttnCase(40 + window, t=6, H=8, Hkv=2, hd=64, n_pos=50)
    run_case(c, base=44, window=window, bidi=True, k_cur=bool(window), ring=bool(window))


def test_windowed_batch_with_k_cur():
    """A windowed batch past the ring's self-consistent regime reads its own
    rows from k_cur/v_cur and earlier positions from the ring."""
    c = AttnCase(91, t=7, H=8, Hkv=4, hd=128, n_pos=60)
    run_case(c, base=53, window=16, ring=True, k_cur=True)


def test_ring_hazard_is_refused():
    c = AttnCase(92, t=7, H=8, Hkv=4, hd=128, n_pos=60)
    kc, vc = c.ring(16, 60)
    with pytest.raises(lmx.LmxError) as e:
        lmx.attention(dev(c.q), dev(kc, torch.float16), dev(vc, torch.float16), n_heads=8,
                      n_kv_heads=4, head_dim=128, base_pos=53, window=16)
    assert e.value.status == lmx.Status.E_RING_HAZARD


def test_repeat_calls_reuse_workspace():
    """Counters are left at zero, so back-to-back calls on one workspace agree."""
    c = AttnCase(17, t=1, H=32, Hkv=8, hd=128, n_pos=20000)
    ws = lmx.Workspace()
    q = dev(c.q)
    kc, vc = dev(c.k16, torch.float16), dev(c.v16, torch.float16)
    outs = [lmx.attention(q, kc, vc, n_heads=32, n_kv_heads=8, head_dim=128, base_pos=19999,
                          workspace=ws).cpu().numpy() for _ in range(5)]
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])
    assert_close(outs[0], c.reference(base_pos=19999))


def test_workspace_reuse_with_different_inputs():
    """Split partials cross workgroups through the workspace: alternating two
    different inputs on one workspace must give each input's own result
    (stale partials from the previous call would show up here)."""
    ws = lmx.Workspace()
    cases = [AttnCase(s, t=1, H=32, Hkv=8, hd=128, n_pos=9000) for s in (21, 22)]
    dev_in = [(dev(c.q), dev(c.k16, torch.float16), dev(c.v16, torch.float16)) for c in cases]
    refs = [c.reference(base_pos=8999) for c in cases]
    for rep in range(3):
        for i, (q, kc, vc) in enumerate(dev_in):
            say(f"workspace reuse rep={rep} case={i}")
            out = lmx.attention(q, kc, vc, n_heads=32, n_kv_heads=8, head_dim=128, base_pos=8999,
                                workspace=ws)
            torch.cuda.synchronize()
            assert_close(out.cpu().numpy(), refs[i], what=f"rep {rep} case {i}")


@pytest.mark.parametrize("ctx", [16, 17, 127, 128, 129, 1023, 2047, 2049])
def test_tile_and_split_edges(ctx):
    """Context lengths around the 16-key tile and the split boundaries."""
    c = AttnCase(ctx + 5, t=1, H=32, Hkv=8, hd=128, n_pos=ctx)
    run_case(c, base=ctx - 1)


def test_one_workspace_serves_every_entry_point():
    """Split-K decode, a key-split prefill and the chunked delta rule keep
    different scratch layouts in the workspace.  Interleaving the three (and
    a second decode shape) on one workspace must give each its oracle
    result: no call may read what another call's layout left there."""
    import oracle
    from tests.helpers import delta_inputs

    ws = lmx.Workspace()
    dec = AttnCase(31, t=1, H=32, Hkv=8, hd=128, n_pos=6000)
    gem = AttnCase(32, t=1, H=16, Hkv=8, hd=256, n_pos=3000)
    pre = AttnCase(33, t=64, H=32, Hkv=8, hd=128, n_pos=2112)
    d_in = [(dev(c.q), dev(c.k16, torch.float16), dev(c.v16, torch.float16)) for c in (dec, gem, pre)]
    refs = [dec.reference(base_pos=5999), gem.reference(base_pos=2999), pre.reference(base_pos=2048)]
    conv, al, be, S0, A, dt = delta_inputs(34, T=100, n_vh=4, n_kh=2, sd=128)
    o_ref, S_ref = oracle.delta_recur(conv, al, be, S0, n_vh=4, n_kh=2, s_dim=128)
    geo = [dict(n_heads=32, n_kv_heads=8, head_dim=128, base_pos=5999),
           dict(n_heads=16, n_kv_heads=8, head_dim=256, base_pos=2999),
           dict(n_heads=32, n_kv_heads=8, head_dim=128, base_pos=2048)]
    for rep in range(2):
        for i in (0, 2, 1, 0):
            say(f"shared workspace rep={rep} attention case {i}")
            q, kc, vc = d_in[i]
            if i == 2:
                out = lmx.attention(q, kc, vc, k_cur=kc[2048:], v_cur=vc[2048:], workspace=ws, **geo[i])
            else:
                out = lmx.attention(q, kc, vc, workspace=ws, **geo[i])
            torch.cuda.synchronize()
            assert_close(out.cpu().numpy(), refs[i], what=f"rep {rep} case {i}")
        say(f"shared workspace rep={rep} delta chunked")
        state = dev(S0.copy())
        o = lmx.delta_chunked(dev(conv), dev(al), dev(be), state, dev(A), dev(dt), n_vh=4, n_kh=2,
                              s_dim=128, chunk=64, workspace=ws)
        torch.cuda.synchronize()
        assert_close(o.cpu().numpy(), o_ref, what="delta o")
        assert_close(state.cpu().numpy().ravel(), S_ref, what="delta S")


@pytest.mark.parametrize("H,Hkv,hd,ctx,window,t,q_f16", [
    (32, 8, 128, 32768, 0, 1, False), (32, 8, 128, 700, 0, 1, True), (32, 8, 128, 1500, 1024, 1, False),
    (32, 8, 128, 3000, 0, 4, False),
    (16, 8, 256, 1500, 1024, 1, True), (16, 8, 256, 5000, 0, 1, False), (16, 8, 256, 900, 0, 3, True)])
def test_k_operand_paths(H, Hkv, hd, ctx, window, t, q_f16, tuning_env):
    """K tiles both ways (head_dim 128 and 256), forced: loaded row-major and
    turned into MFMA operands through LDS, or each lane's operand bytes loaded
    directly.  The operands are the same, so the outputs are the same bits."""
    c = AttnCase(ctx + t + hd, t=t, H=H, Hkv=Hkv, hd=hd, n_pos=ctx, q_f16=q_f16)
    base = ctx - t
    kc, vc = c.ring(window, ctx) if window else (c.k16, c.v16)
    q = dev(c.q.astype(np.float16)) if q_f16 else dev(c.q)
    kd, vd = dev(kc, torch.float16), dev(vc, torch.float16)
    ref = c.reference(base_pos=base, window=window)
    outs = []
    for krows in ("0", "1"):
        tuning_env("LMX_DECODE_KROWS", krows)
        say(f"K operand path krows={krows} ctx={ctx} w={window} t={t}")
        out = lmx.attention(q, kd, vd, n_heads=H, n_kv_heads=Hkv, head_dim=hd, base_pos=base, window=window)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
        assert_close(outs[-1], ref, what=f"krows={krows}")
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("H,Hkv,ctx,window,t,q_f16,k_cur", [
    (16, 1, 32768, 0, 1, False, False),   # Gemma 4 global layer at 32k, fp32 q (two column blocks)
    (16, 1, 5000, 0, 1, True, False),     # f16 q (one column block)
    (32, 2, 3000, 0, 2, False, False),    # two kv heads, two query rows
    (64, 2, 2500, 0, 1, False, False),    # two 16-head blocks a kv head
    (16, 1, 70, 0, 1, False, False),      # one split: the kernel writes the output itself
    (16, 1, 2000, 512, 1, False, False),  # a ring (general addressing)
    (16, 1, 900, 256, 3, True, True),     # a windowed batch whose rows come from k_cur
])
def test_many_heads_decode_hd512(H, Hkv, ctx, window, t, q_f16, k_cur, tuning_env):
    """head_dim 512 with 16 query heads a kv head: attn_decode_mh_kernel (both
    products on the matrix cores, all heads on one read of each row) against
    the oracle, and against attn_decode_kernel (LMX_DECODE_MH=0) on the same
    inputs."""
    c = AttnCase(ctx + 31 * t + H + window, t=t, H=H, Hkv=Hkv, hd=512, n_pos=ctx, q_f16=q_f16, qk_norm=True)
    base = ctx - t
    outs = []
    for mh in ("1", "0"):
        tuning_env("LMX_DECODE_MH", mh)
        say(f"hd 512 decode mh={mh} H={H} Hkv={Hkv} ctx={ctx} w={window} t={t} q_f16={q_f16} k_cur={k_cur}")
        outs.append(run_case(c, base=base, window=window, ring=bool(window), k_cur=k_cur, scale=1.0))
    say(f"  mh max_abs={outs[0][0]:.2e} / attn_decode_kernel {outs[1][0]:.2e}")


def test_many_heads_decode_hd512_gate_and_batched():
    """The output gate on both of the mh kernel's write paths (its own, with
    one split, and the merge's), and ragged batched decode at head_dim 512
    with 16 heads on one kv head."""
    H, Hkv, hd = 16, 1, 512
    for ctx in (60, 4000):
        c = AttnCase(ctx + 5, t=1, H=H, Hkv=Hkv, hd=hd, n_pos=ctx, qk_norm=True)
        gate = np.random.default_rng(ctx).standard_normal((1, H * hd)).astype(np.float32)
        out = lmx.attention(dev(c.q), dev(c.k16, torch.float16), dev(c.v16, torch.float16), n_heads=H,
                            n_kv_heads=Hkv, head_dim=hd, base_pos=ctx - 1, scale=1.0, gate=dev(gate))
        torch.cuda.synchronize()
        ref = c.reference(base_pos=ctx - 1, scale=1.0) / (1.0 + np.exp(-gate.astype(np.float64)))
        assert_close(out.cpu().numpy(), ref, what=f"gated hd 512 ctx {ctx}")
    lens = [33, 700, 4096, 1999]
    ks, vs, qs, refs = [], [], [], []
    for i, n in enumerate(lens):
        c = AttnCase(900 + i, t=1, H=H, Hkv=Hkv, hd=hd, n_pos=n, qk_norm=True)
        refs.append(c.reference(base_pos=n - 1, scale=1.0))
        qs.append(c.q)
        ks.append(dev(c.k16, torch.float16))
        vs.append(dev(c.v16, torch.float16))
    max_ctx = max(lens)
    out = lmx.attention_decode_batched(dev(np.concatenate(qs)), lmx.BatchedCaches(ks, vs),
                                       dev(np.array(lens, np.int32)), max_ctx=max_ctx, n_heads=H,
                                       n_kv_heads=Hkv, head_dim=hd, n_slots=max_ctx, scale=1.0)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for i, n in enumerate(lens):
        assert_close(got[i:i + 1], refs[i], what=f"batched hd 512 seq {i} ctx {n}")
