"""GPU parity: KV append (bit-exact f16 rows and slots), the token-sequential
and chunked delta rule, and ragged multi-sequence decode."""
import ctypes
import sys

import numpy as np
import pytest

import oracle
from tests.helpers import AttnCase, assert_close, delta_inputs

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


# ---------------------------------------------------------------- kv append --
@pytest.mark.parametrize("window,base,t,n_slots", [
    (0, 0, 1, 8), (0, 5, 17, 40), (0, 4096, 512, 4608),
    (8, 0, 5, 8), (8, 6, 5, 8), (8, 3, 21, 8), (1024, 1000, 4096, 1024),
])
def test_kv_append_matches_write_cache(window, base, t, n_slots):
    say(f"kv_append w={window} base={base} t={t} slots={n_slots}")
    kv_dim = 1024
    k = oracle.normal(window + base + t, (t, kv_dim)) * np.float32(3.0)
    v = oracle.normal(window + base + t + 1, (t, kv_dim))
    init = np.full((n_slots, kv_dim), 0x3C00, np.uint16)  # 1.0 everywhere
    ek, ev = init.copy(), init.copy()
    oracle.write_cache(k, ek, base, window)
    oracle.write_cache(v, ev, base, window)
    kc, vc = dev(init, torch.float16), dev(init, torch.float16)
    lmx.write_cache(dev(k), dev(v), kc, vc, base_pos=base, window=window)
    torch.cuda.synchronize()
    assert np.array_equal(kc.cpu().view(torch.int16).numpy().view(np.uint16), ek)
    assert np.array_equal(vc.cpu().view(torch.int16).numpy().view(np.uint16), ev)


def test_append_then_decode_matches_reference_cache_path():
    """write_cache then attention, decode step by step, equals the oracle."""
    H, Hkv, hd, n = 8, 2, 128, 40
    c = AttnCase(55, t=n, H=H, Hkv=Hkv, hd=hd, n_pos=n)
    kc = torch.zeros((n, Hkv * hd), dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    for pos in range(n):
        lmx.write_cache(dev(c.kf[pos:pos + 1]), dev(c.vf[pos:pos + 1]), kc, vc, base_pos=pos)
        out = lmx.attention(dev(c.q[pos:pos + 1]), kc, vc, n_heads=H, n_kv_heads=Hkv, head_dim=hd,
                            base_pos=pos)
        ref = oracle.attention(c.q[pos:pos + 1], c.kf, c.vf, n_heads=H, n_kv_heads=Hkv, head_dim=hd,
                               base_pos=pos)
        assert_close(out.cpu().numpy(), ref, what=f"pos {pos}")


# -------------------------------------------------------------- delta rule --
def _delta_gpu(fn, conv, al, be, S0, A, dt, n_vh, n_kh, sd, **kw):
    state = dev(S0.copy())
    out = fn(dev(conv), dev(al), dev(be), state, dev(A), dev(dt), n_vh=n_vh, n_kh=n_kh, s_dim=sd, **kw)
    torch.cuda.synchronize()
    return out.cpu().numpy(), state.cpu().numpy()


@pytest.mark.parametrize("n_vh,n_kh,sd,T,s0", [(4, 2, 64, 37, 0.0), (4, 2, 64, 5, 0.5),
                                               (32, 16, 128, 64, 0.0), (32, 16, 128, 1, 0.3),
                                               (6, 3, 128, 130, 0.1)])
def test_delta_recur(n_vh, n_kh, sd, T, s0):
    say(f"delta_recur n_vh={n_vh} n_kh={n_kh} sd={sd} T={T} s0={s0}")
    conv, al, be, S0, A, dt = delta_inputs(T + n_vh, T=T, n_vh=n_vh, n_kh=n_kh, sd=sd, s0_scale=s0)
    o_ref, S_ref = oracle.delta_recur(conv, al, be, S0, n_vh=n_vh, n_kh=n_kh, s_dim=sd)
    o, S = _delta_gpu(lmx.delta_recur, conv, al, be, S0, A, dt, n_vh, n_kh, sd)
    assert_close(o, o_ref, what="o")
    assert_close(S, S_ref, what="S")


@pytest.mark.parametrize("T,chunk", [(37, 16), (64, 64), (200, 64), (256, 32), (250, 32), (99, 32)])
def test_delta_chunked_matches_sequential(T, chunk):
    # (250, 32) and (99, 32): a ragged last chunk at C = 32, where the scan's
    # K^T operand comes from LDS rows the token waves wrote and the rows past
    # T only from zero-filled prep pieces
    n_vh, n_kh, sd = 8, 4, 128
    say(f"delta_chunked T={T} chunk={chunk}")
    conv, al, be, S0, A, dt = delta_inputs(T + 7, T=T, n_vh=n_vh, n_kh=n_kh, sd=sd, s0_scale=0.2)
    o_ref, S_ref = oracle.delta_recur(conv, al, be, S0, n_vh=n_vh, n_kh=n_kh, s_dim=sd)
    o, S = _delta_gpu(lmx.delta_chunked, conv, al, be, S0, A, dt, n_vh, n_kh, sd, chunk=chunk)
    assert_close(o, o_ref, what="o")
    assert_close(S, S_ref, what="S")


@pytest.mark.parametrize("n_vh,n_kh,T,chunk", [(4, 4, 150, 64), (12, 3, 99, 32), (8, 2, 150, 64),
                                                (6, 4, 150, 64), (2, 4, 150, 64)],
                         ids=["one_v_head_a_k_head", "three", "four", "uneven", "more_k_heads"])
def test_delta_chunked_head_ratios(n_vh, n_kh, T, chunk):
    """v-heads per k-head other than two: with one, the one-launch form shares
    no item with the scan workgroups; with three or four, a scan workgroup's
    share of a first-round item is several v-heads, each with its own flag;
    uneven (6 on 4: k-heads 0 and 1 serve two, 2 and 3 one), some scan
    workgroups' share is empty; with more k-heads than v-heads, k-heads 2 and 3
    serve none."""
    sd = 128
    say(f"delta_chunked n_vh={n_vh} n_kh={n_kh} T={T} chunk={chunk}")
    conv, al, be, S0, A, dt = delta_inputs(T + n_vh, T=T, n_vh=n_vh, n_kh=n_kh, sd=sd, s0_scale=0.2)
    o_ref, S_ref = oracle.delta_recur(conv, al, be, S0, n_vh=n_vh, n_kh=n_kh, s_dim=sd)
    o, S = _delta_gpu(lmx.delta_chunked, conv, al, be, S0, A, dt, n_vh, n_kh, sd, chunk=chunk)
    assert_close(o, o_ref, what="o")
    assert_close(S, S_ref, what="S")


# ------------------------------------------------------- ragged batch decode --
def _batched(B, lens, H=32, Hkv=8, hd=128, seed=0, q_f16=False):
    say(f"batched B={B} lens={lens}")
    cases = [AttnCase(seed + i, t=1, H=H, Hkv=Hkv, hd=hd, n_pos=int(n), q_f16=q_f16)
             for i, n in enumerate(lens)]
    max_ctx = int(max(lens))
    ks = [dev(np.pad(c.k16, ((0, max_ctx - c.n_pos), (0, 0))), torch.float16) for c in cases]
    vs = [dev(np.pad(c.v16, ((0, max_ctx - c.n_pos), (0, 0))), torch.float16) for c in cases]
    q = np.concatenate([c.q for c in cases])
    qd = dev(q.astype(np.float16)) if q_f16 else dev(q)
    caches = lmx.BatchedCaches(ks, vs)
    ctx = dev(np.array(lens, np.int32))
    out = lmx.attention_decode_batched(qd, caches, ctx, max_ctx=max_ctx, n_heads=H, n_kv_heads=Hkv,
                                       head_dim=hd)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for i, c in enumerate(cases):
        assert_close(out[i:i + 1], c.reference(base_pos=c.n_pos - 1), what=f"seq {i}")
    return out, cases, ks, vs


def test_batched_ragged_b8():
    rng = np.random.default_rng(8)
    _batched(8, rng.integers(1024, 32769, 8).tolist(), seed=100)


def test_batched_ragged_b32():
    # B = 32 takes the batch-scaled split target (8192 workgroups): 128 splits
    # per unit at an 8k longest context, merged in 16 parts
    rng = np.random.default_rng(32)
    _batched(32, rng.integers(64, 8193, 32).tolist(), seed=400)


def test_batched_small_and_f16_query():
    _batched(5, [1, 2, 64, 65, 700], seed=200, q_f16=True)


def test_batched_single_sequence_equals_attn_fwd():
    out, cases, ks, vs = _batched(1, [5000], seed=300)
    c = cases[0]
    single = lmx.attention(dev(c.q), ks[0], vs[0], n_heads=32, n_kv_heads=8, head_dim=128,
                           base_pos=4999)
    assert np.array_equal(single.cpu().numpy(), out)


def test_delta_chunked_c5_full_size_matches_sequential_kernel():
    """C5 at full size (T=4096, 32 v-heads, 16 k-heads, d=128, chunk 64): the
    chunked kernel (split-bf16 products) against the token-sequential fp32
    kernel, which the oracle pins at smaller sizes; both outputs and the final
    state within the attention tolerance."""
    n_vh, n_kh, sd, T = 32, 16, 128, 4096
    say(f"delta_chunked C5 full size T={T} n_vh={n_vh} n_kh={n_kh} vs delta_recur")
    conv, al, be, S0, A, dt = delta_inputs(4099, T=T, n_vh=n_vh, n_kh=n_kh, sd=sd, s0_scale=0.0)
    o_seq, S_seq = _delta_gpu(lmx.delta_recur, conv, al, be, S0, A, dt, n_vh, n_kh, sd)
    o_chk, S_chk = _delta_gpu(lmx.delta_chunked, conv, al, be, S0, A, dt, n_vh, n_kh, sd, chunk=64)
    e_o = assert_close(o_chk, o_seq, what="o")
    e_s = assert_close(S_chk, S_seq, what="S")
    say(f"  o max_abs={e_o[0]:.2e} rel={e_o[1]:.2e}; S max_abs={e_s[0]:.2e} rel={e_s[1]:.2e}")


@pytest.mark.parametrize("T,n_vh,n_kh,sd,chunk", [(4096, 32, 16, 128, 64), (2577, 32, 16, 128, 64),
                                                  (250, 8, 4, 64, 32), (99, 4, 2, 128, 32),
                                                  (37, 4, 2, 64, 64), (150, 4, 4, 128, 64),
                                                  (99, 12, 3, 128, 32), (150, 8, 2, 128, 64),
                                                  (150, 6, 4, 128, 64)])
def test_delta_chunked_one_launch_matches_two(T, n_vh, n_kh, sd, chunk, tuning_env):
    """The one-launch form (prep workgroups publish a ready flag per (chunk,
    v-head); scan workgroups wait for it) against prep and scan as two
    launches (LMX_DELTA_FUSED=0).  Each item and chunk runs the same
    arithmetic, so o and the state are bit-identical.  The workspace is
    filled with 0x5A bytes before each call, so its flags start nonzero: the
    call itself must clear them, and it leaves the error word (a wait that
    gave up) at 0; the two-launch form does not touch it."""
    say(f"delta_chunked one launch vs two T={T} n_vh={n_vh} n_kh={n_kh} sd={sd} chunk={chunk}")
    conv, al, be, S0, A, dt = delta_inputs(T + 5, T=T, n_vh=n_vh, n_kh=n_kh, sd=sd, s0_scale=0.1)
    n_ch = -(-T // chunk)
    err_at = 4 * (n_vh * n_ch * (2 * chunk * chunk + 2 * chunk) + n_kh * n_ch * 2 * chunk * sd + n_vh * n_ch)
    op = lmx.dop(n_tok=T, n_vh=n_vh, n_kh=n_kh, s_dim=sd)
    ws = lmx.Workspace(lmx.lib().lmx_deltanet_chunked_workspace_bytes(ctypes.byref(op), chunk),
                       device=torch.device("cuda"))
    base = ws.base - ws.buf.data_ptr()
    runs = {}
    for fused in ("1", "0"):
        tuning_env("LMX_DELTA_FUSED", fused)
        ws.buf.fill_(0x5A)
        state = dev(S0.copy())
        out = lmx.delta_chunked(dev(conv), dev(al), dev(be), state, dev(A), dev(dt), n_vh=n_vh, n_kh=n_kh,
                                s_dim=sd, chunk=chunk, workspace=ws)
        torch.cuda.synchronize()
        err = int(ws.buf[base + err_at:base + err_at + 4].cpu().numpy().view(np.uint32)[0])
        runs[fused] = (out.cpu().numpy(), state.cpu().numpy(), err)
    assert runs["1"][2] == 0, "a scan workgroup gave up waiting for a ready flag"
    assert runs["0"][2] == 0x5A5A5A5A
    np.testing.assert_array_equal(runs["1"][0], runs["0"][0])
    np.testing.assert_array_equal(runs["1"][1], runs["0"][1])


def test_delta_chunked_flag_wait_gives_up(tuning_env):
    """The one-launch form's waits are bounded.  LMX_DELTA_FUSED=starve (tests
    only) launches it with no prep workgroups and a 64-poll bound: every scan
    workgroup's first wait gives up, records it in the error word and lets the
    workgroup finish, so the call returns (its results are meaningless).  A
    normal call on the same workspace afterwards is correct again."""
    T, n_vh, n_kh, sd, chunk = 200, 4, 2, 128, 64
    say("delta_chunked flag wait gives up (no prep workgroups)")
    conv, al, be, S0, A, dt = delta_inputs(T + 9, T=T, n_vh=n_vh, n_kh=n_kh, sd=sd, s0_scale=0.1)
    n_ch = -(-T // chunk)
    err_at = 4 * (n_vh * n_ch * (2 * chunk * chunk + 2 * chunk) + n_kh * n_ch * 2 * chunk * sd + n_vh * n_ch)
    op = lmx.dop(n_tok=T, n_vh=n_vh, n_kh=n_kh, s_dim=sd)
    ws = lmx.Workspace(lmx.lib().lmx_deltanet_chunked_workspace_bytes(ctypes.byref(op), chunk),
                       device=torch.device("cuda"))
    base = ws.base - ws.buf.data_ptr()

    def run():
        state = dev(S0.copy())
        out = lmx.delta_chunked(dev(conv), dev(al), dev(be), state, dev(A), dev(dt), n_vh=n_vh, n_kh=n_kh,
                                s_dim=sd, chunk=chunk, workspace=ws)
        torch.cuda.synchronize()
        err = int(ws.buf[base + err_at:base + err_at + 4].cpu().numpy().view(np.uint32)[0])
        return out.cpu().numpy(), state.cpu().numpy(), err

    tuning_env("LMX_DELTA_FUSED", "starve")
    assert run()[2] == 1
    tuning_env("LMX_DELTA_FUSED", "1")
    o, S, err = run()
    assert err == 0
    o_ref, S_ref = oracle.delta_recur(conv, al, be, S0, n_vh=n_vh, n_kh=n_kh, s_dim=sd)
    assert_close(o, o_ref, what="o")
    assert_close(S, S_ref, what="S")


@pytest.mark.parametrize("T", [2577, 6400])
def test_delta_chunked_prep_items_per_workgroup(T):
    """The chunk prep walks (chunk, k-head) items with a stride of its grid
    (at most 512 workgroups) and prefetches each next item's rows: T=2577
    gives 656 items (some workgroups take two, the rest one, and the last
    chunk is ragged), T=6400 gives 1600 (three or four each).  Against the
    token-sequential kernel, with a nonzero initial state."""
    n_vh, n_kh, sd = 32, 16, 128
    say(f"delta_chunked prep items T={T} items={-(-T // 64) * n_kh}")
    conv, al, be, S0, A, dt = delta_inputs(T + 11, T=T, n_vh=n_vh, n_kh=n_kh, sd=sd, s0_scale=0.1)
    o_seq, S_seq = _delta_gpu(lmx.delta_recur, conv, al, be, S0, A, dt, n_vh, n_kh, sd)
    o_chk, S_chk = _delta_gpu(lmx.delta_chunked, conv, al, be, S0, A, dt, n_vh, n_kh, sd, chunk=64)
    e_o = assert_close(o_chk, o_seq, what="o")
    e_s = assert_close(S_chk, S_seq, what="S")
    say(f"  o max_abs={e_o[0]:.2e} rel={e_o[1]:.2e}; S max_abs={e_s[0]:.2e} rel={e_s[1]:.2e}")
