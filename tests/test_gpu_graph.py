"""GPU: the entry points replayed from a captured HIP graph.

A serving loop captures its decode step once and replays it; the library's
launches are stream-ordered, allocate nothing and clear workspace flags with a
kernel (no hipMemsetAsync node).  Each case runs eagerly for the expected
result, is captured, and is replayed three times with other eager work of the
same entry point (on other inputs) and a device sync between replays; every
replay must reproduce the eager output bit for bit (same kernels, same
arguments, fixed reduction order).
"""
import sys

import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import llmoxide_amd as lmx  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def replay_check(run, reset=None, other=None, outs=()):
    """run() launches the case; outs are the tensors it writes.  reset()
    restores in-place state before each run; other() is unrelated eager work."""
    if reset:
        reset()
    run()
    torch.cuda.synchronize()
    want = [o.clone() for o in outs]
    g = torch.cuda.CUDAGraph()
    if reset:
        reset()
    with torch.cuda.graph(g):
        run()
    torch.cuda.synchronize()
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        if reset:
            reset()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (o, w) in enumerate(zip(outs, want)):
            assert torch.equal(o, w), f"replay {rep}, output {i} differs from the eager run"
        if other:
            other()
        torch.cuda.synchronize()
    del g


def test_graph_decode_split_merge():
    say("case graph decode H=32 Hkv=8 hd=128 ctx=4096 (split + merge)")
    g = torch.Generator(device="cuda").manual_seed(3)
    n = 4096
    k = torch.randn((n, 1024), generator=g, device="cuda").half()
    v = torch.randn((n, 1024), generator=g, device="cuda").half()
    q = torch.randn((1, 32 * 128), generator=g, device="cuda")
    q2 = torch.randn((1, 32 * 128), generator=g, device="cuda")
    out = torch.empty((1, 32 * 128), device="cuda")
    out2 = torch.empty_like(out)
    ws = lmx.Workspace()
    kw = dict(n_heads=32, n_kv_heads=8, head_dim=128, base_pos=n - 1, workspace=ws)
    replay_check(lambda: lmx.attention(q, k, v, out=out, **kw),
                 other=lambda: lmx.attention(q2, k, v, out=out2, **kw), outs=[out])


def test_graph_decode_batched():
    say("case graph batched decode B=3 ragged (700, 3000, 1500)")
    g = torch.Generator(device="cuda").manual_seed(4)
    lens = [700, 3000, 1500]
    ks = [torch.randn((m, 1024), generator=g, device="cuda").half() for m in lens]
    vs = [torch.randn((m, 1024), generator=g, device="cuda").half() for m in lens]
    caches = lmx.BatchedCaches(ks, vs)
    q = torch.randn((3, 32 * 128), generator=g, device="cuda")
    ctx = torch.tensor(lens, dtype=torch.int32, device="cuda")
    out = torch.empty((3, 32 * 128), device="cuda")
    out2 = torch.empty_like(out)
    ws = lmx.Workspace()
    kw = dict(max_ctx=3000, n_heads=32, n_kv_heads=8, head_dim=128, n_slots=3000, workspace=ws)
    replay_check(lambda: lmx.attention_decode_batched(q, caches, ctx, out=out, **kw),
                 other=lambda: lmx.attention_decode_batched(q * 0.5, caches, ctx, out=out2, **kw),
                 outs=[out])


def test_graph_prefill_key_splits():
    say("case graph prefill chunk 128 on a 2048 cache (key splits + merge)")
    g = torch.Generator(device="cuda").manual_seed(5)
    base, t = 2048, 128
    k = torch.randn((base + t, 1024), generator=g, device="cuda").half()
    v = torch.randn((base + t, 1024), generator=g, device="cuda").half()
    q = torch.randn((t, 32 * 128), generator=g, device="cuda").half()
    out = torch.empty((t, 32 * 128), device="cuda")
    out2 = torch.empty_like(out)
    ws = lmx.Workspace()
    kw = dict(n_heads=32, n_kv_heads=8, head_dim=128, base_pos=base, workspace=ws)
    replay_check(lambda: lmx.attention(q, k, v, out=out, **kw),
                 other=lambda: lmx.attention(q * 0.5, k, v, out=out2, **kw), outs=[out])


@pytest.mark.parametrize("T,n_vh,n_kh", [(200, 4, 2), (4096, 32, 16)], ids=["small", "c5"])
def test_graph_delta_chunked(T, n_vh, n_kh):
    """The chunked delta rule captured and replayed: at C5 size its one-launch
    form (256 prep beside 256 scan workgroups, after the flag-clearing
    kernel) runs in the graph."""
    say(f"case graph delta chunked T={T} Hv={n_vh} Hk={n_kh} d=128")
    g = torch.Generator(device="cuda").manual_seed(6)
    sd = 128
    conv = torch.randn((T, 2 * n_kh * sd + n_vh * sd), generator=g, device="cuda")
    qk = conv[:, :2 * n_kh * sd].view(T, 2 * n_kh, sd)
    qk /= qk.norm(dim=-1, keepdim=True)
    al = torch.randn((T, n_vh), generator=g, device="cuda")
    be = torch.randn((T, n_vh), generator=g, device="cuda")
    A = torch.full((n_vh,), -1.0, device="cuda")
    dt = torch.zeros(n_vh, device="cuda")
    S0 = torch.randn((n_vh, sd, sd), generator=g, device="cuda") * 0.1
    state = torch.empty_like(S0)
    state2 = torch.empty_like(S0)
    out = torch.empty((T, n_vh * sd), device="cuda")
    out2 = torch.empty_like(out)
    ws = lmx.Workspace()
    kw = dict(n_vh=n_vh, n_kh=n_kh, s_dim=sd, chunk=64, workspace=ws)

    def other():
        state2.copy_(S0)
        lmx.delta_chunked(conv, al * 0.5, be, state2, A, dt, out=out2, **kw)

    replay_check(lambda: lmx.delta_chunked(conv, al, be, state, A, dt, out=out, **kw),
                 reset=lambda: state.copy_(S0), other=other, outs=[out, state])
