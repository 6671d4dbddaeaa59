"""The KV manager on the GPU: several sequences' caches in one arena, filled
through the manager's per-layer pointers with lmx_kv_append, a ragged decode
step through lmx_attn_decode_batched on the manager's batch tables, against
the oracle's attention for each sequence on its own (cpu.rs:342-387), plus
the session's turn logic (session.rs:546-570): a prompt that extends the
resident ids reuses them, an unrelated one wipes the sequence's caches."""
import sys

import numpy as np
import pytest

import oracle
from tests.helpers import assert_close

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import llmoxide_amd as lmx  # noqa: E402

H, HKV, HD = 16, 8, 128
KV = HKV * HD
LAYERS = [(0, KV, -1), (64, KV, -1), (64, KV, 1)]  # global, ring 64, sharing the ring
N_CTX = 600


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class Seq:
    """One sequence's K/V rows by absolute position, as f32 and as the f16 values stored."""

    def __init__(self, seed, n):
        self.k = oracle.normal(seed * 10 + 1, (N_CTX, KV))
        self.v = oracle.normal(seed * 10 + 2, (N_CTX, KV))
        self.kf = oracle.from_f16_bits(oracle.to_f16_bits(self.k))
        self.vf = oracle.from_f16_bits(oracle.to_f16_bits(self.v))
        self.tokens = [int(x) for x in (seed * 1000 + np.arange(n))]


def append(m, s, seq, lo, hi):
    for layer in (0, 1):
        k, v = m.layer_tensors(s, layer)
        _, _, _, w = m.layer_cache(s, layer)
        lmx.write_cache(torch.from_numpy(seq.k[lo:hi]).cuda(), torch.from_numpy(seq.v[lo:hi]).cuda(),
                        k, v, base_pos=lo, window=w)


def decode_step(m, handles, seqs, layer, seed):
    """Append each sequence's next row, then one batched decode on `layer`."""
    for s, seq in zip(handles, seqs):
        n = m.len(s)
        append(m, s, seq, n, n + 1)
    kp, vp, ctx, mx = m.batch(layer, handles, extra=1)
    _, _, slots, w = m.layer_cache(handles[0], layer)
    q = oracle.normal(seed, (len(handles), H * HD))
    out = lmx.attention_decode_batched(
        torch.from_numpy(q).cuda(), lmx.BatchedCaches.from_addresses(kp, vp),
        torch.tensor(ctx, dtype=torch.int32, device="cuda"), max_ctx=mx, n_heads=H,
        n_kv_heads=HKV, head_dim=HD, window=w, n_slots=slots)
    torch.cuda.synchronize()
    for b, (seq, c) in enumerate(zip(seqs, ctx)):
        ref = oracle.attention(q[b:b + 1], seq.kf, seq.vf, n_heads=H, n_kv_heads=HKV, head_dim=HD,
                               base_pos=c - 1, window=w)
        assert_close(out[b:b + 1].cpu().numpy(), ref, what=f"seq {b} layer {layer}")
    return ctx


def test_ragged_decode_through_the_manager():
    say("kvm ragged decode")
    m = lmx.KvManager(LAYERS, n_ctx=N_CTX, max_seqs=4)
    lens = (130, 7, 300)
    seqs = [Seq(i + 1, n) for i, n in enumerate(lens)]
    handles = [m.open() for _ in seqs]
    for s, seq in zip(handles, seqs):
        assert m.begin(s, seq.tokens) == 0            # nothing resident yet
        append(m, s, seq, 0, len(seq.tokens))
        m.commit(s, seq.tokens)
    # one decode step: the new rows go to every layer, then the global layer attends
    ctx = decode_step(m, handles, seqs, 0, seed=90)
    assert ctx == [131, 8, 301]
    # the ring layer (window 64) over the same step, read through layer 2, which
    # shares layer 1's cache: its tables point at layer 1's blocks
    assert m.batch(2, handles, extra=1)[:2] == m.batch(1, handles, extra=1)[:2]
    kp, vp, ctx2, mx = m.batch(2, handles, extra=1)
    assert ctx2 == ctx
    for s in handles:
        m.commit(s, [7])
    # a second step on the ring layer after the commits (positions past the window)
    assert decode_step(m, handles, seqs, 1, seed=95) == [132, 9, 302]


def test_turns_reuse_or_wipe():
    say("kvm turns")
    m = lmx.KvManager(LAYERS, n_ctx=N_CTX, max_seqs=2)
    seq = Seq(7, 40)
    s = m.open()
    m.begin(s, seq.tokens[:30])
    append(m, s, seq, 0, 30)
    m.commit(s, seq.tokens[:30])
    # the next turn extends what is resident: positions [30, 40) only
    assert m.begin(s, seq.tokens) == 30
    append(m, s, seq, 30, 40)
    m.commit(s, seq.tokens[30:])
    assert m.len(s) == 40
    decode_step(m, [s], [seq], 0, seed=96)
    m.commit(s, [1])
    # an unrelated prompt: the sequence's caches are overwritten with zeros
    assert m.begin(s, [5, 6, 7]) == 0
    torch.cuda.synchronize()
    assert m.len(s) == 0
    for layer in (0, 1):
        k, v = m.layer_tensors(s, layer)
        assert not k.any().item() and not v.any().item()
