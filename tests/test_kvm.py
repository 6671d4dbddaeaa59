"""The multi-sequence KV manager's bookkeeping (lmx_kvm_*), on the CPU with a
caller-owned arena address that is never dereferenced.  What is pinned, and
against which reference code:
  * sizing: config.rs:279-293 (kv_slots = min(window, n_ctx) for a ring,
    n_ctx for a global layer; bytes = slots * kv_dim * 2 (K, V) * 2 (f16) per
    owning layer; sharing layers allocate nothing), cache.rs:86-104;
  * prefix reuse: session.rs:497-513, enumerated against a brute-force
    restatement of its rule over all short token lists;
  * write position: cache.rs:146-149 (truncate), session.rs:568-571, 607-609
    (what becomes resident, embedding spans end comparability)."""
import ctypes
import itertools

import pytest

import llmoxide_amd as lmx

ARENA = 0x1000000  # 256-byte aligned, never dereferenced in these tests
BIG = 1 << 40


def manager(layers, n_ctx=300, max_seqs=3, arena_bytes=BIG):
    return lmx.KvManager(layers, n_ctx=n_ctx, max_seqs=max_seqs, arena=(ARENA, arena_bytes))


# Gemma-like: global, ring 1024, ring 64, a layer sharing layer 0's cache, a
# layer sharing the ring-64 layer's.
GEMMA_LIKE = [(0, 2048, -1), (1024, 2048, -1), (64, 1024, -1), (0, 2048, 0), (64, 1024, 2)]


def kv_bytes(layers, n_ctx):  # config.rs:286-293
    return sum((min(w, n_ctx) if w else n_ctx) * d * 2 * 2 for (w, d, s) in layers if s < 0)


@pytest.mark.parametrize("n_ctx", [300, 1024, 5000])
def test_arena_is_kv_bytes_per_sequence(n_ctx):
    m = manager(GEMMA_LIKE, n_ctx=n_ctx, max_seqs=4)
    assert m.arena_bytes == 4 * kv_bytes(GEMMA_LIKE, n_ctx)


def test_slots_windows_and_sharing():
    m = manager(GEMMA_LIKE, n_ctx=300)
    s = m.open()
    k0, v0, n0, w0 = m.layer_cache(s, 0)
    assert (n0, w0) == (300, 0)                       # global: n_ctx slots, linear
    assert m.layer_cache(s, 1)[2:] == (300, 300)      # ring 1024 clamps to n_ctx (config.rs:281)
    assert m.layer_cache(s, 2)[2:] == (64, 64)        # ring of the window
    assert m.layer_cache(s, 3) == (k0, v0, n0, w0)    # shares layer 0 (cache.rs:97-103)
    assert m.layer_cache(s, 4) == m.layer_cache(s, 2)


def test_blocks_are_aligned_disjoint_and_inside_the_arena():
    m = manager(GEMMA_LIKE, n_ctx=300, max_seqs=3)
    spans = []
    for _ in range(3):
        s = m.open()
        for layer in (0, 1, 2):
            k, v, slots, _ = m.layer_cache(s, layer)
            d = GEMMA_LIKE[layer][1]
            for a in (k, v):
                assert a % 256 == 0
                spans.append((a, a + slots * d * 2))
    spans.sort()
    assert spans[0][0] >= ARENA and spans[-1][1] <= ARENA + m.arena_bytes
    for (a0, a1), (b0, _) in zip(spans, spans[1:]):
        assert a1 <= b0


def reuse_rule(cached, comparable, prompt):  # session.rs:497-513, restated
    if not comparable:
        return 0
    n = 0
    while n < min(len(cached), len(prompt)) and cached[n] == prompt[n]:
        n += 1
    return n if n == len(cached) and n < len(prompt) else 0


def test_reusable_prefix_reference_cases():
    m = manager([(0, 8, -1)])
    s = m.open()
    assert m.reusable_prefix(s, [1, 2]) == 0          # nothing resident
    m.commit(s, [1, 2, 3])
    assert m.reusable_prefix(s, [1, 2, 3, 4]) == 3    # strictly extends: reuse all
    assert m.reusable_prefix(s, [1, 2, 3]) == 0       # not longer than resident
    assert m.reusable_prefix(s, [1, 2, 9, 4]) == 0    # diverges: no rewind
    assert m.reusable_prefix(s, [1, 2]) == 0          # shorter


def test_reusable_prefix_matches_the_rule_exhaustively():
    m = manager([(0, 8, -1)], max_seqs=1)
    toks = [1, 2]
    for nc in range(4):
        for cached in itertools.product(toks, repeat=nc):
            s = m.open()
            m.commit(s, list(cached))
            for npr in range(5):
                for prompt in itertools.product(toks, repeat=npr):
                    assert m.reusable_prefix(s, list(prompt)) == reuse_rule(cached, True, prompt)
            m.close(s)


def test_embedding_rows_end_reuse_and_truncate_drops_the_tail():
    m = manager([(0, 8, -1)])
    s = m.open()
    m.commit(s, [5, 6, 7])
    m.truncate(s, 2)                                  # cache.rs:146-149
    assert m.len(s) == 2
    assert m.reusable_prefix(s, [5, 6, 9]) == 2       # the dropped id no longer counts
    m.truncate(s, 10)
    assert m.len(s) == 2                              # truncate never grows
    m.commit(s, None, n=4)                            # an embedding span (session.rs:569-571)
    assert m.len(s) == 6
    assert m.reusable_prefix(s, [5, 6, 1, 1, 1, 1, 1]) == 0
    m.close(s)
    s = m.open()
    assert m.len(s) == 0 and m.reusable_prefix(s, [5]) == 0


def test_context_limits():
    m = manager([(0, 8, -1)], n_ctx=10)
    s = m.open()
    m.commit(s, list(range(9)))
    with pytest.raises(lmx.LmxError) as e:
        m.commit(s, [1, 2])
    assert e.value.status == lmx.Status.E_CONTEXT
    # rejected before any device work (the null stream is never used)
    arr = (ctypes.c_int32 * 11)(*range(11))
    r = ctypes.c_uint32()
    assert lmx.lib().lmx_kvm_begin(m.h, s, arr, 11, ctypes.byref(r), None) == lmx.Status.E_CONTEXT
    with pytest.raises(lmx.LmxError) as e:
        m.batch(0, [s], extra=2)
    assert e.value.status == lmx.Status.E_CONTEXT
    assert m.batch(0, [s], extra=1)[2:] == ([10], 10)


def test_sequence_slots():
    m = manager([(0, 8, -1)], max_seqs=2)
    a, b = m.open(), m.open()
    assert {a, b} == {0, 1}
    with pytest.raises(lmx.LmxError) as e:
        m.open()
    assert e.value.status == lmx.Status.E_FULL
    m.close(a)
    assert m.open() == a
    with pytest.raises(lmx.LmxError) as e:
        m.len(7)
    assert e.value.status == lmx.Status.E_SHAPE


def test_batch_tables():
    m = manager(GEMMA_LIKE, n_ctx=300)
    seqs = [m.open() for _ in range(3)]
    for s, n in zip(seqs, (5, 0, 17)):
        m.commit(s, list(range(n)))
    kp, vp, ctx, mx = m.batch(2, seqs, extra=1)
    assert ctx == [6, 1, 18] and mx == 18
    assert kp == [m.layer_cache(s, 2)[0] for s in seqs]
    assert vp == [m.layer_cache(s, 2)[1] for s in seqs]


@pytest.mark.parametrize("layers", [
    [(0, 12, -1)],               # kv_dim not a multiple of 8
    [(0, 8, 0)],                 # shares itself
    [(0, 8, -1), (0, 8, 1)],     # shares a later layer
    [(0, 8, -2)],
])
def test_invalid_layouts_are_refused(layers):
    with pytest.raises(ValueError):
        manager(layers)


def test_arena_size_and_alignment_are_checked():
    with pytest.raises(lmx.LmxError) as e:
        lmx.KvManager([(0, 8, -1)], n_ctx=16, max_seqs=2, arena=(ARENA, 100))
    assert e.value.status == lmx.Status.E_WORKSPACE
    with pytest.raises(lmx.LmxError) as e:
        lmx.KvManager([(0, 8, -1)], n_ctx=16, max_seqs=2, arena=(ARENA + 8, BIG))
    assert e.value.status == lmx.Status.E_ALIGN


def ring_reads_stale(w, hw, pos):
    """Brute force: store positions 0..hw-1 in order into a ring of w slots,
    then ask whether the query at pos sees a slot holding another position
    than the one it expects (cache.rs:21-38: slot = p % w, visible
    [max(0, pos - w + 1), pos]; pos itself is rewritten before it is read)."""
    ring = [None] * w
    for p in range(hw):
        ring[p % w] = p
    lo = max(0, pos - w + 1)
    return any(ring[x % w] != x for x in range(lo, pos))


def test_truncate_on_a_ring_leaves_the_sequence_stale_exactly_when_slots_were_overwritten():
    for w in (1, 2, 3, 4, 7):
        for hw in range(0, 17):
            for pos in range(0, hw + 1):
                m = manager([(0, 8, -1), (w, 8, -1)], n_ctx=32, max_seqs=1)
                s = m.open()
                m.commit(s, list(range(hw)))
                m.truncate(s, pos)
                stale = ring_reads_stale(w, hw, pos)
                if stale:
                    assert m.reusable_prefix(s, list(range(hw + 1))) == 0
                    for call in (lambda: m.batch(0, [s]), lambda: m.commit(s, [1])):
                        with pytest.raises(lmx.LmxError) as e:
                            call()
                        assert e.value.status == lmx.Status.E_RING_HAZARD
                else:
                    assert m.batch(1, [s])[2] == [pos + 1], (w, hw, pos)
                    m.commit(s, [1])
                    assert m.len(s) == pos + 1


def test_truncate_on_linear_layers_keeps_the_prefix_reusable():
    m = manager([(0, 8, -1), (0, 8, 0)], n_ctx=64, max_seqs=1)
    s = m.open()
    m.commit(s, list(range(40)))
    m.truncate(s, 3)
    assert m.reusable_prefix(s, [0, 1, 2, 9]) == 3
    m.commit(s, [9])
    assert m.len(s) == 4


def test_a_ring_wider_than_the_context_never_goes_stale():
    m = manager([(1024, 8, -1)], n_ctx=100, max_seqs=1)   # ring clamps to 100 slots
    s = m.open()
    m.commit(s, list(range(100)))
    m.truncate(s, 10)
    assert m.reusable_prefix(s, list(range(11))) == 10
