"""GPU parity of the attention prologue (lmx_attn_prologue): per-head RMS norm
with gain, NeoX RoPE over n_rot dims, optional V norm and the f16 KV store,
against the oracle (cpu.rs:286-327; qwen35/cpu.rs:294-304).

Q is compared within the path's tolerance; the cache rows are compared as
decoded f16 values within one f16 rounding step, since the GPU's RMS sum runs
in a different order than the reference's sequential f32 sum."""
import sys

import numpy as np
import pytest

import oracle
from tests.helpers import assert_close
from tests.test_oracle_prologue import CONFIGS, make

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


def run(cfg, t, base_pos, n_slots=None, seed=3, overrides=None):
    q, k, v, kw, window = make(cfg, t=t, base_pos=base_pos, seed=seed)
    kw = dict(kw, **(overrides or {}))
    n_slots = n_slots or (window or base_pos + t)
    say(f"prologue {cfg} t={t} base={base_pos} window={window} slots={n_slots}")
    init = np.full((n_slots, kw["n_kv_heads"] * kw["head_dim"]), 0x3C00, np.uint16)
    q_ref, kc_ref, vc_ref = oracle.attn_prologue(q, k, v, n_slots=n_slots, window=window,
                                                 k_cache=init, v_cache=init, **kw)
    qd = dev(q)
    kc, vc = dev(init.copy(), torch.float16), dev(init.copy(), torch.float16)
    g = {name: (None if kw.get(name) is None else dev(kw[name]))
         for name in ("q_gain", "k_gain", "rope_factors")}
    lmx.attn_prologue(qd, dev(k), dev(v), kc, vc, n_heads=kw["n_heads"], n_kv_heads=kw["n_kv_heads"],
                      head_dim=kw["head_dim"], base_pos=base_pos, q_stride=kw["q_stride"],
                      n_rot=kw["n_rot"], window=window, v_norm=kw.get("v_norm", False),
                      rope_base=kw["rope_base"], **g)
    torch.cuda.synchronize()
    assert_close(qd.cpu().numpy(), q_ref, abs_tol=1e-4, rel_tol=1e-5, what="q")
    for name, got, ref in (("k", kc, kc_ref), ("v", vc, vc_ref)):
        gb = got.cpu().view(torch.int16).numpy().view(np.uint16)
        ga, ra = oracle.from_f16_bits(gb), oracle.from_f16_bits(ref)
        bad = np.abs(ga - ra) > np.abs(ra) * 2.0 ** -10 + 2.0 ** -24
        assert not bad.any(), f"{name}: {int(bad.sum())} cache values differ by more than one f16 step"
        # rows the call does not store keep their initial bits
        untouched = np.all(ref == 0x3C00, axis=1)
        assert np.array_equal(gb[untouched], ref[untouched]), f"{name}: wrote outside its slots"


@pytest.mark.parametrize("cfg", sorted(CONFIGS))
def test_prologue_matches_oracle(cfg):
    run(cfg, t=7, base_pos=37)


@pytest.mark.parametrize("cfg", ["qwen3", "gemma_global"])
def test_prologue_decode_token_at_large_position(cfg):
    run(cfg, t=1, base_pos=32767)


def test_prologue_ring_wraps_within_one_call():
    # 40 tokens into a 16-slot ring: only the last 16 positions survive
    run("gemma_swa", t=40, base_pos=5)


def test_prologue_prefill_batch():
    run("qwen3", t=300, base_pos=0, seed=9)


def test_prologue_without_norms_is_rope_and_store_only():
    run("qwen3", t=5, base_pos=11, overrides=dict(q_gain=None, k_gain=None))


@pytest.mark.parametrize("n_rot", [0, 32, 96])
def test_prologue_partial_rotation_widths(n_rot):
    # n_rot 32 pairs lanes within one register, 96 pairs across registers at a
    # lane offset (the LDS exchange), 0 rotates nothing
    run("qwen3", t=6, base_pos=1000, overrides=dict(n_rot=n_rot))
