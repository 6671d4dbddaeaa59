"""Head sizes outside the kernels' native set (64/128/256/512) against the
oracle (cpu.rs:342-387): any multiple of 4 up to 512 is the reference's
domain (vec4 rows, attn.wgsl:36-46), and its vision tower calls attention with
head_dim = embedding_length / head_count, bidirectionally at scale 1.0
(crates/model/src/vision.rs:77-86; crates/gpu/src/vision.rs:587-631).  These
calls run through zero-padded copies at the next native size; the padded dims
must not leak into the scores or the output."""
import sys

import numpy as np
import pytest

from tests.helpers import AttnCase, assert_close

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import llmoxide_amd as lmx  # noqa: E402


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.cuda()


def run(c, *, base, window=0, bidi=False, scale=None, ring=False, k_cur=False, gate=None):
    say(f"head_dim={c.hd} t={c.t} H={c.H} Hkv={c.Hkv} base={base} w={window} bidi={bidi} "
        f"ring={ring} k_cur={k_cur} q_f16={c.q_f16} gate={gate is not None}")
    end = base + c.t
    if ring:
        kc, vc = c.ring(window, base) if k_cur else c.ring(window, end)
    else:
        kc, vc = c.k16[:end], c.v16[:end]
    q = dev(c.q.astype(np.float16)) if c.q_f16 else dev(c.q)
    kw = {}
    if k_cur:
        kw = dict(k_cur=dev(c.k16[base:end], torch.float16), v_cur=dev(c.v16[base:end], torch.float16))
    if gate is not None:
        kw["gate"] = dev(gate)
    out = lmx.attention(q, dev(kc, torch.float16), dev(vc, torch.float16), n_heads=c.H, n_kv_heads=c.Hkv,
                        head_dim=c.hd, base_pos=base, window=window, bidi=bidi, scale=scale,
                        kv_dim=c.kv_dim, **kw)
    torch.cuda.synchronize()
    ref = c.reference(base_pos=base, window=window, bidi=bidi, scale=scale)
    if gate is not None:
        ref = ref / (1.0 + np.exp(-gate.astype(np.float64)))
    return assert_close(out.cpu().numpy(), ref, what=f"head_dim {c.hd}")


@pytest.mark.parametrize("hd", [72, 80, 96])
@pytest.mark.parametrize("q_f16", [False, True])
def test_decode(hd, q_f16):
    c = AttnCase(hd + 3 * q_f16, t=1, H=16, Hkv=4, hd=hd, n_pos=1500, q_f16=q_f16)
    run(c, base=1499)


@pytest.mark.parametrize("hd", [4, 12, 36, 200, 500])
def test_decode_odd_sizes(hd):
    # the smallest head, sizes padded to each native size, and 500 -> 512;
    # Hkv = 1 puts the last head at the end of each row
    c = AttnCase(hd, t=1, H=4, Hkv=1, hd=hd, n_pos=300)
    run(c, base=299)


@pytest.mark.parametrize("hd", [72, 80, 96])
def test_vision_bidi_prefill_scale_one(hd):
    # the vision tower's call: H = Hkv, bidirectional, scale 1.0, RMS-normed
    # q and k (its rms_norm before attention)
    c = AttnCase(hd + 7, t=300, H=8, Hkv=8, hd=hd, n_pos=300, qk_norm=True)
    run(c, base=0, bidi=True, scale=1.0)


@pytest.mark.parametrize("hd", [72, 120])
def test_causal_prefill_with_history(hd):
    c = AttnCase(hd + 11, t=150, H=12, Hkv=4, hd=hd, n_pos=150 + 333, q_f16=True, qk_norm=True)
    run(c, base=333)


def test_window_ring_with_k_cur():
    c = AttnCase(91, t=70, H=8, Hkv=2, hd=80, n_pos=260)
    run(c, base=190, window=128, ring=True, k_cur=True)


def test_kv_dim_padding_and_gate():
    # cache rows wider than Hkv * hd (kv_dim 4 elements past), and the output
    # gate applied after the padded dims are dropped
    c = AttnCase(92, t=33, H=6, Hkv=3, hd=44, n_pos=100, kv_dim=3 * 44 + 4)
    gate = np.random.default_rng(5).standard_normal((33, 6 * 44)).astype(np.float32)
    run(c, base=67, gate=gate)


def test_native_sizes_unchanged():
    # a native size takes no padded copy: workspace as before (0 for a short
    # unsplit decode at hd 128 is not assumed; only that padding adds space)
    p128 = lmx.attn_params(n_tokens=300, n_heads=8, n_kv_heads=8, head_dim=128, base_pos=0, n_slots=300)
    p120 = lmx.attn_params(n_tokens=300, n_heads=8, n_kv_heads=8, head_dim=120, base_pos=0, n_slots=300)
    import ctypes
    w128 = lmx.lib().lmx_attn_workspace_bytes(ctypes.byref(p128))
    w120 = lmx.lib().lmx_attn_workspace_bytes(ctypes.byref(p120))
    assert w120 > w128
