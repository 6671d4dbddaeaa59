"""GPU parity of the attention epilogue (lmx_attn_fwd_ext): query heads read
in place from Qwen3.5's fused [query | gate] projection and the output scaled
by sigmoid(gate) where it is written, against the oracle's attention on the
deinterleaved queries followed by its gate (qwen35/cpu.rs:324-363).  Covers
every kernel path that writes the output: the split-K merge, a single split
written by the wave itself, the multi-wave workgroup combine, and prefill with
f32 and f16 queries."""
import sys

import numpy as np
import pytest

import oracle
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


def fused_case(seed, *, t, H, Hkv, hd, n_pos, q_f16=False):
    c = AttnCase(seed, t=t, H=H, Hkv=Hkv, hd=hd, n_pos=n_pos, q_f16=q_f16)
    gate = (2.0 * oracle.normal(seed * 10 + 7, (t, H * hd))).astype(np.float32)
    fused = np.empty((t, H, 2 * hd), np.float32)
    fused[:, :, :hd] = c.q.reshape(t, H, hd)
    fused[:, :, hd:] = gate.reshape(t, H, hd)
    return c, gate, fused


def run(seed, *, t, H, Hkv, hd, n_pos, base, q_f16=False, gated=True):
    say(f"gated attention t={t} H={H} Hkv={Hkv} hd={hd} ctx={base + t} q_f16={q_f16} gate={gated}")
    c, gate, fused = fused_case(seed, t=t, H=H, Hkv=Hkv, hd=hd, n_pos=n_pos, q_f16=q_f16)
    kc, vc = dev(c.k16[:base + t], torch.float16), dev(c.v16[:base + t], torch.float16)
    kw = dict(n_heads=H, n_kv_heads=Hkv, head_dim=hd, base_pos=base, kv_dim=c.kv_dim)
    if q_f16:
        # f16 queries cannot share a buffer with the f32 gate: strided q, separate gate
        fq = dev(fused.astype(np.float16))
        g = dev(gate)
        out = lmx.attention(fq, kc, vc, q_stride=2 * hd, gate=g if gated else None, **kw)
    else:
        fq = dev(fused)
        flat = fq.view(-1)
        out = lmx.attention(fq, kc, vc, q_stride=2 * hd, gate=flat[hd:] if gated else None,
                            gate_stride=2 * hd, **kw)
    torch.cuda.synchronize()
    ref = c.reference(base_pos=base)
    if gated:
        ref = oracle.attn_gate(ref, gate, dim=hd).reshape(ref.shape)
    assert_close(out.cpu().numpy(), ref, what="gated attention")


@pytest.mark.parametrize("hd", [128, 256])
def test_decode_split_and_merge(hd):
    run(1, t=1, H=8, Hkv=2, hd=hd, n_pos=3000, base=2999)


def test_decode_qwen3_shape_one_wave_per_head():
    run(2, t=1, H=32, Hkv=8, hd=128, n_pos=20000, base=19999)


def test_decode_single_split_written_by_the_wave():
    run(3, t=1, H=32, Hkv=8, hd=128, n_pos=40, base=39)


def test_few_tokens_multi_wave_workgroup_combine():
    # Hkv = 2: two waves per kv head, combined in the workgroup
    run(4, t=3, H=8, Hkv=2, hd=256, n_pos=50, base=47)


def test_prefill_f32_fused():
    run(5, t=96, H=8, Hkv=2, hd=256, n_pos=96, base=0)


def test_prefill_f16_queries_with_separate_gate():
    run(6, t=160, H=8, Hkv=2, hd=128, n_pos=200, base=40, q_f16=True)


@pytest.mark.parametrize("t", [1, 96])
def test_strided_queries_without_gate(t):
    run(7, t=t, H=8, Hkv=2, hd=128, n_pos=300, base=300 - t, gated=False)


@pytest.mark.parametrize("q_f16", [False, True])
def test_prefill_ping_pong_kernel_gated(q_f16, tuning_env):
    # the head_dim-128 ping-pong prefill kernel, forced at a small size
    tuning_env("LMX_PREFILL_KERNEL", "pp")
    run(8, t=300, H=8, Hkv=2, hd=128, n_pos=340, base=40, q_f16=q_f16)


@pytest.mark.parametrize("q_f16", [False, True])
def test_prefill_key_split_merge_gated(q_f16):
    # a short chunk on a long cache: the keys are cut into splits whose
    # partials the merge kernel combines and gates
    run(9, t=100, H=8, Hkv=2, hd=128, n_pos=3100, base=3000, q_f16=q_f16)
