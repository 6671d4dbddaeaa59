"""lmx_attn_fwd_noalloc (the attention entry point that takes no workspace)
against lmx_attn_fwd with a caller-allocated workspace, through the C ABI.

Both run the same kernels, so the outputs must agree bit for bit.  Each case
makes two calls in a row on the library's per-GPU scratch, the second with a
smaller input, so partials left by the first call must not leak into the
second.  Cases: split-K decode (C2 shape, 32k then 5k context) and a
key-split prefill chunk (512 tokens on a 4k cache, then 256 on 2k).
"""
import ctypes
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


def both(c: AttnCase, base: int, q_f16: bool):
    """(no-alloc output, workspace output) for one case."""
    L = lmx.lib()
    end = base + c.t
    p = lmx.attn_params(n_tokens=c.t, n_heads=c.H, n_kv_heads=c.Hkv, head_dim=c.hd, base_pos=base,
                        n_slots=end)
    need = L.lmx_attn_workspace_bytes(ctypes.byref(p))
    say(f"noalloc case t={c.t} H={c.H} hd={c.hd} base={base} q_f16={q_f16} need={need}")
    assert 0 < need <= lmx.NOALLOC_SCRATCH_BYTES
    q = dev(c.q.astype(np.float16)) if q_f16 else dev(c.q)
    qdt = lmx.F16 if q_f16 else lmx.F32
    kc, vc = dev(c.k16[:end], torch.float16), dev(c.v16[:end], torch.float16)
    out_na = torch.full((c.t, c.H * c.hd), float("nan"), dtype=torch.float32, device="cuda")
    out_ws = torch.full_like(out_na, float("nan"))
    stream = torch.cuda.current_stream().cuda_stream
    rc = L.lmx_attn_fwd_noalloc(ctypes.byref(p), q.data_ptr(), qdt, kc.data_ptr(), vc.data_ptr(),
                                lmx.F16, None, None, out_na.data_ptr(), stream)
    assert rc == 0, lmx.Status(rc)
    ws = torch.empty(need + 256, dtype=torch.uint8, device="cuda")
    base_ptr = ws.data_ptr() + (-ws.data_ptr()) % 256
    assert L.lmx_workspace_init(base_ptr, need, stream) == 0  # zeroed once before first use
    rc = L.lmx_attn_fwd(ctypes.byref(p), q.data_ptr(), qdt, kc.data_ptr(), vc.data_ptr(), lmx.F16,
                        None, None, out_ws.data_ptr(), base_ptr, need, stream)
    assert rc == 0, lmx.Status(rc)
    torch.cuda.synchronize()
    return out_na.cpu().numpy(), out_ws.cpu().numpy()


@pytest.mark.parametrize("cases", [
    # split-K decode: 128 splits a unit at 32k, then fewer at 5k
    [dict(t=1, H=32, Hkv=8, hd=128, base=32767, q_f16=False),
     dict(t=1, H=32, Hkv=8, hd=128, base=4999, q_f16=False)],
    # key-split prefill: 512 tokens on a 4k cache, then 256 on 2k
    [dict(t=512, H=32, Hkv=8, hd=128, base=4096, q_f16=True),
     dict(t=256, H=32, Hkv=8, hd=128, base=2000, q_f16=True)],
])
def test_noalloc_matches_the_workspace_entry_point(cases):
    for i, kw in enumerate(cases):
        base, q_f16 = kw.pop("base"), kw.pop("q_f16")
        c = AttnCase(101 + i + base, n_pos=base + kw["t"], q_f16=q_f16, qk_norm=q_f16, **kw)
        got, want = both(c, base, q_f16)
        assert np.all(np.isfinite(got))
        assert np.array_equal(got, want), f"call {i}: differs from lmx_attn_fwd"
        if kw["t"] == 1:  # and both agree with the oracle
            assert_close(got, c.reference(base_pos=base), what=f"call {i}")


def test_noalloc_refuses_a_shape_beyond_its_scratch():
    L = lmx.lib()
    # a 896-token chunk of 73 heads on a 20k cache: two key splits of 896 x 73
    # partial rows of head_dim 128, about 68 MB
    p = lmx.attn_params(n_tokens=896, n_heads=73, n_kv_heads=1, head_dim=128, base_pos=20000,
                        n_slots=20896)
    assert L.lmx_attn_workspace_bytes(ctypes.byref(p)) > lmx.NOALLOC_SCRATCH_BYTES
    x = torch.zeros(16, device="cuda")
    rc = L.lmx_attn_fwd_noalloc(ctypes.byref(p), x.data_ptr(), lmx.F32, x.data_ptr(), x.data_ptr(),
                                lmx.F16, None, None, x.data_ptr() + 4096 * 64, None)
    assert rc == lmx.Status.E_WORKSPACE
