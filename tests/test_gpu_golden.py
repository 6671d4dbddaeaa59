"""GPU parity against the committed golden fixtures (tests/golden/): the HIP
path, called through the C-ABI, on the fixture inputs, within the path's
tolerance of the stored oracle outputs.  The tiny-hd attention fixtures are
below the kernels' head_dim range (64/128/256) and are checked on the CPU only.
"""
import os
import sys

import numpy as np
import pytest

from tests.golden import make_golden as mg
from tests.helpers import assert_close

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import llmoxide_amd as lmx  # noqa: E402

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(HERE, name), allow_pickle=False)


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.cuda()


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_attn_c1_decode_matches_fixture():
    say("golden attn C1 decode")
    f = load("attn_c1.npz")
    c = mg.attn_c1_inputs()
    assert mg.digest(c.q, c.k16, c.v16) == str(f["input_sha256"])
    out = lmx.attention(dev(c.q), dev(c.k16, torch.float16), dev(c.v16, torch.float16),
                        n_heads=mg.C1["H"], n_kv_heads=mg.C1["Hkv"], head_dim=mg.C1["hd"],
                        base_pos=mg.C1["base_pos"])
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), f["out"], what="C1 decode")


@pytest.mark.parametrize("chunked", [False, True])
def test_delta_c5_slice_matches_fixture(chunked):
    say(f"golden delta C5 slice chunked={chunked}")
    f = load("delta_c5_slice.npz")
    conv, al, be, S0, A, dt = mg.delta_c5_inputs()
    assert mg.digest(conv, al, be, S0) == str(f["input_sha256"])
    d = mg.DELTA_C5
    state = dev(S0.copy())
    kw = dict(n_vh=d["n_vh"], n_kh=d["n_kh"], s_dim=d["sd"])
    if chunked:
        out = lmx.delta_chunked(dev(conv), dev(al), dev(be), state, dev(A), dev(dt), chunk=64, **kw)
    else:
        out = lmx.delta_recur(dev(conv), dev(al), dev(be), state, dev(A), dev(dt), **kw)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), f["o"], what="o")
    assert_close(state.cpu().numpy().reshape(-1), f["S"].reshape(-1), what="S")
