"""GPU parity of the delta-net front (lmx_deltanet_front) and back
(lmx_deltanet_back) against the oracle (qwen35/cpu.rs:193-216, 250-259), and
the whole delta layer front -> chunked scan -> back against the sequential
oracle."""
import sys

import numpy as np
import pytest

import oracle
from tests.helpers import assert_close
from tests.test_oracle_delta_io import C5, TINY, front_inputs

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import llmoxide_amd as lmx  # noqa: E402


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("shape", [TINY, C5], ids=["tiny", "c5"])
@pytest.mark.parametrize("t", [1, 2, 3, 5, 64, 65, 300])
def test_front_matches_oracle(shape, t):
    say(f"delta front {shape['conv_dim']} t={t}")
    x, taps, state = front_inputs(shape, t, t)
    kw = dict(key_dim=shape["key_dim"], s_dim=shape["s_dim"])
    ref, st_ref = oracle.delta_front(x, taps, state, **kw)
    sd = dev(state)
    out = lmx.delta_front(dev(x), dev(taps), sd, **kw)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), ref, abs_tol=1e-5, rel_tol=1e-5, what="conv_out")
    np.testing.assert_array_equal(sd.cpu().numpy(), st_ref)  # the window is copied, bit for bit


@pytest.mark.parametrize("t", [67, 200])
@pytest.mark.parametrize("shape", [dict(conv_dim=384, key_dim=128, s_dim=64, kernel=4),
                                   dict(conv_dim=1280, key_dim=256, s_dim=128, kernel=3),
                                   dict(conv_dim=1536, key_dim=256, s_dim=128, kernel=6),
                                   dict(conv_dim=2048, key_dim=512, s_dim=64, kernel=8),
                                   dict(conv_dim=1024, key_dim=256, s_dim=64, kernel=2),
                                   dict(conv_dim=1792, key_dim=512, s_dim=128, kernel=5),
                                   dict(conv_dim=768, key_dim=128, s_dim=64, kernel=7)],
                         ids=["two_channel", "one_wave_of_four", "k6_two_waves", "k8", "k2", "k5", "k7"])
def test_front_block_edges(shape, t):
    """16-byte form at conv widths 2-8, with q/k and v channels in one wave and
    both interior and edge token chunks; in the first case (conv_dim % 256 ==
    128) the last 256-channel block is only half inside conv_dim."""
    say(f"delta front edges {shape} t={t}")
    x, taps, state = front_inputs(shape, t, 11)
    kw = dict(key_dim=shape["key_dim"], s_dim=shape["s_dim"])
    ref, st_ref = oracle.delta_front(x, taps, state, **kw)
    sd = dev(state)
    out = lmx.delta_front(dev(x), dev(taps), sd, **kw)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), ref, abs_tol=1e-5, rel_tol=1e-5, what="conv_out")
    np.testing.assert_array_equal(sd.cpu().numpy(), st_ref)


@pytest.mark.parametrize("t", [1, 3, 6, 9])
@pytest.mark.parametrize("offset", [0, 1], ids=["16byte", "two_channel"])
@pytest.mark.parametrize("shape", [dict(conv_dim=2048, key_dim=512, s_dim=64, kernel=8),
                                   dict(conv_dim=640, key_dim=128, s_dim=64, kernel=8)],
                         ids=["k8_c2048", "k8_c640"])
def test_front_batches_shorter_than_the_window(shape, offset, t):
    """Seven window rows and batches of 1-9 tokens: outputs mix old window rows
    and batch rows, and the new window mixes both too (t < 7). x placed
    `offset` floats past a 16-byte boundary picks the form (0: 16-byte,
    1: two-channel); c640 ends in a half-filled 256-channel block."""
    say(f"delta front short batch {shape} offset={offset} t={t}")
    x, taps, state = front_inputs(shape, t, 40 + t)
    kw = dict(key_dim=shape["key_dim"], s_dim=shape["s_dim"])
    ref, st_ref = oracle.delta_front(x, taps, state, **kw)
    n = t * shape["conv_dim"]
    flat = torch.zeros(n + 4, dtype=torch.float32, device="cuda")
    xd = flat[offset:offset + n].view(t, shape["conv_dim"])
    xd.copy_(dev(x))
    assert xd.data_ptr() % 16 == 4 * offset
    sd = dev(state)
    out = lmx.delta_front(xd, dev(taps), sd, **kw)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), ref, abs_tol=1e-5, rel_tol=1e-5, what="conv_out")
    np.testing.assert_array_equal(sd.cpu().numpy(), st_ref)


def test_front_unaligned_input_takes_the_two_channel_form():
    """x 4 bytes off a 16-byte boundary: the two-channel kernel runs. Both forms
    meet the oracle; they sum the head norm in different orders, so their
    outputs may differ in the last bit, and the windows are equal."""
    say("delta front unaligned x")
    t = 70
    x, taps, state = front_inputs(C5, t, 12)
    kw = dict(key_dim=C5["key_dim"], s_dim=C5["s_dim"])
    ref, st_ref = oracle.delta_front(x, taps, state, **kw)
    flat = torch.zeros(t * C5["conv_dim"] + 4, dtype=torch.float32, device="cuda")
    xu = flat[1:1 + t * C5["conv_dim"]].view(t, C5["conv_dim"])
    xu.copy_(dev(x))
    assert xu.data_ptr() % 16 == 4
    sd_u, sd_a = dev(state), dev(state)
    out_u = lmx.delta_front(xu, dev(taps), sd_u, **kw)
    out_a = lmx.delta_front(dev(x), dev(taps), sd_a, **kw)
    torch.cuda.synchronize()
    assert_close(out_u.cpu().numpy(), ref, abs_tol=1e-5, rel_tol=1e-5, what="conv_out (two-channel)")
    assert_close(out_a.cpu().numpy(), ref, abs_tol=1e-5, rel_tol=1e-5, what="conv_out (16-byte)")
    np.testing.assert_allclose(out_u.cpu().numpy(), out_a.cpu().numpy(), rtol=1e-6, atol=1e-6)
    np.testing.assert_array_equal(sd_u.cpu().numpy(), st_ref)
    np.testing.assert_array_equal(sd_a.cpu().numpy(), st_ref)


def test_front_chained_calls_carry_the_window():
    say("delta front chained")
    x, taps, state = front_inputs(C5, 70, 4)
    kw = dict(key_dim=C5["key_dim"], s_dim=C5["s_dim"])
    ref, st_ref = oracle.delta_front(x, taps, state, **kw)
    sd, xd, td = dev(state), dev(x), dev(taps)
    outs = [lmx.delta_front(xd[a:b].contiguous(), td, sd, **kw) for a, b in ((0, 2), (2, 67), (67, 70))]
    torch.cuda.synchronize()
    assert_close(torch.cat(outs).cpu().numpy(), ref, abs_tol=1e-5, rel_tol=1e-5, what="conv_out")
    np.testing.assert_array_equal(sd.cpu().numpy(), st_ref)


@pytest.mark.parametrize("n_vh,t", [(32, 37), (3, 37), (1, 1)], ids=["c5_heads", "ragged", "one_row"])
@pytest.mark.parametrize("s_dim", [64, 128, 256])
def test_back_matches_oracle(s_dim, n_vh, t):
    """16-byte form: whole workgroups, a ragged last wave (111 rows) and a
    single row, at each head size."""
    say(f"delta back s_dim={s_dim} n_vh={n_vh} t={t}")
    o = oracle.normal(s_dim + 1, (t, n_vh * s_dim))
    z = oracle.normal(s_dim + 2, (t, n_vh * s_dim))
    w = (1.0 + 0.2 * oracle.normal(s_dim + 3, (s_dim,))).astype(np.float32)
    ref = oracle.delta_back(o, z, w, n_vh=n_vh, s_dim=s_dim)
    od = dev(o)
    lmx.delta_back(od, dev(z), dev(w), n_vh=n_vh, s_dim=s_dim)
    torch.cuda.synchronize()
    assert_close(od.cpu().numpy(), ref, abs_tol=1e-5, rel_tol=1e-5, what="o")


def test_back_unaligned_gate_takes_the_row_form():
    """z 4 bytes off a 16-byte boundary: the one-wave-a-row kernel runs and
    meets the oracle."""
    say("delta back unaligned z")
    n_vh, t, s_dim = 32, 21, 128
    o = oracle.normal(201, (t, n_vh * s_dim))
    z = oracle.normal(202, (t, n_vh * s_dim))
    w = (1.0 + 0.2 * oracle.normal(203, (s_dim,))).astype(np.float32)
    ref = oracle.delta_back(o, z, w, n_vh=n_vh, s_dim=s_dim)
    flat = torch.zeros(z.size + 4, dtype=torch.float32, device="cuda")
    zu = flat[1:1 + z.size].view(z.shape)
    zu.copy_(dev(z))
    assert zu.data_ptr() % 16 == 4
    od = dev(o)
    lmx.delta_back(od, zu, dev(w), n_vh=n_vh, s_dim=s_dim)
    torch.cuda.synchronize()
    assert_close(od.cpu().numpy(), ref, abs_tol=1e-5, rel_tol=1e-5, what="o (row form)")


def test_delta_layer_front_scan_back_matches_oracle():
    """C5 delta layer at T=200: front, chunked scan, back on the GPU against the
    oracle's front, sequential recurrence and back."""
    say("delta layer front+scan+back")
    n_vh, n_kh, sd = 32, 16, 128
    T = 200
    x, taps, cstate = front_inputs(C5, T, 8)
    al = oracle.normal(81, (T, n_vh))
    be = oracle.normal(82, (T, n_vh))
    z = oracle.normal(83, (T, n_vh * sd))
    w = (1.0 + 0.2 * oracle.normal(84, (sd,))).astype(np.float32)
    S0 = (0.1 * oracle.normal(85, (n_vh * sd * sd,))).astype(np.float32)
    kw = dict(key_dim=C5["key_dim"], s_dim=sd)
    conv, _ = oracle.delta_front(x, taps, cstate, **kw)
    o_ref, S_ref = oracle.delta_recur(conv, al, be, S0, n_vh=n_vh, n_kh=n_kh, s_dim=sd)
    y_ref = oracle.delta_back(o_ref, z, w, n_vh=n_vh, s_dim=sd)

    A = dev(np.full(n_vh, -1.0, np.float32))
    dt = dev(np.zeros(n_vh, np.float32))
    state = dev(S0.copy())
    conv_d = lmx.delta_front(dev(x), dev(taps), dev(cstate), **kw)
    o = lmx.delta_chunked(conv_d, dev(al), dev(be), state, A, dt, n_vh=n_vh, n_kh=n_kh, s_dim=sd, chunk=64)
    lmx.delta_back(o, dev(z), dev(w), n_vh=n_vh, s_dim=sd)
    torch.cuda.synchronize()
    assert_close(o.cpu().numpy(), y_ref, what="layer output")
    assert_close(state.cpu().numpy(), S_ref, what="S")
