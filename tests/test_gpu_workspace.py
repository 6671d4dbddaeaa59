"""lmx_workspace_init: the fill kernels zero exactly [ws, ws + ws_bytes).

The 16-byte form splits the buffer into eighths, one per XCD; these cases
cover buffers of fewer quads than eighths, quad counts that do not divide by
8, several grid strides, and the 4-byte form (a buffer 4 bytes off a 16-byte
boundary, or a length that is not a multiple of 16).  Guard bytes on both
sides must keep their value."""
import sys

import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import llmoxide_amd as lmx  # noqa: E402

GUARD = 256


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("offset", [0, 4], ids=["aligned16", "off4"])
@pytest.mark.parametrize("n_bytes", [4, 16, 48, 112, 128, 144, 4096 + 16, 65536 * 16 + 48,
                                     8192 * 256 * 16 + 16 * 13, 20, 1000])
def test_workspace_init_zeroes_exactly_its_bytes(n_bytes, offset):
    say(f"workspace_init n={n_bytes} offset={offset}")
    buf = torch.full((GUARD + n_bytes + GUARD,), 0xA5, dtype=torch.uint8, device="cuda")
    base = buf.data_ptr() + GUARD + offset
    n = n_bytes - offset if offset and n_bytes > offset else n_bytes
    n -= n % 4
    rc = lmx.lib().lmx_workspace_init(base, n, None)
    assert rc == 0, lmx.lib().lmx_status_str(rc)
    torch.cuda.synchronize()
    host = buf.cpu()
    lo = GUARD + offset
    assert not host[lo:lo + n].any().item(), "bytes inside the range left nonzero"
    assert (host[:lo] == 0xA5).all().item(), "bytes before the range written"
    assert (host[lo + n:] == 0xA5).all().item(), "bytes after the range written"
