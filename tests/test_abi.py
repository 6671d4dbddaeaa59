"""The C-ABI library loads, exports every symbol include/lmx/attn.h declares,
and rejects bad arguments on the host (no GPU needed: every call here returns
before anything is enqueued)."""
import ctypes
import os
import re
import subprocess

import pytest

import llmoxide_amd as lmx

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lmx", "attn.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lmx_\w+)\s*\(", text)))


def test_header_compiles_as_c_and_cxx(tmp_path):
    src = tmp_path / "t.c"
    src.write_text('#include "lmx/attn.h"\nint main(void){return lmx_version()==0;}\n')
    for cc, extra in (("gcc", ["-std=c99"]), ("g++", ["-x", "c++", "-std=c++17"])):
        r = subprocess.run([cc, *extra, "-fsyntax-only", "-Wall", "-Werror", "-I",
                            os.path.join(ROOT, "include"), str(src)], capture_output=True, text=True)
        assert r.returncode == 0, r.stderr


def test_library_exports_every_declared_symbol():
    L = lmx.lib()
    names = declared_functions()
    assert len(names) == 31
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(lmx.SIGNATURES)
    out = subprocess.run(["nm", "-D", "--defined-only", lmx.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (lmx_\w+)", out))
    assert exported == set(names)


def test_status_strings_and_version():
    L = lmx.lib()
    assert L.lmx_version() == 106
    for s in lmx.Status:
        assert L.lmx_status_str(int(s))
    assert L.lmx_status_str(999) == b"unknown status"


def _params(**kw):
    base = dict(n_tokens=1, n_heads=32, n_kv_heads=8, head_dim=128, base_pos=0, n_slots=16)
    base.update(kw)
    return lmx.attn_params(**base)


FAKE = 0x100000  # never dereferenced: validation fails first


def _fwd(p, q=FAKE, k=FAKE, v=FAKE, out=FAKE + (1 << 24), kc=None, vc=None, qdt=lmx.F32,
         kvdt=lmx.F16):
    return lmx.lib().lmx_attn_fwd(ctypes.byref(p), q, qdt, k, v, kvdt, kc, vc, out, None, 0, None)


@pytest.mark.parametrize("kw,code", [
    (dict(n_tokens=0), lmx.Status.E_SHAPE),
    (dict(n_heads=30), lmx.Status.E_SHAPE),
    (dict(head_dim=514), lmx.Status.E_UNSUPPORTED),
    (dict(head_dim=98), lmx.Status.E_UNSUPPORTED),
    (dict(head_dim=0, scale=1.0), lmx.Status.E_UNSUPPORTED),
    (dict(kv_dim=512), lmx.Status.E_SHAPE),
    (dict(kv_dim=8 * 128 + 4), lmx.Status.E_SHAPE),        # native rows: multiples of 8
    (dict(head_dim=72, kv_dim=8 * 72 + 2), lmx.Status.E_SHAPE),  # padded rows: of 4
    (dict(base_pos=16), lmx.Status.E_CONTEXT),
    (dict(n_tokens=17), lmx.Status.E_CONTEXT),
    (dict(window=32, n_slots=16), lmx.Status.E_SHAPE),
    (dict(scale=float("nan")), lmx.Status.E_SHAPE),
    (dict(window=16, n_tokens=12, base_pos=8), lmx.Status.E_RING_HAZARD),
])
def test_attn_fwd_rejects_bad_geometry(kw, code):
    assert _fwd(_params(**kw)) == code


def test_attn_fwd_rejects_bad_pointers_and_dtypes():
    p = _params()
    assert _fwd(p, q=None) == lmx.Status.E_NULL
    assert _fwd(p, out=None) == lmx.Status.E_NULL
    assert _fwd(p, kc=FAKE) == lmx.Status.E_NULL  # k_cur without v_cur
    assert _fwd(p, q=FAKE + 2) == lmx.Status.E_ALIGN
    assert _fwd(p, kvdt=lmx.F32) == lmx.Status.E_UNSUPPORTED
    assert _fwd(p, qdt=7) == lmx.Status.E_UNSUPPORTED
    assert lmx.lib().lmx_attn_fwd(None, FAKE, 0, FAKE, FAKE, 1, None, None, FAKE, None, 0, None) == lmx.Status.E_NULL


def _fwd_ext(p, ext, q=FAKE, out=FAKE + (1 << 24)):
    x = lmx.AttnExt(**ext)
    return lmx.lib().lmx_attn_fwd_ext(ctypes.byref(p), ctypes.byref(x), q, lmx.F32, FAKE, FAKE,
                                      lmx.F16, None, None, out, None, 0, None)


GATE = FAKE + (1 << 26)


@pytest.mark.parametrize("ext,code", [
    (dict(q_stride=64), lmx.Status.E_SHAPE),                     # below head_dim
    (dict(q_stride=132), lmx.Status.E_SHAPE),                    # not a multiple of 8
    (dict(gate_stride=130, gate=GATE), lmx.Status.E_SHAPE),      # not a multiple of 4
    (dict(gate_stride=64, gate=GATE), lmx.Status.E_SHAPE),       # below head_dim
    (dict(q_stride=256, gate=GATE + 4), lmx.Status.E_ALIGN),     # gate not 16-byte aligned
])
def test_attn_fwd_ext_rejects_bad_layouts(ext, code):
    assert _fwd_ext(_params(), ext) == code


def test_attn_fwd_ext_rejects_out_overlapping_q_or_gate():
    p = _params(n_tokens=2, n_slots=64, base_pos=10)
    # the fused [query | gate] rows of 2 tokens x 32 heads x 256 floats
    assert _fwd_ext(p, dict(q_stride=256), out=FAKE + 4096) == lmx.Status.E_SHAPE
    assert _fwd_ext(p, dict(q_stride=256, gate=GATE, gate_stride=256),
                    out=GATE + 1024) == lmx.Status.E_SHAPE


def test_attn_fwd_rejects_out_overlapping_q():
    p = _params(n_tokens=2, n_slots=32768, base_pos=30000)  # split: needs a workspace
    assert _fwd(p, out=FAKE) == lmx.Status.E_SHAPE
    # f16 queries: 2 tokens x 32 heads x 128 halfs = 16 KiB from q
    assert _fwd(p, out=FAKE + 16384 - 16, qdt=lmx.F16) == lmx.Status.E_SHAPE
    # out ending where q begins, or starting where the f32 queries end, does
    # not overlap: validation goes on to the (missing) workspace
    assert _fwd(p, out=FAKE - 32768) == lmx.Status.E_WORKSPACE
    assert _fwd(p, out=FAKE + 32768) == lmx.Status.E_WORKSPACE


def test_decode_needs_workspace_when_split():
    p = _params(n_slots=32768, base_pos=32767)
    need = lmx.lib().lmx_attn_workspace_bytes(ctypes.byref(p))
    assert need > 0
    assert _fwd(p) == lmx.Status.E_WORKSPACE
    # no split at tiny context: no workspace
    assert lmx.lib().lmx_attn_workspace_bytes(ctypes.byref(_params(n_slots=16, base_pos=3))) == 0


def test_workspace_bytes_is_zero_for_invalid_params():
    assert lmx.lib().lmx_attn_workspace_bytes(ctypes.byref(_params(n_heads=31))) == 0
    assert lmx.lib().lmx_attn_workspace_bytes(None) == 0


def test_kv_append_validation():
    L = lmx.lib()
    d = lmx.KvDesc(4, 1024, 10, 0, 12)
    assert L.lmx_kv_append(ctypes.byref(d), FAKE, FAKE, FAKE, FAKE, lmx.F16, None) == lmx.Status.E_CONTEXT
    d = lmx.KvDesc(4, 1022, 0, 0, 12)
    assert L.lmx_kv_append(ctypes.byref(d), FAKE, FAKE, FAKE, FAKE, lmx.F16, None) == lmx.Status.E_SHAPE
    d = lmx.KvDesc(4, 1024, 0, 0, 12)
    assert L.lmx_kv_append(ctypes.byref(d), FAKE, None, FAKE, FAKE, lmx.F16, None) == lmx.Status.E_NULL
    assert L.lmx_kv_append(ctypes.byref(d), FAKE, FAKE, FAKE, FAKE, lmx.F32, None) == lmx.Status.E_UNSUPPORTED
    assert L.lmx_kv_append(ctypes.byref(d), FAKE + 4, FAKE, FAKE, FAKE, lmx.F16, None) == lmx.Status.E_ALIGN
    d = lmx.KvDesc(4, 1024, 0, 8, 4)
    assert L.lmx_kv_append(ctypes.byref(d), FAKE, FAKE, FAKE, FAKE, lmx.F16, None) == lmx.Status.E_SHAPE


def test_batched_validation():
    L = lmx.lib()
    p = _params(n_slots=1024)
    call = lambda p, n, mx, **kw: L.lmx_attn_decode_batched(
        ctypes.byref(p), n, mx, kw.get("ctx", FAKE), FAKE, FAKE, FAKE, lmx.F32, lmx.F16, FAKE, None, 0, None)
    assert call(p, 0, 100) == lmx.Status.E_SHAPE
    assert call(p, 4, 2000) == lmx.Status.E_CONTEXT
    assert call(_params(n_tokens=2, n_slots=1024), 4, 100) == lmx.Status.E_SHAPE
    assert call(p, 4, 100, ctx=None) == lmx.Status.E_NULL
    # one long sequence is split over many workgroups and needs partials
    big = _params(n_slots=32768)
    assert L.lmx_attn_decode_batched_workspace_bytes(ctypes.byref(big), 1, 32768) > 0


def test_deltanet_validation():
    L = lmx.lib()
    op = lmx.dop(n_tok=4, n_vh=32, n_kh=16, s_dim=128)
    args = [FAKE] * 7
    assert L.lmx_deltanet_recur(ctypes.byref(op), *args[:5], None, FAKE, None) == lmx.Status.E_NULL
    bad = lmx.dop(n_tok=4, n_vh=32, n_kh=16, s_dim=96)
    assert L.lmx_deltanet_recur(ctypes.byref(bad), *args, None) == lmx.Status.E_UNSUPPORTED
    bad = lmx.dop(n_tok=0, n_vh=32, n_kh=16, s_dim=128)
    assert L.lmx_deltanet_recur(ctypes.byref(bad), *args, None) == lmx.Status.E_SHAPE
    op2 = lmx.dop(n_tok=4, n_vh=32, n_kh=16, s_dim=128)
    op2.key_dim = 100
    assert L.lmx_deltanet_recur(ctypes.byref(op2), *args, None) == lmx.Status.E_SHAPE
    assert L.lmx_deltanet_chunked(ctypes.byref(op), *args, 48, None, 0, None) == lmx.Status.E_SHAPE
    assert L.lmx_deltanet_chunked_workspace_bytes(ctypes.byref(op), 48) == 0


@pytest.mark.parametrize("T,n_vh,n_kh,sd", [(4096, 32, 16, 128), (37, 4, 2, 64), (200, 8, 4, 128)])
def test_deltanet_chunked_workspace_size(T, n_vh, n_kh, sd):
    # per (v-head, chunk): Tb and M (chunk^2 floats each) and the decays (2 chunk);
    # chunks of 32 and 64 add the split-bf16 K and Q of every (chunk, k-head),
    # 2 * chunk * s_dim floats' worth, and the one-launch form's ready flag of
    # every (chunk, v-head), its error word and one word per scan workgroup
    # (n_vh * s_dim / 16); all rounded up to 256 bytes
    L = lmx.lib()
    op = lmx.dop(n_tok=T, n_vh=n_vh, n_kh=n_kh, s_dim=sd)
    for chunk in (16, 32, 64):
        n_ch = (T + chunk - 1) // chunk
        floats = n_vh * n_ch * (2 * chunk * chunk + 2 * chunk)
        if chunk >= 32:
            floats += n_kh * n_ch * 2 * chunk * sd + n_vh * n_ch + 1 + n_vh * sd // 16
        want = (floats * 4 + 255) // 256 * 256
        assert L.lmx_deltanet_chunked_workspace_bytes(ctypes.byref(op), chunk) == want


def test_batched_decode_workspace_stops_growing():
    # the split target grows with the batch up to 16384 workgroups (B = 64 at
    # Qwen3-8B shape), so the partials' workspace is bounded for large batches
    L = lmx.lib()
    p = _params(n_slots=32768)
    ws = {B: L.lmx_attn_decode_batched_workspace_bytes(ctypes.byref(p), B, 32768) for B in (8, 32, 64, 256)}
    assert ws[8] < ws[32] < ws[64]
    assert ws[64] <= ws[256] < 1.05 * ws[64]   # ceil effects only past B = 64
    assert ws[256] < 150_000_000


def _pro(**kw):
    base = dict(n_tokens=4, n_heads=32, n_kv_heads=8, head_dim=128, q_stride=128, n_rot=128,
                base_pos=0, window=0, n_slots=16, v_norm=0, rms_eps=1e-6, rope_base=1e6)
    base.update(kw)
    return lmx.PrologueDesc(*[base[f] for f, _ in lmx.PrologueDesc._fields_])


def _pcall(d, q=FAKE, k=FAKE, v=FAKE, qg=None, kg=None, fac=None, kc=FAKE, vc=FAKE, dt=lmx.F16):
    return lmx.lib().lmx_attn_prologue(None if d is None else ctypes.byref(d), q, k, v, qg, kg, fac,
                                       kc, vc, dt, None)


@pytest.mark.parametrize("kw,code", [
    (dict(n_tokens=0), lmx.Status.E_SHAPE),
    (dict(n_kv_heads=0), lmx.Status.E_SHAPE),
    (dict(head_dim=96, q_stride=96, n_rot=96), lmx.Status.E_UNSUPPORTED),
    (dict(n_rot=63), lmx.Status.E_SHAPE),
    (dict(n_rot=256), lmx.Status.E_SHAPE),
    (dict(q_stride=64), lmx.Status.E_SHAPE),
    (dict(rope_base=0.0), lmx.Status.E_SHAPE),
    (dict(rms_eps=float("nan")), lmx.Status.E_SHAPE),
    (dict(base_pos=13), lmx.Status.E_CONTEXT),
    (dict(window=32, n_slots=16), lmx.Status.E_SHAPE),
])
def test_prologue_rejects_bad_geometry(kw, code):
    assert _pcall(_pro(**kw)) == code


def test_prologue_rejects_bad_pointers_and_dtypes():
    d = _pro()
    assert _pcall(None) == lmx.Status.E_NULL
    for name in ("q", "k", "v", "kc", "vc"):
        assert _pcall(d, **{name: None}) == lmx.Status.E_NULL, name
    assert _pcall(d, dt=lmx.F32) == lmx.Status.E_UNSUPPORTED
    assert _pcall(d, q=FAKE + 2) == lmx.Status.E_ALIGN
    assert _pcall(d, qg=FAKE + 1) == lmx.Status.E_ALIGN
    assert _pcall(d, kc=FAKE + 1) == lmx.Status.E_ALIGN


def test_delta_front_back_validation():
    L = lmx.lib()
    front = lambda **kw: L.lmx_deltanet_front(
        ctypes.byref(lmx.DeltaFrontDesc(*[dict(n_tok=4, conv_dim=8192, key_dim=2048, s_dim=128, kernel=4,
                                               eps=1e-6, **{})[f] if f not in kw else kw[f]
                                          for f, _ in lmx.DeltaFrontDesc._fields_])),
        kw.get("x", FAKE), FAKE, FAKE, kw.get("out", FAKE + (1 << 20)), None)
    assert front(n_tok=0) == lmx.Status.E_SHAPE
    assert front(conv_dim=8000) == lmx.Status.E_SHAPE
    assert front(s_dim=96) == lmx.Status.E_UNSUPPORTED
    assert front(key_dim=5000) == lmx.Status.E_SHAPE
    assert front(kernel=1) == lmx.Status.E_UNSUPPORTED
    assert front(kernel=9) == lmx.Status.E_UNSUPPORTED
    assert front(eps=float("nan")) == lmx.Status.E_SHAPE
    assert front(x=None) == lmx.Status.E_NULL
    assert front(x=FAKE + 2) == lmx.Status.E_ALIGN
    assert front(out=FAKE + 64) == lmx.Status.E_SHAPE  # output overlays the batch
    back = lambda s_dim=128, n_tok=4, o=FAKE: L.lmx_deltanet_back(
        ctypes.byref(lmx.DeltaBackDesc(n_tok, 32, s_dim, 1e-6)), o, FAKE, FAKE, None)
    assert back(s_dim=96) == lmx.Status.E_UNSUPPORTED
    assert back(n_tok=0) == lmx.Status.E_SHAPE
    assert back(o=None) == lmx.Status.E_NULL
    assert back(o=FAKE + 1) == lmx.Status.E_ALIGN


def _mv(ty=12, rows=8, in_dim=512, n_tok=1, w=FAKE, x=FAKE + (1 << 24), y=FAKE + (1 << 25)):
    d = lmx.QmvDesc(ty, rows, in_dim, n_tok)
    return lmx.lib().lmx_matvec(ctypes.byref(d), w, x, y, None)


def test_matvec_validates_before_launching():
    assert _mv(w=None) == lmx.Status.E_NULL
    assert _mv(ty=2) == lmx.Status.E_UNSUPPORTED          # Q4_0: not a path type
    assert _mv(ty=12, in_dim=320) == lmx.Status.E_SHAPE   # not a whole number of 256-blocks
    assert _mv(ty=8, in_dim=96) == lmx.Status.E_SHAPE     # Q8_0 units are 64 wide
    assert _mv(in_dim=16384 + 256) == lmx.Status.E_SHAPE
    assert _mv(rows=0) == lmx.Status.E_SHAPE
    assert _mv(w=FAKE + 8) == lmx.Status.E_ALIGN
    assert _mv(y=FAKE + (1 << 24) + 64) == lmx.Status.E_SHAPE  # y over x



def test_decode_workspace_grows_with_the_context():
    """A workspace sized once at the largest context serves every smaller one:
    the reported size never decreases as the context grows (one query at the
    end of the cache, the documented decode sizing shape), for the headline
    shape, Gemma's hd 256 and a ring window."""
    L = lmx.lib()
    for (H, Hkv, hd, w) in ((32, 8, 128, 0), (16, 8, 256, 0), (16, 8, 256, 1024), (8, 1, 512, 0)):
        prev = 0
        ctxs = sorted(set(list(range(1, 4100, 7)) + list(range(4100, 40001, 389)) + [38912, 40000]))
        for ctx in ctxs:
            p = _params(n_heads=H, n_kv_heads=Hkv, head_dim=hd, window=w,
                        n_slots=(w or 40000), base_pos=ctx - 1)
            b = L.lmx_attn_workspace_bytes(ctypes.byref(p))
            assert b >= prev, (H, Hkv, hd, w, ctx, b, prev)
            prev = b


def test_decode_workspace_covers_few_token_batches():
    L = lmx.lib()
    for base in (100, 5000, 32000):
        prev = 0
        for t in range(1, 9):
            p = _params(n_tokens=t, base_pos=base, n_slots=40000)
            b = L.lmx_attn_workspace_bytes(ctypes.byref(p))
            assert b >= prev, (base, t)
            prev = b


def test_batched_workspace_grows_with_the_batch():
    L = lmx.lib()
    for max_ctx in (900, 8192, 32768):
        p = _params(n_slots=max_ctx)
        prev = 0
        for B in range(1, 80):
            b = L.lmx_attn_decode_batched_workspace_bytes(ctypes.byref(p), B, max_ctx)
            assert b >= prev, (max_ctx, B, b, prev)
            prev = b


def test_noalloc_validates_and_refuses_shapes_beyond_its_scratch():
    """lmx_attn_fwd_noalloc checks like lmx_attn_fwd and refuses, before any
    device work, a call whose partials exceed LMX_NOALLOC_SCRATCH_BYTES."""
    L = lmx.lib()

    def call(p, q=FAKE, out=FAKE + (1 << 24)):
        return L.lmx_attn_fwd_noalloc(ctypes.byref(p), q, lmx.F32, FAKE, FAKE, lmx.F16, None, None,
                                      out, None)
    assert call(_params(n_tokens=0)) == lmx.Status.E_SHAPE
    assert call(_params(head_dim=514)) == lmx.Status.E_UNSUPPORTED
    limit = 64 << 20
    # the configured shapes fit: C2 decode at 32k, a C3 512-token chunk on 4k
    for kw in (dict(n_slots=32768, base_pos=32767), dict(n_tokens=512, n_slots=4608, base_pos=4096)):
        assert 0 < L.lmx_attn_workspace_bytes(ctypes.byref(_params(**kw))) <= limit
    # a shape beyond the scratch is refused before anything is enqueued
    # (a 896-token chunk of 73 heads on a 20k cache: 7 x 73 = 511 query-tile
    # workgroups, cut in two key splits of 896 x 73 partial rows each)
    candidates = [_params(n_tokens=896, n_heads=73, n_kv_heads=1, head_dim=128, n_slots=20896,
                          base_pos=20000)]
    big = [p for p in candidates if L.lmx_attn_workspace_bytes(ctypes.byref(p)) > limit]
    assert big
    assert call(big[0]) == lmx.Status.E_WORKSPACE


def test_padded_head_dims_validate_and_size_their_copies():
    """head_dim outside 64/128/256/512 (a multiple of 4 up to 512) is taken
    through zero-padded copies held in the workspace: the size query covers
    them, a call without that workspace is refused before any device work,
    the rows may be 4-element (8-byte) aligned, and the batched decode keeps
    native sizes only."""
    L = lmx.lib()
    for hd in (4, 72, 80, 96, 200, 500):
        p = _params(head_dim=hd, kv_dim=8 * hd, n_tokens=40, n_slots=300, base_pos=260)
        need = L.lmx_attn_workspace_bytes(ctypes.byref(p))
        hp = 64 if hd <= 64 else 128 if hd <= 128 else 256 if hd <= 256 else 512
        # at least the padded Q, K, V and out
        assert need >= 40 * 32 * hp * 4 + 2 * 300 * 8 * hp * 2 + 40 * 32 * hp * 4, (hd, need)
        assert _fwd(p) == lmx.Status.E_WORKSPACE
    # 4-element rows and 8-byte aligned f16 buffers pass validation
    p = _params(head_dim=72, n_heads=1, n_kv_heads=1, kv_dim=76, n_tokens=3, n_slots=10, base_pos=7)
    assert _fwd(p, k=FAKE + 8, v=FAKE + 8) == lmx.Status.E_WORKSPACE
    assert _fwd(p, k=FAKE + 4) == lmx.Status.E_ALIGN
    # native sizes keep 16-byte rows
    assert _fwd(_params(), k=FAKE + 8) == lmx.Status.E_ALIGN
    pb = _params(head_dim=72)
    assert L.lmx_attn_decode_batched(ctypes.byref(pb), 1, 16, FAKE, FAKE, FAKE, FAKE, lmx.F32,
                                     lmx.F16, FAKE + (1 << 24), None, 0, None) == lmx.Status.E_UNSUPPORTED
