"""llmoxide_amd -- MI355X (gfx950) attention hot path for llmoxide.

The product is ``libllmoxide_amd.so``, a C-ABI library (``include/lmx/attn.h``)
of hand-written HIP kernels.  This module is the host-side mirror of the
reference's dispatch interface for that path, in Python over ``ctypes``:

=========================  ==================================================
this module                reference dispatch it mirrors
=========================  ==================================================
``write_cache``            ``write_cache`` (ops.wgsl:323-346; qwen35.rs:1062-1074)
``attn_prologue``          per-head ``rms_norm`` + ``rope``/``rope_partial`` on Q
                           and K (+ V norm) + both ``write_cache``
                           (ops.wgsl:49-91, 186-218, 269-306, 323-346)
``attention``              ``scores_pass``/``softmax_pass``/``weighted_v``
                           (attn.wgsl:84-232; qwen35.rs:1076-1094,
                           forward.rs:988-1011)
``attention_decode_batched``  the same, one query per sequence, ragged
``delta_recur``            ``delta_recur`` (deltanet.wgsl:193-239;
                           qwen35.rs:960-965)
``delta_chunked``          chunked prefill form of ``delta_recur``
``delta_front``            ``conv_silu``/``conv_shift``/``conv_commit``/
                           ``l2norm_qk`` (deltanet.wgsl:54-173)
``delta_back``             ``rms_norm`` + ``mul_silu`` after the recurrence
                           (qwen35.rs:968-986)
=========================  ==================================================

Tensors are torch tensors on a ROCm device (torch provides device memory and
streams only).  Every call goes through the C ABI; there is no CPU fallback:
if the library is missing, :func:`lib` raises.
"""
from __future__ import annotations

import ctypes
import enum
import math
import os
from typing import Optional, Sequence, Tuple

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libllmoxide_amd.so")


class Status(enum.IntEnum):
    OK = 0
    E_NULL = 1
    E_SHAPE = 2
    E_UNSUPPORTED = 3
    E_WORKSPACE = 4
    E_CONTEXT = 5
    E_RING_HAZARD = 6
    E_ALIGN = 7
    E_LAUNCH = 8
    E_DEVICE = 9
    E_FULL = 10
    E_HOST = 11


F32, F16 = 0, 1

# LMX_NOALLOC_SCRATCH_BYTES (include/lmx/attn.h): the per-GPU scratch of
# lmx_attn_fwd_noalloc
NOALLOC_SCRATCH_BYTES = 64 << 20


class LmxError(RuntimeError):
    """A call rejected by the library; ``.status`` is the :class:`Status`."""

    def __init__(self, fn: str, status: int):
        self.status = Status(status)
        super().__init__(f"{fn}: {self.status.name} ({lib().lmx_status_str(status).decode()})")


class AttnParams(ctypes.Structure):
    """lmx_attn_params: the reference's ``Attn`` uniform (attn.wgsl:22-34)
    without ``max_vis``, plus ``n_slots``."""
    _fields_ = [
        ("n_tokens", ctypes.c_uint32),
        ("n_heads", ctypes.c_uint32),
        ("n_kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("kv_dim", ctypes.c_uint32),
        ("base_pos", ctypes.c_uint32),
        ("window", ctypes.c_uint32),
        ("n_slots", ctypes.c_uint32),
        ("bidi", ctypes.c_uint32),
        ("scale", ctypes.c_float),
    ]


class KvDesc(ctypes.Structure):
    _fields_ = [
        ("n_tokens", ctypes.c_uint32),
        ("kv_dim", ctypes.c_uint32),
        ("base_pos", ctypes.c_uint32),
        ("window", ctypes.c_uint32),
        ("n_slots", ctypes.c_uint32),
    ]


class Dop(ctypes.Structure):
    """lmx_dop: the reference's ``DOp`` uniform (deltanet.wgsl:20-34), the
    fields the recurrence reads."""
    _fields_ = [
        ("n_tok", ctypes.c_uint32),
        ("conv_dim", ctypes.c_uint32),
        ("key_dim", ctypes.c_uint32),
        ("d_inner", ctypes.c_uint32),
        ("s_dim", ctypes.c_uint32),
        ("n_vh", ctypes.c_uint32),
        ("n_kh", ctypes.c_uint32),
        ("scale", ctypes.c_float),
    ]


class PrologueDesc(ctypes.Structure):
    """lmx_prologue_desc: geometry of the norm / rotate / store prologue."""
    _fields_ = [
        ("n_tokens", ctypes.c_uint32),
        ("n_heads", ctypes.c_uint32),
        ("n_kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("q_stride", ctypes.c_uint32),
        ("n_rot", ctypes.c_uint32),
        ("base_pos", ctypes.c_uint32),
        ("window", ctypes.c_uint32),
        ("n_slots", ctypes.c_uint32),
        ("v_norm", ctypes.c_uint32),
        ("rms_eps", ctypes.c_float),
        ("rope_base", ctypes.c_float),
    ]


class DeltaFrontDesc(ctypes.Structure):
    """lmx_delta_front_desc: the conv / window / q-k norm front of the delta-net."""
    _fields_ = [
        ("n_tok", ctypes.c_uint32),
        ("conv_dim", ctypes.c_uint32),
        ("key_dim", ctypes.c_uint32),
        ("s_dim", ctypes.c_uint32),
        ("kernel", ctypes.c_uint32),
        ("eps", ctypes.c_float),
    ]


class AttnExt(ctypes.Structure):
    """lmx_attn_ext: query head stride and optional sigmoid output gate."""
    _fields_ = [
        ("q_stride", ctypes.c_uint32),
        ("gate_stride", ctypes.c_uint32),
        ("gate", ctypes.c_void_p),
    ]


class QmvDesc(ctypes.Structure):
    """lmx_qmv_desc: a quantized (or dense) weight matrix times token vectors."""
    _fields_ = [
        ("type", ctypes.c_uint32),
        ("rows", ctypes.c_uint32),
        ("in_dim", ctypes.c_uint32),
        ("n_tok", ctypes.c_uint32),
    ]


# ggml type codes lmx_matvec takes (crates/gguf: GgmlType)
QTYPES = {"f32": 0, "f16": 1, "q8_0": 8, "q4_k": 12, "q6_k": 14, "bf16": 30}


class KvmLayer(ctypes.Structure):
    """lmx_kvm_layer: one layer of a KV manager (window, row size, sharing)."""
    _fields_ = [
        ("window", ctypes.c_uint32),
        ("kv_dim", ctypes.c_uint32),
        ("kv_source", ctypes.c_int32),
    ]


class KvmDesc(ctypes.Structure):
    """lmx_kvm_desc: layers, positions per sequence and sequence slots."""
    _fields_ = [
        ("n_layers", ctypes.c_uint32),
        ("n_ctx", ctypes.c_uint32),
        ("max_seqs", ctypes.c_uint32),
        ("layers", ctypes.POINTER(KvmLayer)),
    ]


class DeltaBackDesc(ctypes.Structure):
    """lmx_delta_back_desc: the gated RMS norm after the recurrence."""
    _fields_ = [
        ("n_tok", ctypes.c_uint32),
        ("n_vh", ctypes.c_uint32),
        ("s_dim", ctypes.c_uint32),
        ("eps", ctypes.c_float),
    ]


# Every symbol include/lmx/attn.h declares, with its ctypes signature.
_VP, _SZ, _I32, _U32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int32, ctypes.c_uint32
_PA, _PK, _PD = ctypes.POINTER(AttnParams), ctypes.POINTER(KvDesc), ctypes.POINTER(Dop)
_PP = ctypes.POINTER(PrologueDesc)
_PF, _PB = ctypes.POINTER(DeltaFrontDesc), ctypes.POINTER(DeltaBackDesc)
_PX = ctypes.POINTER(AttnExt)
_PQ = ctypes.POINTER(QmvDesc)
_PKD, _PI32, _PU32 = ctypes.POINTER(KvmDesc), ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_uint32)
_PVP = ctypes.POINTER(ctypes.c_void_p)
SIGNATURES = {
    "lmx_status_str": (ctypes.c_char_p, [ctypes.c_int]),
    "lmx_version": (ctypes.c_int, []),
    "lmx_tuning_reload": (None, []),
    "lmx_workspace_init": (ctypes.c_int, [_VP, _SZ, _VP]),
    "lmx_kv_append": (ctypes.c_int, [_PK, _VP, _VP, _VP, _VP, ctypes.c_int, _VP]),
    "lmx_attn_prologue": (ctypes.c_int, [_PP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, ctypes.c_int,
                                         _VP]),
    "lmx_attn_workspace_bytes": (_SZ, [_PA]),
    "lmx_attn_fwd": (ctypes.c_int, [_PA, _VP, ctypes.c_int, _VP, _VP, ctypes.c_int, _VP, _VP, _VP,
                                    _VP, _SZ, _VP]),
    "lmx_attn_fwd_ext": (ctypes.c_int, [_PA, _PX, _VP, ctypes.c_int, _VP, _VP, ctypes.c_int, _VP,
                                        _VP, _VP, _VP, _SZ, _VP]),
    "lmx_attn_fwd_noalloc": (ctypes.c_int, [_PA, _VP, ctypes.c_int, _VP, _VP, ctypes.c_int, _VP, _VP,
                                            _VP, _VP]),
    "lmx_attn_decode_batched_workspace_bytes": (_SZ, [_PA, _I32, _I32]),
    "lmx_attn_decode_batched": (ctypes.c_int, [_PA, _I32, _I32, _VP, _VP, _VP, _VP, ctypes.c_int,
                                               ctypes.c_int, _VP, _VP, _SZ, _VP]),
    "lmx_deltanet_recur": (ctypes.c_int, [_PD, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP]),
    "lmx_deltanet_front": (ctypes.c_int, [_PF, _VP, _VP, _VP, _VP, _VP]),
    "lmx_deltanet_back": (ctypes.c_int, [_PB, _VP, _VP, _VP, _VP]),
    "lmx_matvec": (ctypes.c_int, [_PQ, _VP, _VP, _VP, _VP]),
    "lmx_kvm_arena_bytes": (_SZ, [_PKD]),
    "lmx_kvm_create": (ctypes.c_int, [_PKD, _VP, _SZ, _PVP]),
    "lmx_kvm_destroy": (None, [_VP]),
    "lmx_kvm_open": (ctypes.c_int, [_VP, _PI32]),
    "lmx_kvm_close": (ctypes.c_int, [_VP, _I32]),
    "lmx_kvm_len": (ctypes.c_int, [_VP, _I32, _PU32]),
    "lmx_kvm_reusable_prefix": (ctypes.c_int, [_VP, _I32, _PI32, _U32, _PU32]),
    "lmx_kvm_begin": (ctypes.c_int, [_VP, _I32, _PI32, _U32, _PU32, _VP]),
    "lmx_kvm_commit": (ctypes.c_int, [_VP, _I32, _PI32, _U32]),
    "lmx_kvm_truncate": (ctypes.c_int, [_VP, _I32, _U32]),
    "lmx_kvm_wipe": (ctypes.c_int, [_VP, _I32, _VP]),
    "lmx_kvm_layer_cache": (ctypes.c_int, [_VP, _I32, _U32, _PVP, _PVP, _PU32, _PU32]),
    "lmx_kvm_batch": (ctypes.c_int, [_VP, _U32, _PI32, _U32, _U32, _PVP, _PVP, _PI32, _PI32]),
    "lmx_deltanet_chunked_workspace_bytes": (_SZ, [_PD, _I32]),
    "lmx_deltanet_chunked": (ctypes.c_int, [_PD, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _I32, _VP, _SZ,
                                            _VP]),
}

_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """Load libllmoxide_amd.so; raise (never fall back) if it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m llmoxide_amd.build` "
                "(there is no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def tuning_reload() -> None:
    """Re-read the LMX_* kernel-choice overrides from the environment (the
    library reads them once, at its first launch)."""
    lib().lmx_tuning_reload()


def _check(fn: str, rc: int) -> None:
    if rc != 0:
        raise LmxError(fn, rc)


# ---------------------------------------------------------------- helpers --
def _torch():
    import torch  # deferred: the ABI checks need no torch
    return torch


def _ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(stream) -> Optional[int]:
    torch = _torch()
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


def _dt(t) -> int:
    torch = _torch()
    if t.dtype == torch.float32:
        return F32
    if t.dtype == torch.float16:
        return F16
    raise TypeError(f"unsupported dtype {t.dtype}")


def _need_cuda(*ts) -> None:
    for t in ts:
        if t is not None and (not t.is_cuda or not t.is_contiguous()):
            raise ValueError("tensors must be contiguous and on the GPU")


class Workspace:
    """A zero-initialized device scratch buffer shared by successive calls.

    Calls on one Workspace must be ordered on one stream (each call writes
    every workspace byte it later reads).  It grows on demand; growth
    re-allocates and re-clears.
    """

    def __init__(self, nbytes: int = 0, device=None):
        self.device = device
        self.buf = None
        self.nbytes = 0
        if nbytes:
            self.ensure(nbytes)

    def ensure(self, nbytes: int, stream=None):
        """Grow to at least ``nbytes`` for work enqueued on ``stream`` (None:
        torch's current stream).  torch's caching allocator orders frees and
        reuse on the current stream only, so on another stream both the new
        buffer and a replaced one are marked as used there
        (``record_stream``): neither is handed out again while the stream
        still has this workspace's kernels queued."""
        torch = _torch()
        if nbytes <= self.nbytes:
            return self
        side = stream is not None and stream != torch.cuda.current_stream()
        if side and self.buf is not None:
            self.buf.record_stream(stream)
        nbytes = (nbytes + 255) // 256 * 256
        self.buf = torch.empty(nbytes + 256, dtype=torch.uint8,
                               device=self.device or torch.device("cuda"))
        if side:
            self.buf.record_stream(stream)
        off = (-self.buf.data_ptr()) % 256
        self.base = self.buf.data_ptr() + off
        self.nbytes = nbytes
        _check("lmx_workspace_init", lib().lmx_workspace_init(self.base, nbytes, _stream(stream)))
        return self


def attn_params(*, n_tokens, n_heads, n_kv_heads, head_dim, base_pos, n_slots, window=0,
                bidi=False, scale=None, kv_dim=None) -> AttnParams:
    scale = 1.0 / math.sqrt(head_dim) if scale is None else scale
    return AttnParams(n_tokens, n_heads, n_kv_heads, head_dim, kv_dim or n_kv_heads * head_dim,
                      base_pos, window, n_slots, int(bool(bidi)), scale)


# --------------------------------------------------------------- the path --
def write_cache(k_new, v_new, k_cache, v_cache, *, base_pos: int, window: int = 0, stream=None):
    """Append f32 rows [t, kv_dim] into f16 caches [n_slots, kv_dim] at
    slot(base_pos + i) (ops.wgsl:323-346).  Either pair may be None."""
    _need_cuda(k_new, v_new, k_cache, v_cache)
    src = k_new if k_new is not None else v_new
    cache = k_cache if k_cache is not None else v_cache
    d = KvDesc(src.shape[0], src.shape[-1], base_pos, window, cache.shape[0])
    rc = lib().lmx_kv_append(ctypes.byref(d), _ptr(k_new), _ptr(v_new), _ptr(k_cache), _ptr(v_cache),
                             F16, _stream(stream))
    _check("lmx_kv_append", rc)


def attn_prologue(q, k_new, v_new, k_cache, v_cache, *, n_heads: int, n_kv_heads: int,
                  head_dim: int, base_pos: int, q_stride: Optional[int] = None,
                  n_rot: Optional[int] = None, window: int = 0, v_norm: bool = False,
                  rms_eps: float = 1e-6, rope_base: float = 1e6, q_gain=None, k_gain=None,
                  rope_factors=None, stream=None):
    """Per-head RMS norm (gain), NeoX RoPE over n_rot dims and the f16 KV store,
    in one launch (cpu.rs:286-327; qwen35/cpu.rs:294-304).  q [t, H*q_stride] f32
    is updated in place; k_new, v_new [t, kv_dim] f32 go to the caches."""
    _need_cuda(q, k_new, v_new, k_cache, v_cache, q_gain, k_gain, rope_factors)
    q_stride = q_stride or head_dim
    n_rot = head_dim if n_rot is None else n_rot
    t = k_new.shape[0]
    d = PrologueDesc(t, n_heads, n_kv_heads, head_dim, q_stride, n_rot, base_pos, window,
                     k_cache.shape[0], int(bool(v_norm)), rms_eps, rope_base)
    rc = lib().lmx_attn_prologue(ctypes.byref(d), _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(q_gain),
                                 _ptr(k_gain), _ptr(rope_factors), _ptr(k_cache), _ptr(v_cache), F16,
                                 _stream(stream))
    _check("lmx_attn_prologue", rc)
    return q


def attention(q, k_cache, v_cache, *, n_heads: int, n_kv_heads: int, head_dim: int,
              base_pos: int, window: int = 0, bidi: bool = False, scale: Optional[float] = None,
              k_cur=None, v_cur=None, out=None, workspace: Optional[Workspace] = None,
              kv_dim: Optional[int] = None, q_stride: Optional[int] = None, gate=None,
              gate_stride: Optional[int] = None, stream=None):
    """GQA attention of q [t, H*hd] (f32/f16) over f16 caches [n_slots, kv_dim].

    Returns out [t, H*hd] f32.  The semantics are the reference's CPU attention
    (cpu.rs:342-387; qwen35/cpu.rs:324-365); see include/lmx/attn.h.

    ``q_stride`` reads query head h of token i at element (i*H + h)*q_stride of
    ``q`` (qwen35's fused [query | gate] heads: 2*hd), and ``gate`` (f32, read
    at (i*H + h)*gate_stride + d) scales the output by sigmoid(gate)
    (qwen35/cpu.rs:359-363); both go through lmx_attn_fwd_ext.
    """
    torch = _torch()
    _need_cuda(q, k_cache, v_cache, k_cur, v_cur, out)
    t = q.shape[0]
    p = attn_params(n_tokens=t, n_heads=n_heads, n_kv_heads=n_kv_heads, head_dim=head_dim,
                    base_pos=base_pos, n_slots=k_cache.shape[0], window=window, bidi=bidi,
                    scale=scale, kv_dim=kv_dim)
    if out is None:
        out = torch.empty((t, n_heads * head_dim), dtype=torch.float32, device=q.device)
    need = lib().lmx_attn_workspace_bytes(ctypes.byref(p))
    ws_ptr, ws_bytes = None, 0
    if need:
        workspace = workspace or Workspace(device=q.device)
        workspace.ensure(need, stream)
        ws_ptr, ws_bytes = workspace.base, workspace.nbytes
    if q_stride is None and gate is None and gate_stride is None:
        rc = lib().lmx_attn_fwd(ctypes.byref(p), _ptr(q), _dt(q), _ptr(k_cache), _ptr(v_cache), F16,
                                _ptr(k_cur), _ptr(v_cur), _ptr(out), ws_ptr, ws_bytes,
                                _stream(stream))
        _check("lmx_attn_fwd", rc)
        return out
    _need_cuda(gate)
    x = AttnExt(q_stride or 0, gate_stride or 0, _ptr(gate))
    rc = lib().lmx_attn_fwd_ext(ctypes.byref(p), ctypes.byref(x), _ptr(q), _dt(q), _ptr(k_cache),
                                _ptr(v_cache), F16, _ptr(k_cur), _ptr(v_cur), _ptr(out), ws_ptr,
                                ws_bytes, _stream(stream))
    _check("lmx_attn_fwd_ext", rc)
    return out


class BatchedCaches:
    """Device pointer tables for :func:`attention_decode_batched`."""

    def __init__(self, k_caches: Sequence, v_caches: Sequence, device=None):
        torch = _torch()
        self.k_caches, self.v_caches = list(k_caches), list(v_caches)
        dev = device or self.k_caches[0].device
        self.k_ptrs = torch.tensor([c.data_ptr() for c in self.k_caches], dtype=torch.int64, device=dev)
        self.v_ptrs = torch.tensor([c.data_ptr() for c in self.v_caches], dtype=torch.int64, device=dev)

    @classmethod
    def from_addresses(cls, k_ptrs: Sequence[int], v_ptrs: Sequence[int], device=None):
        """Tables of raw cache addresses (e.g. from :meth:`KvManager.batch`);
        pass ``n_slots`` to :func:`attention_decode_batched` with them."""
        torch = _torch()
        self = cls.__new__(cls)
        self.k_caches, self.v_caches = [], []
        dev = device or torch.device("cuda")
        self.k_ptrs = torch.tensor(list(k_ptrs), dtype=torch.int64, device=dev)
        self.v_ptrs = torch.tensor(list(v_ptrs), dtype=torch.int64, device=dev)
        return self


def attention_decode_batched(q, caches: BatchedCaches, ctx_lens, *, max_ctx: int, n_heads: int,
                             n_kv_heads: int, head_dim: int, window: int = 0,
                             scale: Optional[float] = None, n_slots: Optional[int] = None,
                             out=None, workspace: Optional[Workspace] = None, stream=None):
    """One query token per sequence: q [B, H*hd], ctx_lens int32 [B] on device."""
    torch = _torch()
    _need_cuda(q, ctx_lens, out)
    B = q.shape[0]
    p = attn_params(n_tokens=1, n_heads=n_heads, n_kv_heads=n_kv_heads, head_dim=head_dim,
                    base_pos=0, n_slots=n_slots or caches.k_caches[0].shape[0], window=window,
                    scale=scale)
    if out is None:
        out = torch.empty((B, n_heads * head_dim), dtype=torch.float32, device=q.device)
    need = lib().lmx_attn_decode_batched_workspace_bytes(ctypes.byref(p), B, max_ctx)
    ws_ptr, ws_bytes = None, 0
    if need:
        workspace = workspace or Workspace(device=q.device)
        workspace.ensure(need, stream)
        ws_ptr, ws_bytes = workspace.base, workspace.nbytes
    rc = lib().lmx_attn_decode_batched(ctypes.byref(p), B, max_ctx, _ptr(ctx_lens),
                                       _ptr(caches.k_ptrs), _ptr(caches.v_ptrs), _ptr(q), _dt(q), F16,
                                       _ptr(out), ws_ptr, ws_bytes, _stream(stream))
    _check("lmx_attn_decode_batched", rc)
    return out


def dop(*, n_tok, n_vh, n_kh, s_dim, scale=None) -> Dop:
    key_dim, d_inner = n_kh * s_dim, n_vh * s_dim
    scale = 1.0 / math.sqrt(s_dim) if scale is None else scale
    return Dop(n_tok, 2 * key_dim + d_inner, key_dim, d_inner, s_dim, n_vh, n_kh, scale)


def delta_recur(conv, alpha, beta, state, ssm_a, dt_bias, *, n_vh, n_kh, s_dim, out=None,
                stream=None):
    """Token-sequential gated delta rule (deltanet.wgsl:193-239).  ``state``
    [n_vh, s_dim, s_dim] f32 is updated in place; returns out [t, d_inner]."""
    torch = _torch()
    _need_cuda(conv, alpha, beta, state, ssm_a, dt_bias, out)
    op = dop(n_tok=conv.shape[0], n_vh=n_vh, n_kh=n_kh, s_dim=s_dim)
    if out is None:
        out = torch.empty((conv.shape[0], op.d_inner), dtype=torch.float32, device=conv.device)
    rc = lib().lmx_deltanet_recur(ctypes.byref(op), _ptr(ssm_a), _ptr(dt_bias), _ptr(alpha),
                                  _ptr(beta), _ptr(conv), _ptr(state), _ptr(out), _stream(stream))
    _check("lmx_deltanet_recur", rc)
    return out


def delta_chunked(conv, alpha, beta, state, ssm_a, dt_bias, *, n_vh, n_kh, s_dim, chunk=64,
                  out=None, workspace: Optional[Workspace] = None, stream=None):
    """Chunked gated delta rule; same contract as :func:`delta_recur`."""
    torch = _torch()
    _need_cuda(conv, alpha, beta, state, ssm_a, dt_bias, out)
    op = dop(n_tok=conv.shape[0], n_vh=n_vh, n_kh=n_kh, s_dim=s_dim)
    if out is None:
        out = torch.empty((conv.shape[0], op.d_inner), dtype=torch.float32, device=conv.device)
    need = lib().lmx_deltanet_chunked_workspace_bytes(ctypes.byref(op), chunk)
    ws_ptr, ws_bytes = None, 0
    if need:
        workspace = workspace or Workspace(device=conv.device)
        workspace.ensure(need, stream)
        ws_ptr, ws_bytes = workspace.base, workspace.nbytes
    rc = lib().lmx_deltanet_chunked(ctypes.byref(op), _ptr(ssm_a), _ptr(dt_bias), _ptr(alpha),
                                    _ptr(beta), _ptr(conv), _ptr(state), _ptr(out), chunk, ws_ptr,
                                    ws_bytes, _stream(stream))
    _check("lmx_deltanet_chunked", rc)
    return out


def delta_front(x, taps, conv_state, conv_out=None, *, key_dim: int, s_dim: int,
                eps: float = 1e-6, stream=None):
    """Causal depthwise conv + SiLU, conv-window update and q/k L2 norm
    (qwen35/cpu.rs:193-216).  x [t, conv_dim], taps [conv_dim, kernel],
    conv_state [kernel-1, conv_dim] (updated).  Returns conv_out [t, conv_dim]."""
    torch = _torch()
    _need_cuda(x, taps, conv_state, conv_out)
    t, conv_dim = x.shape
    if conv_out is None:
        conv_out = torch.empty_like(x)
    d = DeltaFrontDesc(t, conv_dim, key_dim, s_dim, taps.shape[-1], eps)
    rc = lib().lmx_deltanet_front(ctypes.byref(d), _ptr(x), _ptr(taps), _ptr(conv_state),
                                  _ptr(conv_out), _stream(stream))
    _check("lmx_deltanet_front", rc)
    return conv_out


def delta_back(o, z, w, *, n_vh: int, s_dim: int, eps: float = 1e-6, stream=None):
    """Gated RMS norm (qwen35/cpu.rs:250-259), in place on o [t, n_vh*s_dim]."""
    _need_cuda(o, z, w)
    d = DeltaBackDesc(o.shape[0], n_vh, s_dim, eps)
    rc = lib().lmx_deltanet_back(ctypes.byref(d), _ptr(o), _ptr(z), _ptr(w), _stream(stream))
    _check("lmx_deltanet_back", rc)
    return o


# ------------------------------------------------------ quantized matvec --
def matvec(w, x, *, qtype, rows: int, in_dim: int, y=None, stream=None):
    """y [n_tok, rows] = W x[t] for W in ggml's on-disk block layout (uint8
    device tensor), x [n_tok, in_dim] f32 (quant.rs:187-271 ``dot_row``)."""
    torch = _torch()
    _need_cuda(w, x, y)
    ty = QTYPES[qtype] if isinstance(qtype, str) else int(qtype)
    n_tok = x.numel() // in_dim
    if y is None:
        y = torch.empty((n_tok, rows), dtype=torch.float32, device=x.device)
    d = QmvDesc(ty, rows, in_dim, n_tok)
    _check("lmx_matvec", lib().lmx_matvec(ctypes.byref(d), _ptr(w), _ptr(x), _ptr(y), _stream(stream)))
    return y


# --------------------------------------------------------------- KV manager --
def _i32s(xs) -> Tuple[ctypes.Array, int]:
    xs = list(xs)
    return (ctypes.c_int32 * max(1, len(xs)))(*xs), len(xs)


class KvManager:
    """Bookkeeping of many sequences' f16 KV caches in one device arena
    (lmx_kvm_*, include/lmx/attn.h): the reference's per-session KvCache
    (cache.rs:65-154) and prefix reuse (session.rs:497-513, 546-570), one per
    sequence slot.

    ``layers`` lists ``(window, kv_dim, kv_source)`` per layer (window 0 for a
    global layer, kv_source -1 for a layer owning its cache).  The arena is a
    zeroed device tensor unless ``arena=(address, nbytes)`` names caller memory.
    """

    def __init__(self, layers, *, n_ctx: int, max_seqs: int, arena=None, device=None):
        self._layers = (KvmLayer * len(layers))(*[KvmLayer(w, d, s) for (w, d, s) in layers])
        self.desc = KvmDesc(len(layers), n_ctx, max_seqs, self._layers)
        self.n_ctx, self.max_seqs = n_ctx, max_seqs
        self.arena_bytes = lib().lmx_kvm_arena_bytes(ctypes.byref(self.desc))
        if not self.arena_bytes:
            raise ValueError("invalid KV manager layout")
        self.arena_t = None
        if arena is None:
            torch = _torch()
            self.arena_t = torch.zeros(self.arena_bytes + 256, dtype=torch.uint8,
                                       device=device or torch.device("cuda"))
            self._off = (-self.arena_t.data_ptr()) % 256
            base, nbytes = self.arena_t.data_ptr() + self._off, self.arena_bytes
        else:
            base, nbytes = arena
        self.base = base
        self.h = ctypes.c_void_p()
        _check("lmx_kvm_create", lib().lmx_kvm_create(ctypes.byref(self.desc), base, nbytes,
                                                      ctypes.byref(self.h)))

    def __del__(self):
        h = getattr(self, "h", None)
        if h and h.value and _lib is not None:
            _lib.lmx_kvm_destroy(h)
            self.h = ctypes.c_void_p()

    def open(self) -> int:
        s = ctypes.c_int32()
        _check("lmx_kvm_open", lib().lmx_kvm_open(self.h, ctypes.byref(s)))
        return s.value

    def close(self, seq: int) -> None:
        _check("lmx_kvm_close", lib().lmx_kvm_close(self.h, seq))

    def len(self, seq: int) -> int:
        n = ctypes.c_uint32()
        _check("lmx_kvm_len", lib().lmx_kvm_len(self.h, seq, ctypes.byref(n)))
        return n.value

    def reusable_prefix(self, seq: int, tokens) -> int:
        arr, n = _i32s(tokens)
        r = ctypes.c_uint32()
        _check("lmx_kvm_reusable_prefix", lib().lmx_kvm_reusable_prefix(self.h, seq, arr, n,
                                                                        ctypes.byref(r)))
        return r.value

    def begin(self, seq: int, tokens, stream=None) -> int:
        arr, n = _i32s(tokens)
        r = ctypes.c_uint32()
        _check("lmx_kvm_begin", lib().lmx_kvm_begin(self.h, seq, arr, n, ctypes.byref(r),
                                                    _stream(stream)))
        return r.value

    def commit(self, seq: int, tokens=None, n: Optional[int] = None) -> None:
        if tokens is None:
            rc = lib().lmx_kvm_commit(self.h, seq, None, int(n))
        else:
            arr, cnt = _i32s(tokens)
            rc = lib().lmx_kvm_commit(self.h, seq, arr, cnt)
        _check("lmx_kvm_commit", rc)

    def truncate(self, seq: int, pos: int) -> None:
        _check("lmx_kvm_truncate", lib().lmx_kvm_truncate(self.h, seq, pos))

    def wipe(self, seq: int, stream=None) -> None:
        _check("lmx_kvm_wipe", lib().lmx_kvm_wipe(self.h, seq, _stream(stream)))

    def layer_cache(self, seq: int, layer: int):
        """(k address, v address, n_slots, window) of the layer's caches."""
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        slots, win = ctypes.c_uint32(), ctypes.c_uint32()
        _check("lmx_kvm_layer_cache", lib().lmx_kvm_layer_cache(
            self.h, seq, layer, ctypes.byref(k), ctypes.byref(v), ctypes.byref(slots),
            ctypes.byref(win)))
        return k.value, v.value, slots.value, win.value

    def layer_tensors(self, seq: int, layer: int):
        """f16 [n_slots, kv_dim] views of the layer's K and V caches in the arena."""
        torch = _torch()
        if self.arena_t is None:
            raise ValueError("caller-owned arena: use layer_cache() addresses")
        k, v, slots, _ = self.layer_cache(seq, layer)
        kv_dim = self._kv_dim(layer)
        views = []
        for addr in (k, v):
            off = addr - self.arena_t.data_ptr()
            views.append(self.arena_t[off:off + slots * kv_dim * 2].view(torch.float16)
                         .view(slots, kv_dim))
        return views[0], views[1]

    def _kv_dim(self, layer: int) -> int:
        L = self._layers[layer]
        while L.kv_source >= 0:
            L = self._layers[L.kv_source]
        return L.kv_dim

    def batch(self, layer: int, seqs, extra: int = 1):
        """Host tables for lmx_attn_decode_batched: (k_ptrs, v_ptrs, ctx_lens, max_ctx)."""
        arr, n = _i32s(seqs)
        kp, vp = (ctypes.c_void_p * n)(), (ctypes.c_void_p * n)()
        cl, mx = (ctypes.c_int32 * n)(), ctypes.c_int32()
        _check("lmx_kvm_batch", lib().lmx_kvm_batch(self.h, layer, arr, n, extra, kp, vp, cl,
                                                    ctypes.byref(mx)))
        return list(kp), list(vp), list(cl), mx.value

