"""CPU oracle for llmoxide's attention hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg import this package, and only as the checker (or the timed CPU baseline),
never as the thing measured or shipped.  The product path (``llmoxide_amd``)
never imports it and fails loudly when its HIP library is missing.

Two layers:

* ``liblmx_oracle.so`` (``lmx_oracle.c``): the C restatement of the reference's
  scalar loops, same loop and summation order in f32.  Reference lines are
  cited per function in the C file.
* ``textbook``: independent float64 NumPy formulations (matrix form, masks as
  boolean matrices) used only to pin the C restatement.  They share no code
  with it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liblmx_oracle.so")


def build(force: bool = False) -> str:
    """Compile liblmx_oracle.so with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH) or (
        os.path.getmtime(_LIB_PATH) < os.path.getmtime(os.path.join(_HERE, "lmx_oracle.c"))
    ):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _LIB_PATH


class OrcAttn(ctypes.Structure):
    _fields_ = [
        ("n_tokens", ctypes.c_uint32),
        ("n_heads", ctypes.c_uint32),
        ("n_kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("kv_dim", ctypes.c_uint32),
        ("base_pos", ctypes.c_uint32),
        ("window", ctypes.c_uint32),
        ("bidi", ctypes.c_uint32),
        ("scale", ctypes.c_float),
    ]


class OrcDop(ctypes.Structure):
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


class OrcPrologue(ctypes.Structure):
    _fields_ = [
        ("n_tokens", ctypes.c_uint32),
        ("n_heads", ctypes.c_uint32),
        ("n_kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("q_stride", ctypes.c_uint32),
        ("n_rot", ctypes.c_uint32),
        ("base_pos", ctypes.c_uint32),
        ("window", ctypes.c_uint32),
        ("v_norm", ctypes.c_uint32),
        ("rms_eps", ctypes.c_float),
        ("rope_base", ctypes.c_float),
    ]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.POINTER
        f32p, u16p = P(ctypes.c_float), P(ctypes.c_uint16)
        L.orc_fill_uniform.argtypes = [ctypes.c_uint64, f32p, ctypes.c_size_t]
        L.orc_fill_normal.argtypes = [ctypes.c_uint64, f32p, ctypes.c_size_t]
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_to_f16.argtypes = [f32p, u16p, ctypes.c_size_t]
        L.orc_from_f16.argtypes = [u16p, f32p, ctypes.c_size_t]
        L.orc_slot.argtypes = [ctypes.c_int64, ctypes.c_int64]
        L.orc_slot.restype = ctypes.c_int64
        L.orc_visible.argtypes = [ctypes.c_int64] * 4 + [ctypes.c_int, P(ctypes.c_int64), P(ctypes.c_int64)]
        L.orc_softmax.argtypes = [f32p, ctypes.c_size_t]
        L.orc_write_cache.argtypes = [ctypes.c_int64] * 4 + [f32p, u16p]
        L.orc_attention.argtypes = [P(OrcAttn), f32p, f32p, f32p, f32p, ctypes.c_int, ctypes.c_int]
        L.orc_attention.restype = ctypes.c_int
        L.orc_delta_recur.argtypes = [P(OrcDop)] + [f32p] * 7
        L.orc_delta_recur_mt.argtypes = [P(OrcDop)] + [f32p] * 7 + [ctypes.c_int]
        L.orc_l2_norm_rows.argtypes = [f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_float]
        L.orc_rms_norm_rows.argtypes = [f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_float]
        L.orc_rope_neox.argtypes = [f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_float, f32p,
                                    ctypes.c_int64]
        L.orc_attn_prologue.argtypes = [P(OrcPrologue), f32p, f32p, f32p, f32p, f32p, f32p, u16p, u16p]
        L.orc_delta_front.argtypes = [ctypes.c_int64] * 5 + [ctypes.c_float] + [f32p] * 4
        L.orc_delta_back.argtypes = [ctypes.c_int64] * 3 + [ctypes.c_float] + [f32p] * 3
        L.orc_attn_gate.argtypes = [ctypes.c_int64] * 3 + [f32p] * 2
        u8p = ctypes.POINTER(ctypes.c_uint8)
        L.orc_block_bytes.argtypes = [ctypes.c_int]
        L.orc_block_bytes.restype = ctypes.c_int64
        L.orc_block_elems.argtypes = [ctypes.c_int]
        L.orc_block_elems.restype = ctypes.c_int64
        L.orc_dequant.argtypes = [ctypes.c_int, u8p, ctypes.c_int64, f32p]
        L.orc_dot_row.argtypes = [ctypes.c_int, u8p, f32p, ctypes.c_int64]
        L.orc_dot_row.restype = ctypes.c_float
        L.orc_matvec.argtypes = [ctypes.c_int, u8p, ctypes.c_int64, ctypes.c_int64, f32p,
                                 ctypes.c_int64, f32p]
        _lib = L
    return _lib


def _f32p(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _u16p(a: np.ndarray):
    assert a.dtype == np.uint16 and a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))


# ------------------------------------------------------------------ inputs --
def uniform(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_fill_uniform(seed, _f32p(out), n)
    return out


def normal(seed: int, shape) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    lib().orc_fill_normal(seed, _f32p(out), n)
    return out.reshape(shape)


def to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_to_f16(_f32p(x), _u16p(out), x.size)
    return out


def from_f16_bits(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_from_f16(_u16p(h), _f32p(out), h.size)
    return out


def round_f16(x: np.ndarray) -> np.ndarray:
    """x rounded to the nearest f16 value, returned as f32."""
    return from_f16_bits(to_f16_bits(x))


def rms_norm_rows(x: np.ndarray, dim: int, eps: float = 1e-6) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).copy()
    lib().orc_rms_norm_rows(_f32p(x), x.size // dim, dim, eps)
    return x


def l2_norm_rows(x: np.ndarray, dim: int, eps: float = 1e-6) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).copy()
    lib().orc_l2_norm_rows(_f32p(x), x.size // dim, dim, eps)
    return x


# ------------------------------------------------------------- bookkeeping --
def slot(pos: int, window: int) -> int:
    return lib().orc_slot(pos, window)


def visible(pos: int, window: int, base_pos: int, n_tokens: int, bidi: bool):
    lo, hi = ctypes.c_int64(), ctypes.c_int64()
    lib().orc_visible(pos, window, base_pos, n_tokens, int(bidi), ctypes.byref(lo), ctypes.byref(hi))
    return lo.value, hi.value


def softmax(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).copy()
    lib().orc_softmax(_f32p(x), x.size)
    return x


def write_cache(src: np.ndarray, cache_bits: np.ndarray, base_pos: int, window: int) -> np.ndarray:
    """Store f32 rows src[t, kv_dim] into an f16 cache (bits), in place."""
    src = np.ascontiguousarray(src, np.float32)
    t, kv_dim = src.shape
    assert cache_bits.dtype == np.uint16 and cache_bits.shape[1] == kv_dim
    lib().orc_write_cache(t, kv_dim, base_pos, window, _f32p(src), _u16p(cache_bits))
    return cache_bits


# --------------------------------------------------------------- attention --
def attention(q, k, v, *, n_heads, n_kv_heads, head_dim, base_pos, window=0,
              bidi=False, scale=None, linear=True, n_threads=1, kv_dim=None):
    """Reference attention (cpu.rs:342-387; qwen35/cpu.rs:324-365).

    q: [t, H*hd] f32.  k, v: f32 rows, by absolute position when ``linear``
    (shape [>= base_pos+t, kv_dim]), else by ring slot (the reference's cache
    after its store).  Returns out [t, H*hd] f32.
    """
    q = np.ascontiguousarray(q, np.float32).reshape(-1, n_heads * head_dim)
    t = q.shape[0]
    kv_dim = kv_dim or n_kv_heads * head_dim
    k = np.ascontiguousarray(k, np.float32).reshape(-1, kv_dim)
    v = np.ascontiguousarray(v, np.float32).reshape(-1, kv_dim)
    p = OrcAttn(t, n_heads, n_kv_heads, head_dim, kv_dim, base_pos, window, int(bidi),
                float(np.float32(1.0) / np.sqrt(np.float32(head_dim))) if scale is None else float(scale))
    out = np.zeros((t, n_heads * head_dim), np.float32)
    rc = lib().orc_attention(ctypes.byref(p), _f32p(q), _f32p(k), _f32p(v), _f32p(out),
                             int(linear), int(n_threads))
    if rc != 0:
        raise ValueError("orc_attention: invalid shape")
    return out


def delta_recur(conv, alpha, beta, S, *, n_vh, n_kh, s_dim, ssm_a=None, dt_bias=None,
                n_threads=1):
    """Gated delta rule (qwen35/cpu.rs:218-245).  Returns (out, S_new).
    ``n_threads`` > 1 splits the independent v-heads over threads; each value
    is computed the same way."""
    conv = np.ascontiguousarray(conv, np.float32)
    n_tok, conv_dim = conv.shape
    key_dim, d_inner = n_kh * s_dim, n_vh * s_dim
    assert conv_dim == 2 * key_dim + d_inner
    alpha = np.ascontiguousarray(alpha, np.float32).reshape(n_tok, n_vh)
    beta = np.ascontiguousarray(beta, np.float32).reshape(n_tok, n_vh)
    ssm_a = np.full(n_vh, -1.0, np.float32) if ssm_a is None else np.ascontiguousarray(ssm_a, np.float32)
    dt_bias = np.zeros(n_vh, np.float32) if dt_bias is None else np.ascontiguousarray(dt_bias, np.float32)
    S = np.ascontiguousarray(S, np.float32).copy()
    out = np.zeros((n_tok, d_inner), np.float32)
    op = OrcDop(n_tok, conv_dim, key_dim, d_inner, s_dim, n_vh, n_kh,
                np.float32(1.0) / np.sqrt(np.float32(s_dim)))
    lib().orc_delta_recur_mt(ctypes.byref(op), _f32p(ssm_a), _f32p(dt_bias), _f32p(alpha),
                             _f32p(beta), _f32p(conv), _f32p(S), _f32p(out), int(n_threads))
    return out, S


def rope_neox(head, pos, base, factors=None):
    """NeoX rotation of one head's leading dims (ops.rs:142-159); returns a copy."""
    h = np.ascontiguousarray(head, np.float32).copy()
    f = None if factors is None else np.ascontiguousarray(factors, np.float32)
    lib().orc_rope_neox(_f32p(h), h.size, int(pos), float(base),
                        None if f is None else _f32p(f), 0 if f is None else f.size)
    return h


def attn_prologue(q, k, v, *, n_heads, n_kv_heads, head_dim, base_pos, n_slots, q_stride=None,
                  n_rot=None, window=0, v_norm=False, rms_eps=1e-6, rope_base=1e6, q_gain=None,
                  k_gain=None, rope_factors=None, k_cache=None, v_cache=None):
    """Norm / rotate / store of the attention inputs (cpu.rs:286-327;
    qwen35/cpu.rs:294-304).  q [t, H*q_stride], k and v [t, kv_dim] f32.
    Returns (q_out, k_cache_bits, v_cache_bits); the caches start as given
    (f16 bits, [n_slots, kv_dim]) or zero."""
    q_stride = q_stride or head_dim
    n_rot = head_dim if n_rot is None else n_rot
    kv_dim = n_kv_heads * head_dim
    q = np.ascontiguousarray(q, np.float32).copy()
    t = q.size // (n_heads * q_stride)
    k = np.ascontiguousarray(k, np.float32).reshape(t, kv_dim).copy()
    v = np.ascontiguousarray(v, np.float32).reshape(t, kv_dim).copy()
    kc = np.zeros((n_slots, kv_dim), np.uint16) if k_cache is None else np.ascontiguousarray(k_cache, np.uint16).copy()
    vc = np.zeros((n_slots, kv_dim), np.uint16) if v_cache is None else np.ascontiguousarray(v_cache, np.uint16).copy()
    keep = [None if a is None else np.ascontiguousarray(a, np.float32) for a in (q_gain, k_gain, rope_factors)]
    p = OrcPrologue(t, n_heads, n_kv_heads, head_dim, q_stride, n_rot, base_pos, window,
                    int(bool(v_norm)), rms_eps, rope_base)
    lib().orc_attn_prologue(ctypes.byref(p), _f32p(q), _f32p(k), _f32p(v),
                            *[None if a is None else _f32p(a) for a in keep], _u16p(kc), _u16p(vc))
    return q, kc, vc


def delta_front(x, taps, state, *, key_dim, s_dim, eps=1e-6):
    """Causal depthwise conv + SiLU, conv-window shift and q/k L2 norm of the
    delta-net input (qwen35/cpu.rs:193-216).  x [t, conv_dim], taps
    [conv_dim, kernel], state [kernel-1, conv_dim].  Returns (conv_out, state_new)."""
    x = np.ascontiguousarray(x, np.float32)
    t, conv_dim = x.shape
    taps = np.ascontiguousarray(taps, np.float32).reshape(conv_dim, -1)
    kernel = taps.shape[1]
    st = np.ascontiguousarray(state, np.float32).reshape(kernel - 1, conv_dim).copy()
    out = np.zeros_like(x)
    lib().orc_delta_front(t, conv_dim, key_dim, s_dim, kernel, eps, _f32p(x), _f32p(taps), _f32p(st),
                          _f32p(out))
    return out, st


def attn_gate(out, gate, *, dim, gate_stride=None):
    """Qwen3.5's attention output gate (qwen35/cpu.rs:359-363): each row of
    ``out`` [rows, dim] times sigmoid(gate row), the gate row r starting at
    element r*gate_stride of ``gate``.  Returns a new array."""
    out = np.ascontiguousarray(out, np.float32).reshape(-1, dim).copy()
    gate = np.ascontiguousarray(gate, np.float32).reshape(-1)
    gs = gate_stride or dim
    assert gate.size >= (out.shape[0] - 1) * gs + dim
    lib().orc_attn_gate(out.shape[0], dim, gs, _f32p(out), _f32p(gate))
    return out


def delta_back(o, z, w, *, n_vh, s_dim, eps=1e-6):
    """Gated RMS norm of the delta-net output (qwen35/cpu.rs:250-259): per
    token and v-head rms_norm(o) * w * silu(z).  Returns a new array."""
    o = np.ascontiguousarray(o, np.float32).copy()
    z = np.ascontiguousarray(z, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    t = o.size // (n_vh * s_dim)
    lib().orc_delta_back(t, n_vh, s_dim, eps, _f32p(o), _f32p(z), _f32p(w))
    return o


# ------------------------------------------------------------- k-quants --
# ggml type codes (GgmlType): the on-disk formats of crates/gguf/src/quant.rs.
F32_T, F16_T, Q8_0, Q4_K, Q6_K, BF16_T = 0, 1, 8, 12, 14, 30
QTYPES = {"f32": F32_T, "f16": F16_T, "q8_0": Q8_0, "q4_k": Q4_K, "q6_k": Q6_K, "bf16": BF16_T}


def _u8p(a: np.ndarray):
    assert a.dtype == np.uint8 and a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))


def block_geometry(ty: int):
    """(bytes, elements) per block of a type."""
    return int(lib().orc_block_bytes(ty)), int(lib().orc_block_elems(ty))


def row_bytes(ty: int, in_dim: int) -> int:
    bb, be = block_geometry(ty)
    assert in_dim % be == 0
    return in_dim // be * bb


def dequant(ty: int, data: np.ndarray, n: int) -> np.ndarray:
    """quant.rs:130-182: n elements decoded to f32."""
    data = np.ascontiguousarray(data, np.uint8)
    out = np.zeros(n, np.float32)
    lib().orc_dequant(ty, _u8p(data), n, _f32p(out))
    return out


def dot_row(ty: int, row: np.ndarray, x: np.ndarray) -> float:
    """quant.rs:187-271: fused decode-and-dot of one row."""
    row = np.ascontiguousarray(row, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    return float(lib().orc_dot_row(ty, _u8p(row), _f32p(x), x.size))


def matvec(ty: int, w: np.ndarray, rows: int, in_dim: int, x: np.ndarray) -> np.ndarray:
    """y[t, r] = dot_row(row r of w, x[t]); x [n_tok, in_dim]."""
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32).reshape(-1, in_dim)
    y = np.zeros((x.shape[0], rows), np.float32)
    if lib().orc_matvec(ty, _u8p(w), rows, in_dim, _f32p(x), x.shape[0], _f32p(y)):
        raise ValueError("orc_matvec: in_dim is not a whole number of blocks")
    return y


def quant_weights(ty: int, rows: int, in_dim: int, seed: int) -> np.ndarray:
    """Random blocks of a type with scales in a sane range (the recipe of the
    reference's quant.rs tests: patterned bytes, then f16 d (and dmin) set)."""
    bb, be = block_geometry(ty)
    n_blocks = rows * in_dim // be
    if ty in (F32_T, F16_T, BF16_T):
        vals = normal(seed, (rows * in_dim,)) * np.float32(0.05)
        if ty == F32_T:
            return vals.view(np.uint8).copy()
        if ty == F16_T:
            return to_f16_bits(vals).view(np.uint8).copy()
        return (vals.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).copy()
    raw = (uniform(seed, n_blocks * bb) * 256).astype(np.uint8).reshape(n_blocks, bb)
    d = to_f16_bits(np.abs(normal(seed + 1, (n_blocks,))) * np.float32(0.01) + np.float32(0.001))
    if ty == Q4_K:
        raw[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
        dm = to_f16_bits(np.abs(normal(seed + 2, (n_blocks,))) * np.float32(0.01))
        raw[:, 2:4] = dm.view(np.uint8).reshape(-1, 2)
    elif ty == Q6_K:
        raw[:, 208:210] = d.view(np.uint8).reshape(-1, 2)
    else:  # Q8_0
        raw[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    return np.ascontiguousarray(raw.reshape(-1))

