"""Independent float64 formulations used only to pin the C oracle.

TEST INFRASTRUCTURE ONLY.  These are written from the mathematics, not from
the reference's loops: attention is ``softmax(scale * Q K^T + mask) V`` with
the mask built as a boolean matrix; the delta rule is the matrix recurrence
``S_t = g_t S_{t-1} (I - b_t k_t k_t^T) + b_t v_t k_t^T``; the chunked delta rule
is the WY/UT form.  None of them shares code with lmx_oracle.c.
"""
from __future__ import annotations

import numpy as np


def mask_matrix(t: int, n_keys: int, base_pos: int, window: int, bidi: bool) -> np.ndarray:
    """Boolean [t, n_keys]: query i (at base_pos+i) may see key position p.

    Causal window: p in [pos-w+1, pos] (or [0, pos] when w == 0).  With bidi the
    upper edge becomes the batch end, still within w-1 ahead of the query.
    """
    pos = base_pos + np.arange(t)[:, None]
    p = np.arange(n_keys)[None, :]
    ok = p <= pos
    if bidi:
        end = base_pos + t - 1
        ok = np.broadcast_to(p <= end, (t, n_keys)).copy()
        if window:
            ok &= p <= pos + window - 1
    if window:
        ok &= p >= pos - window + 1
    return ok


def attention(q, k, v, *, n_heads, n_kv_heads, head_dim, base_pos, window=0,
              bidi=False, scale=None):
    """float64 GQA attention over keys indexed by absolute position."""
    q = np.asarray(q, np.float64).reshape(-1, n_heads, head_dim)
    t = q.shape[0]
    k = np.asarray(k, np.float64).reshape(-1, n_kv_heads, head_dim)
    v = np.asarray(v, np.float64).reshape(-1, n_kv_heads, head_dim)
    n_keys = k.shape[0]
    scale = 1.0 / np.sqrt(head_dim) if scale is None else float(scale)
    g = n_heads // n_kv_heads
    kh = np.repeat(k, g, axis=1)  # [n_keys, H, hd], head h reads kv head h // g
    vh = np.repeat(v, g, axis=1)
    s = np.einsum("thd,phd->htp", q, kh) * scale
    m = mask_matrix(t, n_keys, base_pos, window, bidi)[None]
    s = np.where(m, s, -np.inf)
    mx = s.max(axis=-1, keepdims=True)
    e = np.where(m, np.exp(s - mx), 0.0)
    p = e / e.sum(axis=-1, keepdims=True)
    o = np.einsum("htp,phd->thd", p, vh)
    return o.reshape(t, n_heads * head_dim)


def softplus(x):
    x = np.asarray(x, np.float64)
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def gates(alpha, beta, ssm_a, dt_bias):
    """Per (token, v-head) decay g = exp(a * softplus(alpha + dt)), mix sigmoid(beta)."""
    g = np.exp(np.asarray(ssm_a, np.float64)[None] * softplus(np.asarray(alpha, np.float64) + np.asarray(dt_bias, np.float64)[None]))
    b = 1.0 / (1.0 + np.exp(-np.asarray(beta, np.float64)))
    return g, b


def delta_recur(conv, alpha, beta, S, *, n_vh, n_kh, s_dim, ssm_a=None, dt_bias=None):
    """float64 matrix form: S <- g S (I - b k k^T) + b v k^T ; o = S q / sqrt(d)."""
    conv = np.asarray(conv, np.float64)
    n_tok = conv.shape[0]
    key_dim = n_kh * s_dim
    ssm_a = -np.ones(n_vh) if ssm_a is None else ssm_a
    dt_bias = np.zeros(n_vh) if dt_bias is None else dt_bias
    g, b = gates(np.asarray(alpha).reshape(n_tok, n_vh), np.asarray(beta).reshape(n_tok, n_vh), ssm_a, dt_bias)
    S = np.asarray(S, np.float64).reshape(n_vh, s_dim, s_dim).copy()
    out = np.zeros((n_tok, n_vh * s_dim))
    eye = np.eye(s_dim)
    for t in range(n_tok):
        for hv in range(n_vh):
            hk = hv % n_kh
            q = conv[t, hk * s_dim:(hk + 1) * s_dim]
            k = conv[t, key_dim + hk * s_dim:key_dim + (hk + 1) * s_dim]
            v = conv[t, 2 * key_dim + hv * s_dim:2 * key_dim + (hv + 1) * s_dim]
            S[hv] = g[t, hv] * S[hv] @ (eye - b[t, hv] * np.outer(k, k)) + b[t, hv] * np.outer(v, k)
            out[t, hv * s_dim:(hv + 1) * s_dim] = S[hv] @ q / np.sqrt(s_dim)
    return out, S.reshape(-1)


def delta_chunked(conv, alpha, beta, S, *, n_vh, n_kh, s_dim, chunk, ssm_a=None, dt_bias=None):
    """float64 chunked (WY/UT) form of the same recurrence.

    Per chunk of C tokens with cumulative in-chunk decay gamma_t = prod g:
      A[t,i]  = b_t (gamma_t/gamma_i) k_t.k_i            (i < t)
      U       = (I+A)^-1 (diag(b) V - diag(b gamma) K S0^T)
      O       = diag(gamma) Q S0^T + (tril(QK^T) * gamma_t/gamma_i) U
      S_C     = gamma_C S0 + U^T diag(gamma_C/gamma) K
    """
    conv = np.asarray(conv, np.float64)
    n_tok = conv.shape[0]
    key_dim = n_kh * s_dim
    ssm_a = -np.ones(n_vh) if ssm_a is None else ssm_a
    dt_bias = np.zeros(n_vh) if dt_bias is None else dt_bias
    g, b = gates(np.asarray(alpha).reshape(n_tok, n_vh), np.asarray(beta).reshape(n_tok, n_vh), ssm_a, dt_bias)
    S = np.asarray(S, np.float64).reshape(n_vh, s_dim, s_dim).copy()
    out = np.zeros((n_tok, n_vh * s_dim))
    for hv in range(n_vh):
        hk = hv % n_kh
        Q = conv[:, hk * s_dim:(hk + 1) * s_dim]
        K = conv[:, key_dim + hk * s_dim:key_dim + (hk + 1) * s_dim]
        V = conv[:, 2 * key_dim + hv * s_dim:2 * key_dim + (hv + 1) * s_dim]
        S0 = S[hv]
        for c0 in range(0, n_tok, chunk):
            c1 = min(n_tok, c0 + chunk)
            Qc, Kc, Vc = Q[c0:c1], K[c0:c1], V[c0:c1]
            lg = np.cumsum(np.log(g[c0:c1, hv]))
            bc = b[c0:c1, hv]
            n = c1 - c0
            lower = np.tril(np.ones((n, n), bool))
            # gamma_t / gamma_i on and below the diagonal, 0 above (never exp'd)
            ratio = np.where(lower, np.exp(np.where(lower, lg[:, None] - lg[None, :], 0.0)), 0.0)
            A = np.tril(bc[:, None] * ratio * (Kc @ Kc.T), -1)
            gam = np.exp(lg)
            rhs = bc[:, None] * Vc - (bc * gam)[:, None] * (Kc @ S0.T)
            U = np.linalg.solve(np.eye(n) + A, rhs)
            P = np.tril(Qc @ Kc.T) * ratio
            O = gam[:, None] * (Qc @ S0.T) + P @ U
            out[c0:c1, hv * s_dim:(hv + 1) * s_dim] = O / np.sqrt(s_dim)
            S0 = gam[-1] * S0 + (U * np.exp(lg[-1] - lg)[:, None]).T @ Kc
        S[hv] = S0
    return out, S.reshape(-1)


def rope_neox(head, pos, base, factors=None):
    """NeoX rotation in closed form, float64: pair i is rotated by
    pos * base^(-2i/d) / factor_i (ops.rs:142-159)."""
    h = np.asarray(head, np.float64).copy()
    d = h.size
    half = d // 2
    i = np.arange(half, dtype=np.float64)
    f = np.ones(half) if factors is None else np.asarray(factors, np.float64)[:half]
    ang = pos * np.power(float(base), -2.0 * i / d) / f
    c, s = np.cos(ang), np.sin(ang)
    x0, x1 = h[:half].copy(), h[half:2 * half].copy()
    h[:half] = x0 * c - x1 * s
    h[half:2 * half] = x0 * s + x1 * c
    return h


def attn_prologue(q, k, v, *, n_heads, n_kv_heads, head_dim, base_pos, q_stride=None, n_rot=None,
                  v_norm=False, rms_eps=1e-6, rope_base=1e6, q_gain=None, k_gain=None,
                  rope_factors=None):
    """Float64 restatement of the per-head norm and rotation (cpu.rs:286-327;
    qwen35/cpu.rs:294-304).  Returns (q_out, k_out, v_out) before the f16 store."""
    q_stride = q_stride or head_dim
    n_rot = head_dim if n_rot is None else n_rot
    q = np.asarray(q, np.float64).reshape(-1, n_heads, q_stride).copy()
    t = q.shape[0]
    k = np.asarray(k, np.float64).reshape(t, n_kv_heads, head_dim).copy()
    v = np.asarray(v, np.float64).reshape(t, n_kv_heads, head_dim).copy()

    def rms(x, gain):
        x = x / np.sqrt(np.mean(x * x) + rms_eps)
        return x if gain is None else x * np.asarray(gain, np.float64)

    for i in range(t):
        pos = base_pos + i
        for h in range(n_heads):
            head = q[i, h, :head_dim]
            if q_gain is not None:
                head = rms(head, q_gain)
            if n_rot:
                head[:n_rot] = rope_neox(head[:n_rot], pos, rope_base, rope_factors)
            q[i, h, :head_dim] = head
        for h in range(n_kv_heads):
            head = k[i, h]
            if k_gain is not None:
                head = rms(head, k_gain)
            if n_rot:
                head[:n_rot] = rope_neox(head[:n_rot], pos, rope_base, rope_factors)
            k[i, h] = head
            if v_norm:
                v[i, h] = rms(v[i, h], None)
    return q.reshape(t, -1), k.reshape(t, -1), v.reshape(t, -1)


def delta_front(x, taps, state, *, key_dim, s_dim, eps=1e-6):
    """Float64 restatement: conv_out[i] = silu(sum_j w[:, j] * [state | x][i + j]),
    the window's last kernel-1 rows as the new state, q/k heads L2-normalized
    with the norm floored at eps."""
    x = np.asarray(x, np.float64)
    t, conv_dim = x.shape
    w = np.asarray(taps, np.float64).reshape(conv_dim, -1)
    kernel = w.shape[1]
    full = np.concatenate([np.asarray(state, np.float64).reshape(kernel - 1, conv_dim), x], axis=0)
    acc = np.zeros((t, conv_dim))
    for j in range(kernel):
        acc += full[j:j + t] * w[:, j]
    out = acc / (1.0 + np.exp(-acc))
    qk = out[:, :2 * key_dim].reshape(t, -1, s_dim)
    nrm = np.maximum(np.sqrt((qk * qk).sum(-1, keepdims=True)), eps)
    out[:, :2 * key_dim] = (qk / nrm).reshape(t, -1)
    return out, full[t:]


def attn_gate(out, gate, *, dim, gate_stride=None):
    """out * sigmoid(gate) in float64, gate row r at element r*gate_stride."""
    out = np.asarray(out, np.float64).reshape(-1, dim)
    gs = gate_stride or dim
    g = np.stack([np.asarray(gate, np.float64).reshape(-1)[r * gs:r * gs + dim]
                  for r in range(out.shape[0])])
    return out / (1.0 + np.exp(-g))


def delta_back(o, z, w, *, n_vh, s_dim, eps=1e-6):
    o = np.asarray(o, np.float64).reshape(-1, n_vh, s_dim)
    z = np.asarray(z, np.float64).reshape(o.shape)
    o = o / np.sqrt((o * o).mean(-1, keepdims=True) + eps) * np.asarray(w, np.float64)
    return (o * (z / (1.0 + np.exp(-z)))).reshape(o.shape[0], -1)


# ------------------------------------------------------------- k-quants --
def _f16(lo, hi):
    return np.frombuffer(np.stack([lo, hi], -1).astype(np.uint8).tobytes(), np.float16).astype(np.float64)


def dequant(ty, data, n):
    """ggml's block layouts decoded in float64, vectorized over blocks (a
    second, independent reading of the formats quant.rs:12-128 describes)."""
    data = np.asarray(data, np.uint8)
    if ty == 0:
        return np.frombuffer(data.tobytes(), np.float32)[:n].astype(np.float64)
    if ty == 1:
        return np.frombuffer(data.tobytes(), np.float16)[:n].astype(np.float64)
    if ty == 30:
        u = np.frombuffer(data.tobytes(), np.uint16)[:n].astype(np.uint32) << 16
        return u.view(np.float32).astype(np.float64)
    if ty == 8:  # Q8_0: f16 d, 32 x i8
        b = data.reshape(-1, 34)
        d = _f16(b[:, 0], b[:, 1])
        q = b[:, 2:].view(np.int8).astype(np.float64)
        return (d[:, None] * q).reshape(-1)[:n]
    if ty == 12:  # Q4_K: f16 d, f16 dmin, 12 bytes of 6-bit (scale, min), 128 nibble bytes
        b = data.reshape(-1, 144)
        d, dmin = _f16(b[:, 0], b[:, 1]), _f16(b[:, 2], b[:, 3])
        q = b[:, 4:16].astype(np.int64)
        sc = np.zeros((b.shape[0], 8), np.int64)
        mn = np.zeros((b.shape[0], 8), np.int64)
        sc[:, :4], mn[:, :4] = q[:, 0:4] & 63, q[:, 4:8] & 63
        sc[:, 4:] = (q[:, 8:12] & 15) | ((q[:, 0:4] >> 6) << 4)
        mn[:, 4:] = (q[:, 8:12] >> 4) | ((q[:, 4:8] >> 6) << 4)
        nib = b[:, 16:].reshape(-1, 4, 32).astype(np.int64)
        vals = np.stack([nib & 15, nib >> 4], 2).reshape(-1, 8, 32)  # sub-block 2p low, 2p+1 high
        out = d[:, None, None] * sc[:, :, None] * vals - dmin[:, None, None] * mn[:, :, None]
        return out.reshape(-1)[:n]
    if ty == 14:  # Q6_K: 128 low-nibble bytes, 64 high-bit bytes, 16 i8 scales, f16 d
        b = data.reshape(-1, 210)
        d = _f16(b[:, 208], b[:, 209])
        scales = b[:, 192:208].view(np.int8).astype(np.int64)
        out = np.zeros((b.shape[0], 256))
        for h in range(2):
            ql = b[:, h * 64:h * 64 + 64].astype(np.int64)
            qh = b[:, 128 + h * 32:128 + h * 32 + 32].astype(np.int64)
            for g in range(4):  # element 128h + 32g + l
                low = (ql[:, :32] if g % 2 == 0 else ql[:, 32:])
                low = (low & 15) if g < 2 else (low >> 4)
                q = (low | (((qh >> (2 * g)) & 3) << 4)) - 32
                s = scales[:, 8 * h + 2 * g + (np.arange(32) // 16)]
                out[:, 128 * h + 32 * g:128 * h + 32 * g + 32] = d[:, None] * s * q
        return out.reshape(-1)[:n]
    raise ValueError(ty)

