// Attention prologue on gfx950: per-head RMS norm, NeoX rotation and the f16
// KV store in one launch.
//
// Replaces the chain the reference records in front of attention: rms_norm
// over Q heads, rope over Q, rms_norm over K heads, rope over K, (Gemma)
// rms_norm over V heads, then write_cache for K and for V (ops.wgsl:49-91,
// 186-218, 269-306, 323-346), each a separate dispatch with its own pass over
// the activations.  Here one workgroup owns one token: it builds the token's
// cos/sin table once (the angle depends on the position and the pair, not on
// the head), then its four waves take the token's Q, K and V head rows in
// turn.  A row is read once, normalized in registers (DPP wave reduction),
// rotated with its pair partner taken from the same lane, a neighbour lane
// or LDS depending on n_rot, and written once: Q back in place as f32, K and
// V straight into the f16 caches.
//
// Angles follow ops.rs:142-159 in double: pair i's angle is pos * s^i with
// s = base^(-2/n_rot) from the same libm pow, divided by the pair's factor,
// and sin / cos are rounded to float.  The reference forms s^i by i
// successive products, this kernel by the bits of i (at most 8 products from
// s^(2^k) the host squares out), so the doubles agree to a few ulps
// (relative 1e-15, i.e. 3e-11 rad at position 32k) and the float sin / cos
// agree unless that lands on a float rounding boundary.  The RMS scale is
// v_rsq_f32 (1 ulp).
#include <cmath>

#include "common.hpp"

namespace lmx {

struct PrologueArgs {
    float* q;
    const float* k;
    const float* v;
    const float* q_gain;
    const float* k_gain;
    const float* factors;
    f16* k_cache;
    f16* v_cache;
    int n_tokens, H, Hkv, hd, q_stride, n_rot, base_pos, window, v_norm;
    float eps;
    double scale_pow[8];  // s^(2^k), s = base^(-2/n_rot): pair i's angle is pos * s^i
};

// NJ = head_dim / 64: lane l holds dims l + 64 j of a row.
template <int NJ>
__global__ __launch_bounds__(256) void attn_prologue_kernel(PrologueArgs a) {
    constexpr int HD = 64 * NJ;
    constexpr int RB = 24 / NJ;  // rows of one batch held in registers (24 VGPRs)
    __shared__ float cs_tab[HD / 2], sn_tab[HD / 2];
    __shared__ float row_s[4][HD];
    const int tok = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pos = a.base_pos + tok;
    const int half = a.n_rot / 2;
    const int kv_dim = a.Hkv * HD;
    // With a ring, a later token of this call that maps to the same slot
    // overwrites this one (the reference stores rows in order): skip it.
    const bool store = !a.window || tok + a.window >= a.n_tokens;
    const size_t slot = a.window ? (size_t)(pos % a.window) : (size_t)pos;
    const int n_rows = a.H + 2 * a.Hkv;
    // Row r of this token: query head r, K head r - H, or V head r - H - Hkv.
    auto row_src = [&](int r) -> const float* {
        if (r < a.H) return a.q + ((size_t)tok * a.H + r) * a.q_stride;
        if (r < a.H + a.Hkv) return a.k + (size_t)tok * kv_dim + (r - a.H) * HD;
        return a.v + (size_t)tok * kv_dim + (r - a.H - a.Hkv) * HD;
    };

    // The gains, then the wave's rows w, w + 4, ... (a batch of up to RB) are
    // requested before any store, right after the angle table is built, so
    // they are in flight across the table's barrier.  (Issued before the
    // table, they kept 32 row registers live through its double-precision
    // sincos: 110 VGPRs, 4 waves a SIMD, against 78 and 6 this way.)  On gfx9
    // a store and a later load share one counter, so waiting on a load issued
    // after a store waits for the store too; here each batch waits once,
    // before its first store.
    float qg[NJ], kg[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) qg[j] = kg[j] = 1.f;
    if (a.q_gain)
#pragma unroll
        for (int j = 0; j < NJ; ++j) qg[j] = a.q_gain[lane + 64 * j];
    if (a.k_gain)
#pragma unroll
        for (int j = 0; j < NJ; ++j) kg[j] = a.k_gain[lane + 64 * j];
    float xb[RB][NJ];
    auto load_batch = [&](int r0) {
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            const int r = r0 + 4 * b;
            if (r < n_rows && (r < a.H || store)) {  // uniform per wave
                const float* src = row_src(r);
#pragma unroll
                for (int j = 0; j < NJ; ++j) xb[b][j] = src[lane + 64 * j];
            }
        }
    };
    for (int i = tid; i < half; i += 256) {
        double theta = (double)pos;  // pos * s^i by the bits of i (i < 256)
#pragma unroll
        for (int k = 0; k < 8; ++k) theta *= (i >> k) & 1 ? a.scale_pow[k] : 1.0;
        double ang = theta;
        if (a.factors) ang = theta / (double)a.factors[i];  // the load is waited on here only
        double s, c;
        sincos(ang, &s, &c);
        cs_tab[i] = (float)c;
        sn_tab[i] = (float)s;
    }
    load_batch(w);
    __syncthreads();

    // Rotation of dim d with its partner p (d + half below half, d - half
    // above): out = x cos + p sin', with sin' = -sin below half.  The partner
    // sits in the same lane when half is a multiple of 64, in lane
    // d +- half of register 0 when n_rot <= 64, else it goes through LDS.
    const int mode = half == 0 ? 0 : (half % 64 == 0 ? 1 : (a.n_rot <= 64 ? 2 : 3));
    const int hj = half / 64;
    float cr[NJ], sr[NJ];
    bool rj[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int d = lane + 64 * j;
        rj[j] = d < a.n_rot;
        const int i = d < half ? d : d - half;
        cr[j] = rj[j] ? cs_tab[i] : 1.f;
        sr[j] = rj[j] ? (d < half ? -sn_tab[i] : sn_tab[i]) : 0.f;
    }
    const int xlane = lane < half ? lane + half : lane - half;

    for (int r0 = w; r0 < n_rows; r0 += 4 * RB) {
        if (r0 != w) load_batch(r0);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the batch is in registers
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            const int r = r0 + 4 * b;
            if (r >= n_rows) continue;  // uniform per wave
            const bool is_q = r < a.H, is_k = !is_q && r < a.H + a.Hkv;
            if (!is_q && !store) continue;  // uniform per wave
            const bool has_gain = is_q ? a.q_gain != nullptr : (is_k && a.k_gain != nullptr);
            const bool norm = (is_q || is_k) ? has_gain : a.v_norm != 0;
            float* x = xb[b];
            if (norm) {
                // ops.rs:40-47: x / sqrt(mean(x^2) + eps), then the gain
                float ss = 0.f;
#pragma unroll
                for (int j = 0; j < NJ; ++j) ss += x[j] * x[j];
                const float sc = __builtin_amdgcn_rsqf(wave_sum64(ss) / (float)HD + a.eps);
#pragma unroll
                for (int j = 0; j < NJ; ++j) x[j] *= sc;
                if (has_gain)
#pragma unroll
                    for (int j = 0; j < NJ; ++j) x[j] *= is_q ? qg[j] : kg[j];
            }
            if ((is_q || is_k) && mode != 0) {
                float p[NJ];
                if (mode == 1) {
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        p[j] = 0.f;
#pragma unroll
                        for (int j2 = 0; j2 < NJ; ++j2) {
                            if (j < hj && j2 == j + hj) p[j] = x[j2];
                            if (j >= hj && j < 2 * hj && j2 + hj == j) p[j] = x[j2];
                        }
                    }
                } else if (mode == 2) {
                    p[0] = __shfl(x[0], xlane, 64);
#pragma unroll
                    for (int j = 1; j < NJ; ++j) p[j] = 0.f;
                } else {
#pragma unroll
                    for (int j = 0; j < NJ; ++j) row_s[w][lane + 64 * j] = x[j];
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        const int d = lane + 64 * j;
                        p[j] = rj[j] ? row_s[w][d < half ? d + half : d - half] : 0.f;
                    }
                    // the slot is rewritten by this wave's next row only after these reads
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                }
#pragma unroll
                for (int j = 0; j < NJ; ++j) x[j] = rj[j] ? x[j] * cr[j] + p[j] * sr[j] : x[j];
            }
            if (is_q) {
                float* dst = a.q + ((size_t)tok * a.H + r) * a.q_stride;
#pragma unroll
                for (int j = 0; j < NJ; ++j) dst[lane + 64 * j] = x[j];
            } else {
                f16* dst = (is_k ? a.k_cache + (r - a.H) * HD : a.v_cache + (r - a.H - a.Hkv) * HD) +
                           slot * kv_dim;
#pragma unroll
                for (int j = 0; j < NJ; ++j) dst[lane + 64 * j] = (f16)x[j];
            }
        }
    }
}

lmx_status attn_prologue(const lmx_prologue_desc* d, float* q, const float* k_new,
                         const float* v_new, const float* q_gain, const float* k_gain,
                         const float* rope_factors, void* k_cache, void* v_cache,
                         hipStream_t st) {
    PrologueArgs a{};
    a.q = q;
    a.k = k_new;
    a.v = v_new;
    a.q_gain = q_gain;
    a.k_gain = k_gain;
    a.factors = rope_factors;
    a.k_cache = static_cast<f16*>(k_cache);
    a.v_cache = static_cast<f16*>(v_cache);
    a.n_tokens = (int)d->n_tokens;
    a.H = (int)d->n_heads;
    a.Hkv = (int)d->n_kv_heads;
    a.hd = (int)d->head_dim;
    a.q_stride = (int)d->q_stride;
    a.n_rot = (int)d->n_rot;
    a.base_pos = (int)d->base_pos;
    a.window = (int)d->window;
    a.v_norm = (int)d->v_norm;
    a.eps = d->rms_eps;
    // ops.rs:145: (base as f64).powf(-2.0 / d as f64), d = the rotated length
    double s = d->n_rot ? std::pow((double)d->rope_base, -2.0 / (double)d->n_rot) : 1.0;
    for (int k = 0; k < 8; ++k, s *= s) a.scale_pow[k] = s;
    (void)hipGetLastError();
    const dim3 grid(d->n_tokens);
    switch (d->head_dim) {
        case 64: hipLaunchKernelGGL(attn_prologue_kernel<1>, grid, dim3(256), 0, st, a); break;
        case 128: hipLaunchKernelGGL(attn_prologue_kernel<2>, grid, dim3(256), 0, st, a); break;
        case 256: hipLaunchKernelGGL(attn_prologue_kernel<4>, grid, dim3(256), 0, st, a); break;
        case 512: hipLaunchKernelGGL(attn_prologue_kernel<8>, grid, dim3(256), 0, st, a); break;
        default: return LMX_E_UNSUPPORTED;
    }
    LMX_CHECK_LAUNCH();
    return LMX_OK;
}

}  // namespace lmx
