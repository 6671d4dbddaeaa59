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
// turn.  A row is read once, normalized in registers (wave reduction),
// staged in the wave's LDS slot for the pair exchange of the rotation, and
// written once: Q back in place as f32, K and V straight into the f16 caches.
//
// Angles follow ops.rs:142-159 exactly: theta starts at pos and is multiplied
// by base^(-2/n_rot) once per pair in double (the host passes the factor from
// the same libm pow), the pair's factor divides it in double, and sin / cos
// are rounded to float.
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
    double theta_scale;
};

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
    return x;
}

// NJ = head_dim / 64: lane l holds dims l + 64 j of a row.
template <int NJ>
__global__ __launch_bounds__(256) void attn_prologue_kernel(PrologueArgs a) {
    constexpr int HD = 64 * NJ;
    __shared__ float cs_tab[HD / 2], sn_tab[HD / 2];
    __shared__ float row_s[4][HD];
    const int tok = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pos = a.base_pos + tok;
    const int half = a.n_rot / 2;

    for (int i = tid; i < half; i += 256) {
        double theta = (double)pos;
        for (int j = 0; j < i; ++j) theta *= a.theta_scale;
        const double ang = theta / (a.factors ? (double)a.factors[i] : 1.0);
        cs_tab[i] = (float)cos(ang);
        sn_tab[i] = (float)sin(ang);
    }
    __syncthreads();

    const int kv_dim = a.Hkv * HD;
    // With a ring, a later token of this call that maps to the same slot
    // overwrites this one (the reference stores rows in order): skip it.
    const bool store = !a.window || tok + a.window >= a.n_tokens;
    const size_t slot = a.window ? (size_t)(pos % a.window) : (size_t)pos;
    const int n_rows = a.H + 2 * a.Hkv;
    for (int r = w; r < n_rows; r += 4) {
        const float* src;
        const float* gain = nullptr;
        bool norm, rot;
        float* dst32 = nullptr;
        f16* dst16 = nullptr;
        if (r < a.H) {
            dst32 = a.q + ((size_t)tok * a.H + r) * a.q_stride;
            src = dst32;
            gain = a.q_gain;
            norm = gain != nullptr;
            rot = true;
        } else if (r < a.H + a.Hkv) {
            const int h = r - a.H;
            src = a.k + (size_t)tok * kv_dim + h * HD;
            gain = a.k_gain;
            norm = gain != nullptr;
            rot = true;
            dst16 = a.k_cache + slot * kv_dim + h * HD;
        } else {
            const int h = r - a.H - a.Hkv;
            src = a.v + (size_t)tok * kv_dim + h * HD;
            norm = a.v_norm != 0;
            rot = false;
            dst16 = a.v_cache + slot * kv_dim + h * HD;
        }
        if (!dst32 && !store) continue;  // uniform per wave

        float x[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) x[j] = src[lane + 64 * j];
        if (norm) {
            // ops.rs:40-47: x / sqrt(mean(x^2) + eps), then the gain
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < NJ; ++j) ss += x[j] * x[j];
            const float sc = 1.f / sqrtf(wave_sum(ss) / (float)HD + a.eps);
#pragma unroll
            for (int j = 0; j < NJ; ++j) x[j] *= sc;
            if (gain)
#pragma unroll
                for (int j = 0; j < NJ; ++j) x[j] *= gain[lane + 64 * j];
        }
        if (rot && half > 0) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) row_s[w][lane + 64 * j] = x[j];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int d = lane + 64 * j;
                if (d < half) {
                    x[j] = row_s[w][d] * cs_tab[d] - row_s[w][d + half] * sn_tab[d];
                } else if (d < a.n_rot) {
                    const int i = d - half;
                    x[j] = row_s[w][i] * sn_tab[i] + row_s[w][d] * cs_tab[i];
                }
            }
            // the slot is rewritten by this wave's next row only after these reads
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        if (dst32) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) dst32[lane + 64 * j] = x[j];
        } else {
#pragma unroll
            for (int j = 0; j < NJ; ++j) dst16[lane + 64 * j] = (f16)x[j];
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
    a.theta_scale = d->n_rot ? std::pow((double)d->rope_base, -2.0 / (double)d->n_rot) : 1.0;
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
