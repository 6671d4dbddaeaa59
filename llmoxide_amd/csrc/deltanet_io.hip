// The delta-net's front and back on gfx950: the causal conv + SiLU + conv
// window + q/k L2 norm ahead of the recurrence, and the gated RMS norm after
// it.
//
// Front.  The reference runs four dispatches (conv_silu, conv_shift,
// conv_commit, l2norm_qk; deltanet.wgsl:54-173): the conv output makes a
// round trip through HBM before the norm, and the window update goes through
// a scratch copy so that no thread reads a row another one is overwriting.
// Here one workgroup owns a 128-channel block (one q/k head at s_dim 128)
// for a chunk of 64 tokens: each wave takes 16 consecutive tokens, a lane
// holds two channels (lane and lane + 64), the K-1 rows before the wave's
// tokens (from the batch, or before it from the window) and its own rows are
// loaded once into registers, the taps slide over them in the reference's
// order, and the head's L2 norm is a wave reduction, so each output row is
// written once.  Only the first chunk's workgroup of a block
// reads the old window, so it alone writes the new one, after its own reads:
// no workgroup ever reads a window row another one writes.
//
// Back.  rms_norm over each v-head then mul_silu (qwen35.rs:968-986): one
// wave per (token, v-head) row, one pass.
#include "common.hpp"

namespace lmx {

constexpr int kFrontTokens = 64;  // tokens per front workgroup (>= kernel - 1)

__device__ __forceinline__ float silu_f(float x) { return x / (1.f + expf(-x)); }

struct FrontArgs {
    const float* x;
    const float* taps;
    float* state;
    float* out;
    int n_tok, conv_dim, key_dim, s_dim, kernel;
    float eps;
};

template <int K>
__global__ __launch_bounds__(256) void delta_front_kernel(FrontArgs a) {
    const int cb = blockIdx.x, tc = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c0 = cb * 128 + lane, c1 = c0 + 64;
    const bool qk = cb * 128 < 2 * a.key_dim;  // the block lies in q|k (key_dim % 64 == 0)
    float t0[K], t1[K];
#pragma unroll
    for (int j = 0; j < K; ++j) {
        t0[j] = a.taps[(size_t)c0 * K + j];
        t1[j] = a.taps[(size_t)c1 * K + j];
    }
    // Wave w takes tokens [tok0, tok0 + 16) of the chunk: the K-1 rows before
    // tok0 and its 16 rows are loaded once, into registers, and the taps slide
    // over them (each batch row is read once per wave, not K times).
    constexpr int NT = kFrontTokens / 4;
    const int tok0 = tc * kFrontTokens + NT * w;
    const int nt = min(NT, a.n_tok - tok0);
    if (nt > 0) {  // uniform per wave
        float r0[NT + K - 1], r1[NT + K - 1];
#pragma unroll
        for (int idx = 0; idx < NT + K - 1; ++idx) {
            const int p = tok0 - (K - 1) + idx;
            r0[idx] = r1[idx] = 0.f;
            if (p < a.n_tok) {  // uniform
                const float* row = p >= 0 ? a.x + (size_t)p * a.conv_dim
                                          : a.state + (size_t)(p + K - 1) * a.conv_dim;
                r0[idx] = row[c0];
                r1[idx] = row[c1];
            }
        }
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            if (i >= nt) continue;  // uniform
            // qwen35/cpu.rs:200-204: the current row's term first, then the
            // window rows oldest first
            float acc0 = r0[i + K - 1] * t0[K - 1], acc1 = r1[i + K - 1] * t1[K - 1];
#pragma unroll
            for (int j = 0; j < K - 1; ++j) {
                acc0 += r0[i + j] * t0[j];
                acc1 += r1[i + j] * t1[j];
            }
            float y0 = silu_f(acc0), y1 = silu_f(acc1);
            if (qk) {
                // ops.rs:197-203: x / max(||x||, eps) per head
                if (a.s_dim == 128) {
                    const float sc = 1.f / fmaxf(sqrtf(wave_sum64(y0 * y0 + y1 * y1)), a.eps);
                    y0 *= sc;
                    y1 *= sc;
                } else {  // s_dim 64: lane holds one channel of each of two heads
                    const float s0 = 1.f / fmaxf(sqrtf(wave_sum64(y0 * y0)), a.eps);
                    const float s1 = 1.f / fmaxf(sqrtf(wave_sum64(y1 * y1)), a.eps);
                    y0 *= s0;
                    y1 *= s1;
                }
            }
            float* orow = a.out + (size_t)(tok0 + i) * a.conv_dim;
            orow[c0] = y0;
            orow[c1] = y1;
        }
    }

    // The window after the batch: row r of the new state is position
    // n_tok + r - (K-1) of [state | x].  The first chunk's workgroup is the
    // only reader of the old state for this block; it gathers every new row
    // into registers, waits for its own conv reads, then writes.
    if (tc == 0) {
        float n0[K - 1], n1[K - 1];
        const int per = (K - 1 + 3) / 4;  // rows per wave
#pragma unroll
        for (int k = 0; k < per; ++k) {
            const int r = w + 4 * k;
            if (r < K - 1) {
                const int p = a.n_tok + r - (K - 1);
                const float* row = p >= 0 ? a.x + (size_t)p * a.conv_dim
                                          : a.state + (size_t)(p + K - 1) * a.conv_dim;
                n0[k] = row[c0];
                n1[k] = row[c1];
            }
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < per; ++k) {
            const int r = w + 4 * k;
            if (r < K - 1) {
                a.state[(size_t)r * a.conv_dim + c0] = n0[k];
                a.state[(size_t)r * a.conv_dim + c1] = n1[k];
            }
        }
    }
}

// NJ = s_dim / 64: lane l holds channels l + 64 j of its row.
template <int NJ>
__global__ __launch_bounds__(256) void delta_back_kernel(float* __restrict__ o,
                                                         const float* __restrict__ z,
                                                         const float* __restrict__ wgt, int n_rows,
                                                         float eps) {
    constexpr int SD = 64 * NJ;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n_rows) return;  // wave-uniform
    float* orow = o + (size_t)row * SD;
    const float* zrow = z + (size_t)row * SD;
    float x[NJ];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        x[j] = orow[lane + 64 * j];
        ss += x[j] * x[j];
    }
    // ops.rs:40-47, then the weight (ops.rs:53-59), then silu(z)
    const float sc = 1.f / sqrtf(wave_sum64(ss) / (float)SD + eps);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int d = lane + 64 * j;
        orow[d] = x[j] * sc * wgt[d] * silu_f(zrow[d]);
    }
}

lmx_status deltanet_front(const lmx_delta_front_desc* d, const float* x, const float* taps,
                          float* conv_state, float* conv_out, hipStream_t st) {
    FrontArgs a{};
    a.x = x;
    a.taps = taps;
    a.state = conv_state;
    a.out = conv_out;
    a.n_tok = (int)d->n_tok;
    a.conv_dim = (int)d->conv_dim;
    a.key_dim = (int)d->key_dim;
    a.s_dim = (int)d->s_dim;
    a.kernel = (int)d->kernel;
    a.eps = d->eps;
    const dim3 grid(d->conv_dim / 128, (d->n_tok + kFrontTokens - 1) / kFrontTokens);
    (void)hipGetLastError();
    switch (d->kernel) {
#define LMX_FRONT(KV) \
    case KV: hipLaunchKernelGGL(delta_front_kernel<KV>, grid, dim3(256), 0, st, a); break;
        LMX_FRONT(2) LMX_FRONT(3) LMX_FRONT(4) LMX_FRONT(5) LMX_FRONT(6) LMX_FRONT(7) LMX_FRONT(8)
#undef LMX_FRONT
        default: return LMX_E_UNSUPPORTED;
    }
    LMX_CHECK_LAUNCH();
    return LMX_OK;
}

lmx_status deltanet_back(const lmx_delta_back_desc* d, float* o, const float* z, const float* w,
                         hipStream_t st) {
    const int n_rows = (int)(d->n_tok * d->n_vh);
    const dim3 grid((n_rows + 3) / 4);
    (void)hipGetLastError();
    switch (d->s_dim) {
        case 64: hipLaunchKernelGGL(delta_back_kernel<1>, grid, dim3(256), 0, st, o, z, w, n_rows, d->eps); break;
        case 128: hipLaunchKernelGGL(delta_back_kernel<2>, grid, dim3(256), 0, st, o, z, w, n_rows, d->eps); break;
        case 256: hipLaunchKernelGGL(delta_back_kernel<4>, grid, dim3(256), 0, st, o, z, w, n_rows, d->eps); break;
        default: return LMX_E_UNSUPPORTED;
    }
    LMX_CHECK_LAUNCH();
    return LMX_OK;
}

}  // namespace lmx
