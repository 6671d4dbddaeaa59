// The delta-net's front and back on gfx950: the causal conv + SiLU + conv
// window + q/k L2 norm ahead of the recurrence, and the gated RMS norm after
// it.
//
// Front.  The reference runs four dispatches (conv_silu, conv_shift,
// conv_commit, l2norm_qk; deltanet.wgsl:54-173): the conv output makes a
// round trip through HBM before the norm, and the window update goes through
// a scratch copy so that no thread reads a row another one is overwriting.
// Here one launch does it all.  A wave owns a block of channels for a run of
// consecutive tokens: the K-1 rows before its tokens (from the batch, or
// before it from the window) and its own rows are loaded once into
// registers, the taps slide over them in the reference's order, and the
// head's L2 norm is a wave reduction, so each output row is written once.
// Two forms: with x, the window and the output 16-byte aligned, a lane holds
// four channels (one 16-byte access a row) and a wave takes 256 channels x 8
// tokens; otherwise a lane holds two (lane and lane + 64) and a wave takes
// 128 channels x 16 tokens.  Workgroups are remapped so that each XCD runs a
// contiguous range of tokens across all channels.  Only the first chunk's
// workgroup of a block reads the old window, so it alone writes the new one,
// after its own reads: no workgroup ever reads a window row another one
// writes.
//
// Back.  rms_norm over each v-head then mul_silu (qwen35.rs:968-986), one
// pass: with o, z and the weight 16-byte aligned a lane holds four channels
// and a wave several (token, v-head) rows; otherwise one wave per row.
#include "common.hpp"

namespace lmx {

constexpr int kFrontTokens = 64;  // tokens per front workgroup (>= kernel - 1)

// x / (1 + e^-x) as x * rcp(1 + 2^(-x log2 e)): the hardware exp2 and
// reciprocal (1 ulp each) in place of the libm-accurate expf and the IEEE
// divide.  The rounding of -x log2 e moves e^-x by about |x| 2^-24 relative,
// so while e^-x is finite (x > -88) the result is within about
// (|x| + 2) 2^-24 of the exact SiLU, relative; below that it is 0 where the
// exact value is under 1e-36.
__device__ __forceinline__ float silu_f(float x) { return x * __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

struct FrontArgs {
    const float* x;
    const float* taps;
    float* state;
    float* out;
    int n_tok, conv_dim, key_dim, s_dim, kernel;
    float eps;
};

// Workgroup (block, chunk) of an n_cb x n_tc grid launched 1-D: with the XCD
// remap each XCD runs a contiguous run of token chunks across every channel
// block (whole rows), rather than the same channel columns of every row.
__device__ __forceinline__ void front_tile(int n_cb, int* cb, int* tc) {
    const int n = (int)gridDim.x;
    const int t = xcd_remap((int)blockIdx.x, n);
    *cb = t % n_cb;
    *tc = t / n_cb;
}

template <int K>
__global__ __launch_bounds__(256) void delta_front_kernel(FrontArgs a) {
    int cb, tc;
    front_tile(a.conv_dim / 128, &cb, &tc);
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

// SiLU, then the per-head L2 norm on q/k channels, of one conv row held four
// channels a lane (the head's s_dim / 4 lanes sum its squares; s_dim is 64
// or 128).
__device__ __forceinline__ f32x4 front_finish(f32x4 acc, bool qk, int lane, int s_dim, float eps) {
    f32x4 y;
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = silu_f(acc[e]);
    // ops.rs:197-203: x / max(||x||, eps) per head
    float ss = row_sum16((y[0] * y[0] + y[1] * y[1]) + (y[2] * y[2] + y[3] * y[3]));
    if (s_dim == 128) {  // two DPP rows a head: rows 0 + 1 and 2 + 3
        const int b = __builtin_bit_cast(int, ss);
        const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
        const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
        const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
        const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
        ss = lane < 32 ? r0 + r1 : r2 + r3;
    }
    if (qk) y *= 1.f / fmaxf(sqrtf(ss), eps);
    return y;
}

// The 16-byte form (x, out and the window 16-byte aligned): a lane holds
// four consecutive channels, so a wave covers a 256-channel block and each
// row it touches is one 16-byte load or store a lane.  A workgroup's four
// waves take 8 consecutive tokens each; as in the two-channel form, a wave
// loads the K-1 rows before its first token and its own 8 rows once (the
// rows it shares with its neighbour come from L2), then stores 8 rows.
constexpr int kFront4Wave = 8;
constexpr int kFront4Tokens = 4 * kFront4Wave;
static_assert(kFront4Tokens >= 7, "only the first chunk may touch the old window");

// One wave's rows.  INTERIOR (no window rows, all NT rows inside the batch,
// all 256 channels live) is straight-line code with unconditional loads and
// stores; the checks an edge wave needs cost the interior ones about a tenth
// of the kernel's time when they sit in its one path.
template <int K, bool INTERIOR>
__device__ __forceinline__ void front4_rows(const FrontArgs& a, const f32x4 (&tp)[K], int c, bool live, bool qk,
                                            int lane, int tok0) {
    constexpr int NT = kFront4Wave;
    const int nt = min(NT, a.n_tok - tok0);
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
    f32x4 r[NT + K - 1];
#pragma unroll
    for (int idx = 0; idx < NT + K - 1; ++idx) {
        const int p = tok0 - (K - 1) + idx;  // position p of [window | x]
        if (INTERIOR) {
            r[idx] = *reinterpret_cast<const f32x4*>(a.x + (size_t)p * a.conv_dim + c);
        } else {
            const float* row = p >= 0 ? a.x + (size_t)p * a.conv_dim : a.state + (size_t)(p + K - 1) * a.conv_dim;
            r[idx] = (p < a.n_tok && live) ? *reinterpret_cast<const f32x4*>(row + c) : z4;
        }
    }
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        if (!INTERIOR && i >= nt) continue;  // uniform
        // qwen35/cpu.rs:200-204: the current row's term first, then the
        // window rows oldest first
        f32x4 acc = r[i + K - 1] * tp[K - 1];
#pragma unroll
        for (int j = 0; j < K - 1; ++j) acc += r[i + j] * tp[j];
        const f32x4 y = front_finish(acc, qk, lane, a.s_dim, a.eps);
        if (INTERIOR || live) *reinterpret_cast<f32x4*>(a.out + (size_t)(tok0 + i) * a.conv_dim + c) = y;
    }
}

template <int K>
__global__ __launch_bounds__(256) void delta_front4_kernel(FrontArgs a) {
    int cb, tc;
    front_tile((a.conv_dim + 255) / 256, &cb, &tc);
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = cb * 256 + 4 * lane;  // this lane's channels c .. c + 3
    const bool live = c < a.conv_dim;   // conv_dim % 128 == 0: all four or none
    const bool qk = c < 2 * a.key_dim;  // whole heads on either side (s_dim | key_dim)
    const int cl = live ? c : 0;        // taps of a dead lane: any in-bounds row
    f32x4 tp[K];                        // tp[j][e] = taps[c + e][j]
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int j = 0; j < K; ++j) tp[j][e] = a.taps[(size_t)(cl + e) * K + j];
    const int tok0 = tc * kFront4Tokens + kFront4Wave * w;
    // uniform per wave
    if (tok0 >= K - 1 && tok0 + kFront4Wave <= a.n_tok && cb * 256 + 256 <= a.conv_dim)
        front4_rows<K, true>(a, tp, c, live, qk, lane, tok0);
    else if (tok0 < a.n_tok)
        front4_rows<K, false>(a, tp, c, live, qk, lane, tok0);

    // The window after the batch (as in delta_front_kernel): the first
    // chunk's workgroup is the only reader of the old window for this block.
    if (tc == 0) {
        constexpr int PW = (K - 1 + 3) / 4;
        const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
        f32x4 nw[PW];
#pragma unroll
        for (int k = 0; k < PW; ++k) {
            const int rr = w + 4 * k, p = a.n_tok + rr - (K - 1);
            const float* row = p >= 0 ? a.x + (size_t)p * a.conv_dim : a.state + (size_t)(p + K - 1) * a.conv_dim;
            nw[k] = (rr < K - 1 && live) ? *reinterpret_cast<const f32x4*>(row + c) : z4;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < PW; ++k) {
            const int rr = w + 4 * k;
            if (rr < K - 1 && live) *reinterpret_cast<f32x4*>(a.state + (size_t)rr * a.conv_dim + c) = nw[k];
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

// The 16-byte form of the back (o, z and the weight 16-byte aligned): a lane
// holds four consecutive channels of a row, so a row is SD / 4 lanes and a
// wave covers 64 / (SD / 4) rows at a step; it takes kBack4Steps steps, all
// loaded before the first store.  The sum of squares is a DPP-row sum (SD
// 64), two rows (128) or the whole wave (256).  Workgroups are XCD-remapped
// so each XCD streams a contiguous range of rows; interior waves run without
// the row checks.
constexpr int kBack4Steps = 4;

template <int SD, bool INTERIOR>
__device__ __forceinline__ void back4_rows(float* __restrict__ o, const float* __restrict__ z, f32x4 wv,
                                           int n_rows, float eps, int row0, int lane) {
    constexpr int L = SD / 4, RPS = 64 / L, R = kBack4Steps;
    const int sub = lane / L, c = 4 * (lane % L);
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
    f32x4 x[R], g[R];
#pragma unroll
    for (int s = 0; s < R; ++s) {
        const int row = row0 + s * RPS + sub;
        const bool in = INTERIOR || row < n_rows;
        x[s] = in ? *reinterpret_cast<const f32x4*>(o + (size_t)row * SD + c) : z4;
        g[s] = in ? *reinterpret_cast<const f32x4*>(z + (size_t)row * SD + c) : z4;
    }
#pragma unroll
    for (int s = 0; s < R; ++s) {
        float ss = (x[s][0] * x[s][0] + x[s][1] * x[s][1]) + (x[s][2] * x[s][2] + x[s][3] * x[s][3]);
        if (L == 16) {
            ss = row_sum16(ss);
        } else if (L == 32) {  // two DPP rows a row of o: rows 0 + 1 and 2 + 3
            const int b = __builtin_bit_cast(int, row_sum16(ss));
            const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
            const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
            const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
            const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
            ss = lane < 32 ? r0 + r1 : r2 + r3;
        } else {
            ss = wave_sum64(ss);
        }
        // ops.rs:40-47, then the weight (ops.rs:53-59), then silu(z)
        const float sc = 1.f / sqrtf(ss / (float)SD + eps);
        f32x4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = x[s][e] * sc * wv[e] * silu_f(g[s][e]);
        const int row = row0 + s * RPS + sub;
        if (INTERIOR || row < n_rows) *reinterpret_cast<f32x4*>(o + (size_t)row * SD + c) = y;
    }
}

template <int SD>
__global__ __launch_bounds__(256) void delta_back4_kernel(float* __restrict__ o, const float* __restrict__ z,
                                                          const float* __restrict__ wgt, int n_rows, float eps) {
    constexpr int RPW = 64 / (SD / 4) * kBack4Steps;  // rows a wave
    const int t = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row0 = (t * 4 + w) * RPW;
    if (row0 >= n_rows) return;  // wave-uniform; no barriers here
    const f32x4 wv = *reinterpret_cast<const f32x4*>(wgt + 4 * (lane % (SD / 4)));
    if (row0 + RPW <= n_rows) back4_rows<SD, true>(o, z, wv, n_rows, eps, row0, lane);
    else back4_rows<SD, false>(o, z, wv, n_rows, eps, row0, lane);
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
    // The 16-byte form where every buffer is 16-byte aligned (rows are then
    // 16-byte multiples too: conv_dim % 128 == 0).
    const bool v4 = ((uintptr_t)x | (uintptr_t)conv_state | (uintptr_t)conv_out) % 16 == 0;
    const int n_cb = v4 ? (d->conv_dim + 255) / 256 : d->conv_dim / 128;
    const int tpw = v4 ? kFront4Tokens : kFrontTokens;
    const dim3 grid(n_cb * ((d->n_tok + tpw - 1) / tpw));
    (void)hipGetLastError();
    switch (d->kernel) {
#define LMX_FRONT(KV)                                                                  \
    case KV:                                                                           \
        if (v4) hipLaunchKernelGGL(delta_front4_kernel<KV>, grid, dim3(256), 0, st, a); \
        else hipLaunchKernelGGL(delta_front_kernel<KV>, grid, dim3(256), 0, st, a);     \
        break;
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
    const bool v4 = ((uintptr_t)o | (uintptr_t)z | (uintptr_t)w) % 16 == 0;
    (void)hipGetLastError();
    if (v4) {
        const int rpg = 4 * (64 / (d->s_dim / 4)) * kBack4Steps;  // rows a workgroup
        const dim3 grid((n_rows + rpg - 1) / rpg);
        switch (d->s_dim) {
            case 64: hipLaunchKernelGGL(delta_back4_kernel<64>, grid, dim3(256), 0, st, o, z, w, n_rows, d->eps); break;
            case 128: hipLaunchKernelGGL(delta_back4_kernel<128>, grid, dim3(256), 0, st, o, z, w, n_rows, d->eps); break;
            case 256: hipLaunchKernelGGL(delta_back4_kernel<256>, grid, dim3(256), 0, st, o, z, w, n_rows, d->eps); break;
            default: return LMX_E_UNSUPPORTED;
        }
    } else {
        const dim3 grid((n_rows + 3) / 4);
        switch (d->s_dim) {
            case 64: hipLaunchKernelGGL(delta_back_kernel<1>, grid, dim3(256), 0, st, o, z, w, n_rows, d->eps); break;
            case 128: hipLaunchKernelGGL(delta_back_kernel<2>, grid, dim3(256), 0, st, o, z, w, n_rows, d->eps); break;
            case 256: hipLaunchKernelGGL(delta_back_kernel<4>, grid, dim3(256), 0, st, o, z, w, n_rows, d->eps); break;
            default: return LMX_E_UNSUPPORTED;
        }
    }
    LMX_CHECK_LAUNCH();
    return LMX_OK;
}

}  // namespace lmx
