// Shared device helpers for the gfx950 kernels of libllmoxide_amd.
//
// Wave64 only: every cross-lane helper here assumes 64-lane wavefronts and
// uses DPP row operations (16-lane rows), which is what CDNA4 executes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lmx/attn.h"

namespace lmx {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;

// v_exp_f32: 2^x, exact 0 for -inf.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Sum over the 16 lanes of a DPP row; every lane of the row gets the total.
__device__ __forceinline__ float row_sum16(float x) {
    x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
    x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
    x += dpp<0x141>(x);  // row_half_mirror: pairs the two quads of each half-row
    x += dpp<0x140>(x);  // row_mirror: pairs the two half-rows
    return x;
}

// Sum over the 64 lanes of a wave (all lanes active); every lane gets the
// total.  Four DPP steps per row, then the four row totals through SGPRs:
// no LDS round trip, unlike a ds_bpermute butterfly.
__device__ __forceinline__ float wave_sum64(float x) {
    x = row_sum16(x);
    const int b = __builtin_bit_cast(int, x);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float shfl_xor(float x, int m) { return __shfl_xor(x, m, 64); }

// Kernel arguments used as a point of no return: the compiler must have each
// one in SGPRs here.  Placed at a kernel's entry it makes every argument load
// go out in one round; left alone the compiler sinks loads past early exits
// and branches, and each later round costs a scalar-cache miss (the caches
// start cold in every launch): 0.3 us a round measured on a 5 us decode split.
template <typename T>
__device__ __forceinline__ void arg_in_sgprs(const T& x) {
    asm volatile("" ::"s"(x));
}
template <typename... T>
__device__ __forceinline__ void args_in_sgprs(const T&... x) {
    (arg_in_sgprs(x), ...);
}

// Qwen3.5's attention output gate: o * sigmoid(g), written as the GPU
// reference's mul_sigmoid writes it, o / (1 + exp(-g)) (ops.wgsl:150-163).
__device__ __forceinline__ float gate_sigmoid(float o, float g) { return o / (1.f + expf(-g)); }
__device__ __forceinline__ f32x4 gate_sigmoid4(f32x4 o, const float* g) {
    const f32x4 gv = *reinterpret_cast<const f32x4*>(g);
    return f32x4{gate_sigmoid(o[0], gv[0]), gate_sigmoid(o[1], gv[1]), gate_sigmoid(o[2], gv[2]),
                 gate_sigmoid(o[3], gv[3])};
}

// Kernel-choice overrides for tests and tuning sweeps, from the environment
// (LMX_PREFILL_KERNEL = pp | tile, LMX_PREFILL_GP = 1 | 2 | 4,
// LMX_PREFILL_KH = 0, LMX_DECODE_KROWS = 0 | 1, LMX_DECODE_MH = 0, LMX_DELTA_FUSED = 0 | starve).
// Read once, at the first
// launch, and again only by lmx_tuning_reload(): no getenv on the launch path,
// so a launch and the workspace-size query it was sized by see the same
// values.  -1 (or 0 for gp) means no override.
struct Tuning {
    int prefill_kernel;  // 1: ping-pong, 0: tile kernel
    int prefill_gp;
    int prefill_kh;      // 0: key halves off
    int decode_krows;    // K rows through LDS (1) or direct operand loads (0)
    int decode_mh;       // 0: head_dim 512 keeps attn_decode_kernel even for 16 heads a kv head
    int delta_fused;     // 0: the chunked delta rule runs prep and scan as two launches;
                         // 2 (tests only): one launch with no prep workgroups and a
                         // 64-poll wait bound, so every flag wait gives up
};
Tuning tuning();  // the current overrides (abi.hip)

// Load N consecutive f16 values (N a multiple of 4) as floats.
template <int N>
__device__ __forceinline__ void load_f16_as_f32(const f16* __restrict__ p, float (&out)[N]) {
    static_assert(N % 4 == 0, "vector width");
    if constexpr (N % 8 == 0) {
#pragma unroll
        for (int i = 0; i < N / 8; ++i) {
            f16x8 v = *reinterpret_cast<const f16x8*>(p + 8 * i);
#pragma unroll
            for (int j = 0; j < 8; ++j) out[8 * i + j] = (float)v[j];
        }
    } else {
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {
            f16x4 v = *reinterpret_cast<const f16x4*>(p + 4 * i);
#pragma unroll
            for (int j = 0; j < 4; ++j) out[4 * i + j] = (float)v[j];
        }
    }
}

template <int N>
__device__ __forceinline__ void load_f32(const float* __restrict__ p, float (&out)[N]) {
    static_assert(N % 4 == 0, "vector width");
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
        f32x4 v = *reinterpret_cast<const f32x4*>(p + 4 * i);
#pragma unroll
        for (int j = 0; j < 4; ++j) out[4 * i + j] = v[j];
    }
}

// Raw f16 lanes held in registers (no conversion), N a multiple of 4.
template <int N>
struct RawF16 {
    static_assert(N % 4 == 0, "vector width");
    f16x4 v[N / 4];
};

template <int N>
__device__ __forceinline__ void load_raw(const f16* __restrict__ p, RawF16<N>& r) {
    if constexpr (N % 8 == 0) {
#pragma unroll
        for (int i = 0; i < N / 8; ++i) {
            f16x8 x = *reinterpret_cast<const f16x8*>(p + 8 * i);
            r.v[2 * i] = f16x4{x[0], x[1], x[2], x[3]};
            r.v[2 * i + 1] = f16x4{x[4], x[5], x[6], x[7]};
        }
    } else {
#pragma unroll
        for (int i = 0; i < N / 4; ++i) r.v[i] = *reinterpret_cast<const f16x4*>(p + 4 * i);
    }
}

template <int N>
__device__ __forceinline__ float raw_at(const RawF16<N>& r, int i) {
    return (float)r.v[i / 4][i % 4];
}

// Where an attention call reads q and gates its output (lmx_attn_ext,
// resolved: strides in elements, gate NULL when there is none).
struct AttnIo {
    int q_stride;
    int gate_stride;
    const float* gate;
};

// Multiply-high constants for p % window over 31-bit p (Granlund-Montgomery:
// m = floor(2^(31+l) / w) + 1 with l = ceil(log2 w) makes
// floor(p / w) == (p * m) >> (31 + l) for every 0 <= p < 2^31).
inline void window_magic(uint32_t w, uint32_t* magic, int* shift) {
    if (w == 0) {
        *magic = 0;
        *shift = 0;
        return;
    }
    int l = 0;
    while ((1ull << l) < w) ++l;
    *magic = (uint32_t)((1ull << (31 + l)) / w + 1);
    *shift = 31 + l;
}

// p % w for 0 <= p < 2^31 with the constants above.
__device__ __forceinline__ int ring_slot(int p, int w, uint32_t magic, int shift) {
    const uint32_t q = (uint32_t)(((uint64_t)(uint32_t)p * magic) >> shift);
    return p - (int)q * w;
}

// Bijective workgroup remap so that consecutive logical ids share an XCD
// (workgroups are dispatched round-robin over the 8 XCDs): XCD x runs a
// contiguous range of about n / 8 logical ids.
__device__ __forceinline__ int xcd_remap(int bid, int n) {
    const int q = n / 8, r = n % 8;
    const int xcd = bid % 8, local = bid / 8;
    return xcd < r ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
}

}  // namespace lmx

// Host-side helpers shared by the entry points.
#define LMX_CHECK_LAUNCH()                                  \
    do {                                                    \
        if (hipGetLastError() != hipSuccess) return LMX_E_LAUNCH; \
    } while (0)
