// Quantized matrix-vector products on gfx950: y[t] = W x[t] for a weight
// matrix in ggml's on-disk block formats (the attention epilogue's
// attn_output projection, and any other projection of the same shape).
//
// Replaces the reference's matvec_* dispatches (quant.wgsl:76-551, 553-826;
// recorded by qwen35.rs/forward.rs through `matvec`), computing what
// crates/gguf/src/quant.rs:187-271 (`dot_row`) computes.
//
// Layout.  W is rows x in_dim in the GGUF row-major block layout, unchanged
// (Q6_K's 210-byte and Q8_0's 34-byte blocks are read where they lie; the
// reference repacks Q6_K to 224 bytes at upload, this kernel instead loads
// the dwords that cover a 2-byte aligned field and funnel-shifts them).
//
// Work split (the direct kernel; the staged one is described at
// qmatvec_lds_kernel).  A workgroup of four waves stages x [n_tok, in_dim] in LDS once,
// then its waves take row groups of RW = 4 rows in turn (the grid is capped,
// so a workgroup serves many groups).  Lane l takes 64-weight units l,
// l + 64, ... of the rows (a Q6_K unit is a quarter of a half-block), reads
// the unit's x from LDS once per token for all RW rows, and streams the rows'
// weight bytes from HBM once (no reuse).  Rows end with a DPP wave sum.
// Quants reach float through v_cvt_f32_ubyte on bytewise-assembled dwords;
// Q6_K's -32 and Q8_0's sign go through the unit's x sums, shared by the rows.
#include "common.hpp"

namespace lmx {

enum QType { kF32 = 0, kF16 = 1, kQ8_0 = 8, kQ4K = 12, kQ6K = 14, kBF16 = 30 };

constexpr int kQmvRows = 4;     // rows per wave (direct kernel)
constexpr int kQmvLdsRows = 2;  // rows per wave (staged kernel: fewer registers, more waves)
constexpr int kQmvWaves = 4;    // waves per workgroup
constexpr int kQmvMaxTok = 4;   // tokens per launch
constexpr int kQmvLdsFloats = 16384;  // x staged in LDS: n_tok * in_dim <= this
constexpr long kQmvMaxWgs = 2048;     // workgroups of a launch (eight per CU)


struct QmvArgs {
    const uint8_t* w;
    const float* x;
    float* y;
    int rows, in_dim, n_tok;
    size_t row_bytes;
};

template <int TY>
struct QTraits;
template <> struct QTraits<kQ4K> { static constexpr int unit = 64, bbytes = 144, belems = 256; };
template <> struct QTraits<kQ6K> { static constexpr int unit = 64, bbytes = 210, belems = 256; };
template <> struct QTraits<kQ8_0> { static constexpr int unit = 64, bbytes = 34, belems = 32; };
template <> struct QTraits<kF32> { static constexpr int unit = 64, bbytes = 4, belems = 1; };
template <> struct QTraits<kF16> { static constexpr int unit = 64, bbytes = 2, belems = 1; };
template <> struct QTraits<kBF16> { static constexpr int unit = 64, bbytes = 2, belems = 1; };

// Weight bytes are streamed: read once, never reused.  LDS: the bytes were
// staged in a wave's LDS slice first (qmatvec_lds_kernel).
template <bool LDS>
__device__ __forceinline__ uint32_t ld_u32(const uint8_t* p) {
    if constexpr (LDS) return *reinterpret_cast<const uint32_t*>(p);
    else return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}
template <bool LDS>
__device__ __forceinline__ uint16_t ld_u16(const uint8_t* p) {
    if constexpr (LDS) return *reinterpret_cast<const uint16_t*>(p);
    else return __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(p));
}

// N dwords of the byte range [p, p + 4N) at a 2-byte aligned p: the aligned
// dwords that cover it, funnel-shifted by 0 or 2 bytes.  An aligned range
// reads exactly its own bytes; a shifted one also reads the 2 bytes before
// and after it, which for every field below lie inside the same block or the
// block before (a shifted block is never the first of the matrix).
template <int N, bool LDS>
__device__ __forceinline__ void ld_words_a2(const uint8_t* p, uint32_t (&out)[N]) {
    // base by pointer arithmetic, not an integer round trip, so the loads
    // stay global ones (a flat load also counts against the LDS wait counter,
    // and every read of the staged x would wait for the weight stream)
    const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3);  // 0 or 2
    const uint8_t* base = p - sh;
    uint32_t raw[N + 1];
#pragma unroll
    for (int i = 0; i < N; ++i) raw[i] = ld_u32<LDS>(base + 4 * i);
    raw[N] = 0u;
    if (sh) raw[N] = ld_u32<LDS>(base + 4 * N);
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], sh);
}

__device__ __forceinline__ float f16_lo(uint32_t w) { return (float)__builtin_bit_cast(f16, (uint16_t)(w & 0xFFFF)); }
__device__ __forceinline__ float f16_hi(uint32_t w) { return (float)__builtin_bit_cast(f16, (uint16_t)(w >> 16)); }
__device__ __forceinline__ float byte_f(uint32_t w, int i) { return (float)((w >> (8 * i)) & 0xFF); }
__device__ __forceinline__ float sbyte_f(uint32_t w, int i) { return (float)(int8_t)((w >> (8 * i)) & 0xFF); }

// quant.rs:33-47: 6-bit scale and min of sub-block j from the 12 packed
// bytes held as three dwords.
__device__ __forceinline__ void q4k_scale_min(const uint32_t (&s)[3], int j, float& sc, float& m) {
    // With jl = j % 4, byte j (j < 4) or j + 4 ... lie at byte jl of the
    // three dwords: B0 = bytes 0-3, B1 = 4-7, B2 = 8-11.  Selects, not a
    // branch, so that callers' loads are not split by a divergent branch.
    const int sh = 8 * (j & 3);
    const uint32_t b0 = (s[0] >> sh) & 0xFF, b1 = (s[1] >> sh) & 0xFF, b2 = (s[2] >> sh) & 0xFF;
    const bool lo = j < 4;
    sc = (float)(lo ? b0 & 63 : (b2 & 0xF) | ((b0 >> 6) << 4));
    m = (float)(lo ? b1 & 63 : (b2 >> 4) | ((b1 >> 6) << 4));
}

// The dot products of one unit of the RW rows with the T staged tokens,
// added into acc[r][t].  `row[r]` points at row r's bytes (for a row past the
// end, the wave's first row again: its result is never stored); uw is the
// unit's index from row[r], ux its index in x (they differ when row[r] is a
// staged chunk of the row).
template <int TY, int T, bool LDS, int RW>
__device__ __forceinline__ void unit_dot(const uint8_t* const (&row)[RW], int uw, int ux,
                                         const float* xs, int in_dim, float (&acc)[RW][T]) {
    if constexpr (TY == kQ4K) {
        // unit u = pair p of block b: sub-blocks 2p (low nibbles of 32 bytes)
        // and 2p + 1 (high nibbles); x chunk [256b + 64p, +64).  The x chunk
        // is walked in steps of four elements (per token), each step applied
        // to all rows, so only a step of x is live at a time.
        const int b = uw >> 2, p = uw & 3;
        const float* xc = xs + 64 * ux;
        uint32_t q[RW][8], hdr[RW][4];
        float a1[RW], c1[RW], a2[RW], c2[RW];
        // every row's bytes requested before any is used
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            const uint8_t* blk = row[r] + (size_t)b * 144;
            if constexpr (!LDS) {
                // three 16-byte loads (blocks are 9 x 16 bytes; W is 16-byte aligned)
                typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
                const u32x4 h4 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(blk));
                const u32x4 qa = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(blk + 16 + 32 * p));
                const u32x4 qb = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(blk + 32 + 32 * p));
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    hdr[r][i] = h4[i];
                    q[r][i] = qa[i];
                    q[r][4 + i] = qb[i];
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) hdr[r][i] = ld_u32<LDS>(blk + 4 * i);
#pragma unroll
                for (int i = 0; i < 8; ++i) q[r][i] = ld_u32<LDS>(blk + 16 + 32 * p + 4 * i);
            }
        }
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            const float d = f16_lo(hdr[r][0]), dmin = f16_hi(hdr[r][0]);
            const uint32_t sc3[3] = {hdr[r][1], hdr[r][2], hdr[r][3]};
            float sc1, m1, sc2, m2;
            q4k_scale_min(sc3, 2 * p, sc1, m1);
            q4k_scale_min(sc3, 2 * p + 1, sc2, m2);
            a1[r] = d * sc1;
            c1[r] = dmin * m1;
            a2[r] = d * sc2;
            c2[r] = dmin * m2;
        }
        float S1[RW][T], S2[RW][T], X1[T], X2[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
            X1[t] = X2[t] = 0.f;
#pragma unroll
            for (int r = 0; r < RW; ++r) S1[r][t] = S2[r][t] = 0.f;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const f32x4 xa = *reinterpret_cast<const f32x4*>(xc + t * in_dim + 4 * i);
                const f32x4 xb = *reinterpret_cast<const f32x4*>(xc + t * in_dim + 32 + 4 * i);
                X1[t] += (xa[0] + xa[1]) + (xa[2] + xa[3]);
                X2[t] += (xb[0] + xb[1]) + (xb[2] + xb[3]);
#pragma unroll
                for (int r = 0; r < RW; ++r) {
                    const uint32_t lo = q[r][i] & 0x0F0F0F0Fu, hi = (q[r][i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        S1[r][t] = fmaf(byte_f(lo, j), xa[j], S1[r][t]);
                        S2[r][t] = fmaf(byte_f(hi, j), xb[j], S2[r][t]);
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int t = 0; t < T; ++t)
                acc[r][t] += a1[r] * S1[r][t] - c1[r] * X1[t] + a2[r] * S2[r][t] - c2[r] * X2[t];
    } else if constexpr (TY == kQ6K) {
        // unit u = quarter k of half h of block b (u = 4b + 2h + k): the 64
        // elements 32g + l of the half with l in [16k, 16k + 16), g < 4.
        // Element 32g + l takes the quant of quant.rs:99-106 from ql[l] (g 0,
        // 2) or ql[l + 32] (g 1, 3) and qh[l], and scale 2g + k (l / 16 = k).
        const int b = uw >> 2, h = (uw >> 1) & 1, k = uw & 1;
        const float* xc = xs + 64 * (ux & ~3) + 128 * h + 16 * k;
        uint32_t qa[RW][4], qb[RW][4], qh[RW][4];
        float sc[RW][4], dd[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            const uint8_t* blk = row[r] + (size_t)b * 210;
            uint32_t scw[2];
            ld_words_a2<4, LDS>(blk + 64 * h + 16 * k, qa[r]);
            ld_words_a2<4, LDS>(blk + 64 * h + 32 + 16 * k, qb[r]);
            ld_words_a2<4, LDS>(blk + 128 + 32 * h + 16 * k, qh[r]);
            ld_words_a2<2, LDS>(blk + 192 + 8 * h, scw);  // this half's 8 i8 scales
            dd[r] = (float)__builtin_bit_cast(f16, ld_u16<LDS>(blk + 208));
#pragma unroll
            for (int g = 0; g < 4; ++g) sc[r][g] = sbyte_f(scw[(2 * g + k) >> 2], (2 * g + k) & 3);
        }
        // Four 6-bit quants per dword, assembled bytewise with masks:
        // group g's low nibbles from ql (g < 2 low halves, g >= 2 high), its
        // two high bits from bits 2g..2g+1 of each qh byte.  The quants go to
        // float unbiased (v_cvt_f32_ubyte) and the -32 is applied once per
        // group through the group's sum of x, which every row shares.
        float G[RW][T][4], XS[T][4];
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                XS[t][g] = 0.f;
#pragma unroll
                for (int r = 0; r < RW; ++r) G[r][t][g] = 0.f;
            }
#pragma unroll
        for (int l4 = 0; l4 < 4; ++l4) {  // l = 16k + 4*l4 .. +3
#pragma unroll
            for (int t = 0; t < T; ++t) {
                f32x4 xv[4];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    xv[g] = *reinterpret_cast<const f32x4*>(xc + t * in_dim + 32 * g + 4 * l4);
                    XS[t][g] += (xv[g][0] + xv[g][1]) + (xv[g][2] + xv[g][3]);
                }
#pragma unroll
                for (int r = 0; r < RW; ++r) {
                    const uint32_t wa = qa[r][l4], wb = qb[r][l4], hh = qh[r][l4];
                    const uint32_t qw[4] = {
                        (wa & 0x0F0F0F0Fu) | ((hh << 4) & 0x30303030u),
                        (wb & 0x0F0F0F0Fu) | ((hh << 2) & 0x30303030u),
                        ((wa >> 4) & 0x0F0F0F0Fu) | (hh & 0x30303030u),
                        ((wb >> 4) & 0x0F0F0F0Fu) | ((hh >> 2) & 0x30303030u)};
#pragma unroll
                    for (int g = 0; g < 4; ++g)
#pragma unroll
                        for (int j = 0; j < 4; ++j) G[r][t][g] = fmaf(byte_f(qw[g], j), xv[g][j], G[r][t][g]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int t = 0; t < T; ++t) {
                float sub = 0.f;
#pragma unroll
                for (int g = 0; g < 4; ++g) sub += sc[r][g] * (G[r][t][g] - 32.f * XS[t][g]);
                acc[r][t] = fmaf(dd[r], sub, acc[r][t]);
            }
    } else if constexpr (TY == kQ8_0) {
        // unit u = blocks 2u, 2u + 1: 68 bytes at 68u (4-byte aligned)
        const float* xc = xs + 64 * ux;
        float X0[T], X1[T];  // the x sums of the two blocks, shared by all rows
#pragma unroll
        for (int t = 0; t < T; ++t) {
            float s0 = 0.f, s1 = 0.f;
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                const f32x4 a = *reinterpret_cast<const f32x4*>(xc + t * in_dim + i);
                const f32x4 c = *reinterpret_cast<const f32x4*>(xc + t * in_dim + 32 + i);
                s0 += (a[0] + a[1]) + (a[2] + a[3]);
                s1 += (c[0] + c[1]) + (c[2] + c[3]);
            }
            X0[t] = s0;
            X1[t] = s1;
        }
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            const uint8_t* p = row[r] + (size_t)68 * uw;
            uint32_t wds[17];
#pragma unroll
            for (int i = 0; i < 17; ++i) wds[i] = ld_u32<LDS>(p + 4 * i);
            const float d0 = f16_lo(wds[0]), d1 = f16_hi(wds[8]);
            // block 0 quants: bytes 2..33 -> words 0..8 shifted by 2;
            // block 1 quants: bytes 36..67 -> words 9..16
            // q + 128 as an unsigned byte (sign bit flipped), converted with
            // v_cvt_f32_ubyte; the +128 leaves through the chunk's x sum.
            uint32_t q0[8], q1[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                q0[i] = __builtin_amdgcn_alignbyte(wds[i + 1], wds[i], 2) ^ 0x80808080u;
                q1[i] = wds[9 + i] ^ 0x80808080u;
            }
#pragma unroll
            for (int t = 0; t < T; ++t) {
                float s0 = 0.f, s1 = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const f32x4 a = *reinterpret_cast<const f32x4*>(xc + t * in_dim + 4 * i);
                    const f32x4 c = *reinterpret_cast<const f32x4*>(xc + t * in_dim + 32 + 4 * i);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        s0 = fmaf(byte_f(q0[i], j), a[j], s0);
                        s1 = fmaf(byte_f(q1[i], j), c[j], s1);
                    }
                }
                acc[r][t] += d0 * (s0 - 128.f * X0[t]) + d1 * (s1 - 128.f * X1[t]);
            }
        }
    } else {
        // dense rows: 64 consecutive weights
        const int u = uw;
        const float* xc = xs + 64 * ux;
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            float wv[64];
            if constexpr (TY == kF32) {
                const float* p = reinterpret_cast<const float*>(row[r]) + 64 * u;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + 4 * i));
#pragma unroll
                    for (int j = 0; j < 4; ++j) wv[4 * i + j] = v[j];
                }
            } else {
                const uint16_t* p = reinterpret_cast<const uint16_t*>(row[r]) + 64 * u;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
                    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p + 8 * i));
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if constexpr (TY == kF16) {
                            wv[8 * i + 2 * j] = f16_lo(v[j]);
                            wv[8 * i + 2 * j + 1] = f16_hi(v[j]);
                        } else {  // bf16: the top half of an f32
                            wv[8 * i + 2 * j] = __builtin_bit_cast(float, v[j] << 16);
                            wv[8 * i + 2 * j + 1] = __builtin_bit_cast(float, v[j] & 0xFFFF0000u);
                        }
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < T; ++t) {
                float s = 0.f;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const f32x4 a = *reinterpret_cast<const f32x4*>(xc + t * in_dim + 4 * i);
#pragma unroll
                    for (int j = 0; j < 4; ++j) s = fmaf(wv[4 * i + j], a[j], s);
                }
                acc[r][t] += s;
            }
        }
    }
}

// x [n_tok, in_dim] into LDS, 16 bytes a thread a step, with four steps'
// loads in flight before the first store: a load-then-store loop waits out a
// full memory round trip per step (four at in_dim 4096).
__device__ __forceinline__ void stage_x(float* xs, const float* x, int nx4, int tid) {
    constexpr int U = 4, NT = kQmvWaves * 64;
    const f32x4* src = reinterpret_cast<const f32x4*>(x);
    f32x4* dst = reinterpret_cast<f32x4*>(xs);
    int i = tid;
    for (; i + (U - 1) * NT < nx4; i += U * NT) {  // all U steps in range: no branch between loads
        f32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = src[i + u * NT];
#pragma unroll
        for (int u = 0; u < U; ++u) dst[i + u * NT] = v[u];
    }
    for (; i < nx4; i += NT) dst[i] = src[i];
}

template <int TY, int T>
__global__ __launch_bounds__(kQmvWaves * 64) void qmatvec_kernel(QmvArgs a) {
    extern __shared__ __attribute__((aligned(16))) float xs[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    stage_x(xs, a.x, a.n_tok * a.in_dim / 4, tid);
    __syncthreads();

    // Row groups of kQmvRows rows, dealt to the waves of all workgroups in
    // turn; x is staged once per workgroup for all of its groups.
    const int n_groups = (a.rows + kQmvRows - 1) / kQmvRows;
    const int n_units = a.in_dim / QTraits<TY>::unit;
    for (int g = blockIdx.x * kQmvWaves + wave; g < n_groups; g += gridDim.x * kQmvWaves) {
        const int r0 = g * kQmvRows;
        const uint8_t* row[kQmvRows];
#pragma unroll
        for (int r = 0; r < kQmvRows; ++r) {
            const int rr = r0 + r < a.rows ? r0 + r : r0;  // past the end: re-read a valid row
            row[r] = a.w + (size_t)rr * a.row_bytes;
        }
        float acc[kQmvRows][T];
#pragma unroll
        for (int r = 0; r < kQmvRows; ++r)
#pragma unroll
            for (int t = 0; t < T; ++t) acc[r][t] = 0.f;
        for (int u = lane; u < n_units; u += 64) unit_dot<TY, T, false, kQmvRows>(row, u, u, xs, a.in_dim, acc);
#pragma unroll
        for (int r = 0; r < kQmvRows; ++r) {
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const float s = wave_sum64(acc[r][t]);
                if (lane == 0 && r0 + r < a.rows) a.y[(size_t)t * a.rows + r0 + r] = s;
            }
        }
    }
}

// ---- Staged variant for the block formats ----------------------------------
//
// The per-unit reads above give each lane 2-16 bytes at a stride of a block:
// one load instruction touches 30-50 cache lines and every line is touched
// again by the next field's load, which keeps the texture addresser busy and
// holds the stream well below HBM rate.  Here a wave takes groups of two rows
// (fewer registers than the direct kernel's four, so more waves stream at
// once: Q6_K 4096 x 12288 20.0 -> 16.7 us) and copies a chunk of 64
// units of each row (16 K-quant blocks, or 128 Q8_0 blocks) into
// its own LDS slice with contiguous 16-byte LDS-DMA loads (the 16-aligned
// window around the chunk, 1 KB per instruction), then runs the same unit_dot
// from LDS.  The slice is private to the wave, so a wait for its own loads
// (vmcnt) is the only synchronisation.  The row group holding the matrix's
// last row takes the direct path, so no window reaches past the matrix.
// Q6_K and Q8_0 take this kernel (lm_head 151936 x 4096 Q6_K: 2.36 -> 4.0
// TB/s).  Q4_K stays direct: a lane's 32 quant bytes already lie next to its
// neighbours', and staging measured slower there.
template <int TY>
struct QChunk;
// units per byte group, bytes per group, DMA instructions per row and chunk
template <> struct QChunk<kQ4K> { static constexpr int upg = 4, gbytes = 144, ni = 3; };
template <> struct QChunk<kQ6K> { static constexpr int upg = 4, gbytes = 210, ni = 4; };
template <> struct QChunk<kQ8_0> { static constexpr int upg = 1, gbytes = 68, ni = 5; };
template <int TY>
constexpr size_t qmv_slice_bytes() { return (size_t)kQmvLdsRows * QChunk<TY>::ni * 1024; }

template <int TY, int T>
__global__ __launch_bounds__(kQmvWaves * 64) void qmatvec_lds_kernel(QmvArgs a) {
    extern __shared__ __attribute__((aligned(16))) float xs[];
    constexpr int NI = QChunk<TY>::ni, UPG = QChunk<TY>::upg, GB = QChunk<TY>::gbytes;
    constexpr int CB = 64 / UPG * GB;  // bytes of a full 64-unit chunk of a row
    static_assert((64 / UPG * GB + 15) / 16 + 1 <= NI * 64, "DMA instructions cover a chunk's window");
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    stage_x(xs, a.x, a.n_tok * a.in_dim / 4, tid);
    __syncthreads();
    uint8_t* slice = reinterpret_cast<uint8_t*>(xs + a.n_tok * a.in_dim) + wave * qmv_slice_bytes<TY>();

    const int n_groups = (a.rows + kQmvLdsRows - 1) / kQmvLdsRows;
    const int n_units = a.in_dim / QTraits<TY>::unit;
    const int n_chunks = (n_units + 63) / 64;
    for (int g = blockIdx.x * kQmvWaves + wave; g < n_groups; g += gridDim.x * kQmvWaves) {
        const int r0 = g * kQmvLdsRows;
        float acc[kQmvLdsRows][T];
#pragma unroll
        for (int r = 0; r < kQmvLdsRows; ++r)
#pragma unroll
            for (int t = 0; t < T; ++t) acc[r][t] = 0.f;
        if (r0 + kQmvLdsRows >= a.rows) {
            // the group with the matrix's last row: direct reads, exact bytes
            const uint8_t* row[kQmvLdsRows];
#pragma unroll
            for (int r = 0; r < kQmvLdsRows; ++r) {
                const int rr = r0 + r < a.rows ? r0 + r : r0;
                row[r] = a.w + (size_t)rr * a.row_bytes;
            }
            for (int u = lane; u < n_units; u += 64) unit_dot<TY, T, false, kQmvLdsRows>(row, u, u, xs, a.in_dim, acc);
        } else {
            for (int c = 0; c < n_chunks; ++c) {
                const int cu = min(64, n_units - 64 * c);  // units in this chunk
                const size_t len = (size_t)(cu / UPG) * GB;
                const uint8_t* lrow[kQmvLdsRows];
#pragma unroll
                for (int r = 0; r < kQmvLdsRows; ++r) {
                    const size_t s0 = (size_t)(r0 + r) * a.row_bytes + (size_t)c * CB;
                    const size_t w0 = s0 & ~(size_t)15;
                    const int n16 = (int)((s0 + len - w0 + 15) / 16);
                    uint8_t* dst = slice + r * (NI * 1024);
#pragma unroll
                    for (int j = 0; j < NI; ++j) {
                        const int i = min(64 * j + lane, n16 - 1);  // every lane loads: a fixed count
                        __builtin_amdgcn_global_load_lds(
                            (const __attribute__((address_space(1))) void*)(a.w + w0 + 16 * (size_t)i),
                            (__attribute__((address_space(3))) void*)(dst + 1024 * j), 16, 0, 0);
                    }
                    lrow[r] = dst + (s0 - w0);
                }
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the slice holds the chunk
                if (lane < cu) unit_dot<TY, T, true, kQmvLdsRows>(lrow, lane, 64 * c + lane, xs, a.in_dim, acc);
            }
        }
#pragma unroll
        for (int r = 0; r < kQmvLdsRows; ++r) {
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const float sum = wave_sum64(acc[r][t]);
                if (lane == 0 && r0 + r < a.rows) a.y[(size_t)t * a.rows + r0 + r] = sum;
            }
        }
    }
}

template <int TY>
static lmx_status launch_lds(const QmvArgs& a, int T, hipStream_t st) {
    const long groups = (a.rows + kQmvLdsRows - 1) / kQmvLdsRows;
    const long wgs = std::min<long>((groups + kQmvWaves - 1) / kQmvWaves, kQmvMaxWgs);
    const dim3 grid((unsigned)wgs);
    const size_t lds = (size_t)T * a.in_dim * sizeof(float) + kQmvWaves * qmv_slice_bytes<TY>();
    switch (T) {
#define LMX_QMV(TT)                                                                                 \
    case TT: {                                                                                      \
        static const bool attr = hipFuncSetAttribute((const void*)qmatvec_lds_kernel<TY, TT>,       \
                                                     hipFuncAttributeMaxDynamicSharedMemorySize,   \
                                                     160 * 1024) == hipSuccess;                      \
        if (!attr) return LMX_E_LAUNCH;                                                             \
        hipLaunchKernelGGL((qmatvec_lds_kernel<TY, TT>), grid, dim3(kQmvWaves * 64), lds, st, a);    \
        break;                                                                                      \
    }
        LMX_QMV(1) LMX_QMV(2) LMX_QMV(3) LMX_QMV(4)
#undef LMX_QMV
        default: return LMX_E_UNSUPPORTED;
    }
    return LMX_OK;
}

template <int TY>
static lmx_status launch_type(const QmvArgs& a, int T, hipStream_t st) {
    // Enough workgroups for every CU to hold several; each loops over row groups.
    const long groups = (a.rows + kQmvRows - 1) / kQmvRows;
    const long wgs = std::min<long>((groups + kQmvWaves - 1) / kQmvWaves, kQmvMaxWgs);
    const dim3 grid((unsigned)wgs);
    const size_t lds = (size_t)T * a.in_dim * sizeof(float);
    switch (T) {
#define LMX_QMV(TT) \
    case TT: hipLaunchKernelGGL((qmatvec_kernel<TY, TT>), grid, dim3(kQmvWaves * 64), lds, st, a); break;
        LMX_QMV(1) LMX_QMV(2) LMX_QMV(3) LMX_QMV(4)
#undef LMX_QMV
        default: return LMX_E_UNSUPPORTED;
    }
    return LMX_OK;
}

// qgemm.hip: the matrix-core GEMM for batches of tokens
lmx_status qgemm(const lmx_qmv_desc* d, const void* w, const float* x, float* y, hipStream_t st);

// From this many tokens the GEMM takes the k-quant formats (the reference's
// GEMM_MIN_TOKENS, crates/gpu/src/lib.rs:1083): one launch reads W once.
constexpr uint32_t kGemmMinTokens = 16;

// Host side: tokens go in tiles of up to kQmvMaxTok (each tile re-reads W),
// or to the GEMM.
lmx_status qmatvec(const lmx_qmv_desc* d, const void* w, const float* x, float* y, hipStream_t st) {
    if (d->n_tok >= kGemmMinTokens && d->in_dim % 128 == 0 &&
        (d->type == kQ4K || d->type == kQ6K || d->type == kQ8_0))
        return qgemm(d, w, x, y, st);
    int unit = 0;
    size_t bb = 0, be = 0;
    switch (d->type) {
        case kQ4K: unit = 64; bb = 144; be = 256; break;
        case kQ6K: unit = 64; bb = 210; be = 256; break;
        case kQ8_0: unit = 64; bb = 34; be = 32; break;
        case kF32: unit = 64; bb = 4; be = 1; break;
        case kF16: case kBF16: unit = 64; bb = 2; be = 1; break;
        default: return LMX_E_UNSUPPORTED;
    }
    if (d->in_dim % unit || d->in_dim % be) return LMX_E_SHAPE;
    const size_t row_bytes = d->in_dim / be * bb;
    int per = kQmvMaxTok;
    while (per > 1 && (size_t)per * d->in_dim > (size_t)kQmvLdsFloats) --per;
    if ((size_t)d->in_dim > (size_t)kQmvLdsFloats) return LMX_E_UNSUPPORTED;
    (void)hipGetLastError();
    for (uint32_t t0 = 0; t0 < d->n_tok; t0 += per) {
        const int T = (int)std::min<uint32_t>(per, d->n_tok - t0);
        QmvArgs a{};
        a.w = static_cast<const uint8_t*>(w);
        a.x = x + (size_t)t0 * d->in_dim;
        a.y = y + (size_t)t0 * d->rows;
        a.rows = (int)d->rows;
        a.in_dim = (int)d->in_dim;
        a.n_tok = T;
        a.row_bytes = row_bytes;
        lmx_status s;
        switch (d->type) {
            case kQ4K: s = launch_type<kQ4K>(a, T, st); break;  // its loads are contiguous already
            case kQ6K: s = launch_lds<kQ6K>(a, T, st); break;
            case kQ8_0: s = launch_lds<kQ8_0>(a, T, st); break;
            case kF32: s = launch_type<kF32>(a, T, st); break;
            case kF16: s = launch_type<kF16>(a, T, st); break;
            default: s = launch_type<kBF16>(a, T, st); break;
        }
        if (s != LMX_OK) return s;
        LMX_CHECK_LAUNCH();
    }
    return LMX_OK;
}

}  // namespace lmx
