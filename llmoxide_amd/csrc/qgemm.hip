// Quantized GEMM on gfx950 matrix cores: Y[t][r] = sum_k W[r][k] X[t][k] for
// a batch of tokens (prefill) and a weight matrix in ggml's on-disk block
// formats Q4_K, Q6_K or Q8_0, read once per launch.
//
// Replaces the reference's prefill GEMM (gemm_q6k in gemm.wgsl:93-95 and
// gemm_q6k.metal:50, chosen from 16 tokens: crates/gpu/src/lib.rs:1039-1046,
// 1083) and computes what its CPU reference dot_row computes
// (crates/gguf/src/quant.rs:187-271), to fp32 accuracy:
//
//   Every block format is  w = s_g * q + o_g  over groups g of 16 or 32
//   consecutive weights, q a small integer:
//     Q4_K  q in [0, 15],     s = d * sc_g, o = -dmin * m_g  (groups of 32)
//     Q6_K  q in [-32, 31],   s = d * sc_g, o = 0            (groups of 16)
//     Q8_0  q in [-128, 127], s = d,        o = 0            (groups of 32)
//   so   y = sum_g  s_g * (sum_{k in g} q_k x_k)  +  o_g * (sum_{k in g} x_k),
//   the order dot_row itself uses for Q4_K (its s1 and x1 per sub-block).
//   The integers q are exact in f16; x is split into f16 x_hi + x_lo
//   (|x - x_hi - x_lo| <= 2^-22 |x|), so each group's integer sum is two
//   v_mfma_f32_32x32x16_f16 products accumulated in fp32, and the group's
//   scale and offset are applied in fp32 (the x sums come from the fp32 x).
//
//   Range: before the split, each token's x is multiplied by a power of two
//   2^k_t (exact).  k_t is the running minimum over the chunks of a bound
//   k_c: 0 while the token's largest |x| in the chunk lies in [2^-6, 2^14),
//   else the k that brings it into [2^14, 2^15).  So no scaled value comes
//   near f16's 65504, and a token whose x are all tiny is scaled up instead
//   of falling into f16 subnormals.  Every partial sum of a token is in one
//   scaled domain: when a chunk changes k_t, the token's accumulated y is
//   first multiplied by the (exact) ratio, and the store multiplies by
//   2^-k_t.  Elements far below their chunk's maximum keep an absolute error
//   of about 2^-22 of the largest value met, as fp32 summation would.  In
//   the common case (k_t = 0 from the first chunk on) the scaling is skipped.
//
// Tiles.  A workgroup owns 64 tokens x 128 weight rows.  Its four consumer
// waves multiply: wave (wm, wn) owns tokens 32 wm .. + 31 and rows
// 64 wn .. + 63, two 32 x 32 MFMA tiles with x as the A operand and q as B,
// so each lane of a result tile holds one weight row and 16 tokens, and a
// group's scale is one value per lane.  K goes through LDS 128 weights at a
// time (half a K-quant super-block, four Q8_0 blocks): x as swizzled f16 hi /
// lo rows, W decoded to f16 integers with each row's group scales, and the
// (token, group) x sums.  Its producer waves, four or eight for W (load and
// decode) and four for x (load, hi / lo split and group sums), stash the next chunk
// into the other of two LDS buffers meanwhile, with the chunk after that
// already in registers.
#include "common.hpp"

namespace lmx {

enum GType { kGQ8_0 = 8, kGQ4K = 12, kGQ6K = 14 };

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#ifndef LMX_QGEMM_ROWS
#define LMX_QGEMM_ROWS 128
#endif
constexpr int kGM = 64;        // tokens per workgroup
constexpr int kGN = LMX_QGEMM_ROWS;  // weight rows per workgroup (64 or 128)
#ifndef LMX_QGEMM_CONS
#define LMX_QGEMM_CONS 4
#endif
constexpr int kGCons = LMX_QGEMM_CONS;         // consumer (MFMA) waves: 4 or 8
constexpr int kNTW = kGN / (16 * kGCons);      // 32-row MFMA tiles per consumer wave
constexpr int kGK = 128;       // weights per LDS chunk
constexpr int kGXF = 2048;                       // float4s of x in a chunk (64 tokens x 128)
constexpr int kGConsT = 64 * kGCons;             // consumer threads
// W-producer threads per row: 4 for Q6_K (one 32-weight unit each: its
// decode is the heaviest), 2 for Q4_K and Q8_0 (two units each; 4 measured
// 2% slower for them).
template <int TY>
constexpr int g_wparts() { return TY == kGQ6K ? 4 : 2; }
// x-producer threads: 512 (four float4s of a chunk each) for Q4_K, whose x
// producers also form the group sums (73 -> 63.5 us against 256), 256 (eight
// each) for Q8_0 (512 measured 5% slower) and Q6_K (eight W waves).
template <int TY>
constexpr int g_xthreads() { return TY == kGQ4K ? 512 : 256; }
template <int TY>
constexpr int g_threads() { return kGConsT + kGN * g_wparts<TY>() + g_xthreads<TY>(); }  // consumers, W, x producers

template <int TY>
struct GTraits;
template <> struct GTraits<kGQ4K> { static constexpr int gs = 32, words = 12; };
template <> struct GTraits<kGQ6K> { static constexpr int gs = 16, words = 9; };
template <> struct GTraits<kGQ8_0> { static constexpr int gs = 32, words = 9; };

struct GemmArgs {
    const uint8_t* w;
    const float* x;
    float* y;
    int rows, in_dim, n_tok;
    size_t row_bytes;
};

// Largest x over each group of 32 lanes (x >= 0): DPP within each 16-lane
// row, then one swizzle between the two rows of a group (no LDS traffic,
// unlike ds_bpermute).
__device__ __forceinline__ float max32(float x) {
    x = fmaxf(x, dpp<0xB1>(x));   // quad_perm [1,0,3,2]
    x = fmaxf(x, dpp<0x4E>(x));   // quad_perm [2,3,0,1]
    x = fmaxf(x, dpp<0x141>(x));  // row_half_mirror
    x = fmaxf(x, dpp<0x140>(x));  // row_mirror
    // swizzle, bitmask mode: lane ^ 16 within 32
    return fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), 0x401F)));
}
// Sum over each aligned group of 8 lanes; every lane of the group gets it.
__device__ __forceinline__ float sum8(float x) {
    x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
    x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
    return x + dpp<0x141>(x);  // row_half_mirror: lane i with 7 - i of its 8
}

// Swizzled offset (in halfs) of 8-half chunk c of LDS row r: the chunk index
// is XORed with the row, so the rows an MFMA operand read touches spread
// over the banks.
__device__ __forceinline__ int sw(int r, int c) { return r * kGK + ((c ^ (r & 15)) << 3); }

// Eight bytes at a 2-byte aligned address as two dwords: the covering
// aligned dwords, funnel-shifted.  A shifted read also touches the 2 bytes
// after the range; every range below ends at least 2 bytes before its block.
__device__ __forceinline__ void ld8_a2(const uint8_t* p, uint32_t* o) {
    const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3);
    const uint32_t* b = reinterpret_cast<const uint32_t*>(p - sh);
    const uint32_t r0 = b[0], r1 = b[1], r2 = sh ? b[2] : 0u;
    o[0] = __builtin_amdgcn_alignbyte(r1, r0, sh);
    o[1] = __builtin_amdgcn_alignbyte(r2, r1, sh);
}

__device__ __forceinline__ float half_bits(uint32_t h) {
    return (float)__builtin_bit_cast(f16, (uint16_t)(h & 0xFFFF));
}
__device__ __forceinline__ uint32_t byte_of(const uint32_t* w, int i) { return (w[i >> 2] >> (8 * (i & 3))) & 0xFF; }

// Raw W bytes of one 32-weight unit (row, part) of a chunk: four units a
// row, each 32 of the chunk's 128 weights.
//  Q4_K: chunk = half hf of a super-block; part p is sub-block 4 hf + p, one
//        nibble (p & 1) of the 32 quant bytes of pair 2 hf + (p >> 1):
//        words 0-3 the block header (d, dmin, 12 scale bytes), 4-11 the
//        pair's quant bytes.
//  Q6_K: chunk = half h; part p takes l in [8 p, 8 p + 8) of every 32-wide
//        quarter: words 0-1 ql[8 p ..], 2-3 ql[32 + 8 p ..], 4-5 qh[8 p ..]
//        (of the half), 6-7 the half's 8 scales, 8 d.
//  Q8_0: chunk = four blocks; part p takes block p (34 bytes: words 0-7
//        bytes 0-31 from a 2-byte aligned start, word 8 bytes 32-33).
template <int TY>
__device__ __forceinline__ void load_w(const uint8_t* row, int k0, int part, uint32_t* rw) {
    if constexpr (TY == kGQ4K) {
        const uint8_t* blk = row + (size_t)(k0 >> 8) * 144;
        const int hf = (k0 >> 7) & 1;
        const u32x4 h4 = *reinterpret_cast<const u32x4*>(blk);
        const uint8_t* qb = blk + 16 + 32 * (2 * hf + (part >> 1));
        const u32x4 q0 = *reinterpret_cast<const u32x4*>(qb);
        const u32x4 q1 = *reinterpret_cast<const u32x4*>(qb + 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            rw[i] = h4[i];
            rw[4 + i] = q0[i];
            rw[8 + i] = q1[i];
        }
    } else if constexpr (TY == kGQ6K) {
        const uint8_t* blk = row + (size_t)(k0 >> 8) * 210;
        const int h = (k0 >> 7) & 1;
        const uint8_t* ql = blk + 64 * h + 8 * part;
        ld8_a2(ql, rw + 0);
        ld8_a2(ql + 32, rw + 2);
        ld8_a2(blk + 128 + 32 * h + 8 * part, rw + 4);
        ld8_a2(blk + 192 + 8 * h, rw + 6);
        rw[8] = *reinterpret_cast<const uint16_t*>(blk + 208);
    } else {
        const uint8_t* blk = row + (size_t)((k0 >> 5) + part) * 34;
#pragma unroll
        for (int i = 0; i < 4; ++i) ld8_a2(blk + 8 * i, rw + 2 * i);
        rw[8] = *reinterpret_cast<const uint16_t*>(blk + 32);
    }
}

// Eight small integers as f16 into 8-half chunk c of LDS row r.
__device__ __forceinline__ void put8(f16* q_s, int r, int c, const int (&v)[8]) {
    f16x8 h;
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = (f16)(float)v[j];
    *reinterpret_cast<f16x8*>(&q_s[sw(r, c)]) = h;
}

// Decode thread (row r, part)'s raw bytes into q_s (f16 integers) and its
// groups' (scale, offset) into so_s.
template <int TY>
__device__ __forceinline__ void stash_w(const uint32_t* rw, int k0, int r, int part, bool live, f16* q_s,
                                        f32x2* so_s) {
    constexpr int NG = kGK / GTraits<TY>::gs;
    if constexpr (TY == kGQ4K) {
        // weights 32 part + e of the chunk: nibble (part & 1) of quant byte e
        // of the pair (quant.rs:54-128)
        const uint32_t* q = rw + 4;
        const int nib = 4 * (part & 1);
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            int v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = (int)((byte_of(q, 8 * cc + j) >> nib) & 0xF);
            put8(q_s, r, 4 * part + cc, v);
        }
        // sub-block j = 4 hf + part: scale and min, quant.rs:33-47
        const int j = 4 * ((k0 >> 7) & 1) + part;
        const float d = half_bits(rw[0]), dmin = half_bits(rw[0] >> 16);
        const uint32_t* sc6 = rw + 1;  // the 12 scale bytes
        uint32_t sc, m;
        if (j < 4) {
            sc = byte_of(sc6, j) & 63;
            m = byte_of(sc6, j + 4) & 63;
        } else {
            sc = (byte_of(sc6, j + 4) & 0xF) | ((byte_of(sc6, j - 4) >> 6) << 4);
            m = (byte_of(sc6, j + 4) >> 4) | ((byte_of(sc6, j) >> 6) << 4);
        }
        so_s[r * NG + part] = live ? f32x2{d * (float)sc, -(dmin * (float)m)} : f32x2{0.f, 0.f};
    } else if constexpr (TY == kGQ6K) {
        // weight 32 k + l of the half (l = 8 part + j): low / high nibble
        // (k >> 1) of ql[l + 32 (k & 1)], with bits 2k, 2k + 1 of qh[l] on
        // top, minus 32
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            int v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t lb = byte_of(rw + 2 * (k & 1), j);
                const uint32_t hb = byte_of(rw + 4, j);
                v[j] = (int)(((lb >> (4 * (k >> 1))) & 0xF) | (((hb >> (2 * k)) & 3) << 4)) - 32;
            }
            put8(q_s, r, 4 * k + part, v);
        }
        // groups of 16: g = 2 k + (l >= 16), written by parts 0 and 2
        if ((part & 1) == 0) {
            const float d = half_bits(rw[8]);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int g = 2 * k + (part >> 1);
                const float sc = (float)(int8_t)byte_of(rw + 6, g);
                so_s[r * NG + g] = live ? f32x2{d * sc, 0.f} : f32x2{0.f, 0.f};
            }
        }
    } else {
        // block part: d at bytes 0-1, quants at bytes 2-33
        const float d = half_bits(byte_of(rw, 0) | (byte_of(rw, 1) << 8));
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            int v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = (int)(int8_t)byte_of(rw, 2 + 8 * cc + j);
            put8(q_s, r, 4 * part + cc, v);
        }
        so_s[r * NG + part] = live ? f32x2{d, 0.f} : f32x2{0.f, 0.f};
    }
}

// Q8_0, two units a thread: blocks 2 pair and 2 pair + 1 of the chunk, 68
// contiguous bytes (dword-aligned when rows are, as 4096-wide ones are) as
// 17 words; separate 34-byte units would put every other block 2 bytes off a
// dword (15-20% slower).
__device__ __forceinline__ void load_q8_pair(const uint8_t* row, int k0, int pair, uint32_t* rw) {
    const uint8_t* blk = row + (size_t)((k0 >> 5) + 2 * pair) * 34;
#pragma unroll
    for (int i = 0; i < 8; ++i) ld8_a2(blk + 8 * i, rw + 2 * i);
    // the last 4 bytes (block 2 pair + 1's final quants) as two 2-byte loads
    rw[16] = (uint32_t)reinterpret_cast<const uint16_t*>(blk + 64)[0] |
             ((uint32_t)reinterpret_cast<const uint16_t*>(blk + 66)[0] << 16);
    rw[17] = 0u;
}
__device__ __forceinline__ void stash_q8_pair(const uint32_t* rw, int r, int pair, bool live, f16* q_s,
                                              f32x2* so_s) {
    constexpr int NG = kGK / GTraits<kGQ8_0>::gs;
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
        // block 2 pair + bi: d at bytes 34 bi, quants at 34 bi + 2
        const int base = 34 * bi;
        const float d = half_bits(byte_of(rw, base) | (byte_of(rw, base + 1) << 8));
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            int v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = (int)(int8_t)byte_of(rw, base + 2 + 8 * cc + j);
            put8(q_s, r, 4 * (2 * pair + bi) + cc, v);
        }
        so_s[r * NG + 2 * pair + bi] = live ? f32x2{d, 0.f} : f32x2{0.f, 0.f};
    }
}

template <int TY>
__global__ __launch_bounds__(g_threads<TY>(), 1) void qgemm_kernel(GemmArgs a) {
    constexpr int GS = GTraits<TY>::gs;
    constexpr int NG = kGK / GS;          // groups per chunk
    constexpr int KPG = GS / 16;          // MFMA k-steps per group
    constexpr bool OFFSET = TY == kGQ4K;  // groups carry an offset (Q4_K's min)
    constexpr int WW = GTraits<TY>::words;
    // Two buffers of every stage: chunk ch lives in buffer ch & 1.
    __shared__ __attribute__((aligned(16))) f16 xh_s[2][kGM * kGK];
    __shared__ __attribute__((aligned(16))) f16 xl_s[2][kGM * kGK];
    __shared__ __attribute__((aligned(16))) f16 q_s[2][kGN * kGK];
    __shared__ __attribute__((aligned(16))) f32x2 so_s[2][kGN * NG];        // (s, o) per row, group
    __shared__ __attribute__((aligned(16))) float xs_s[2][OFFSET ? NG * kGM : 4];  // x sums per group, token
    // Per token: the ratio 2^(k_new - k_old) of its x scale in this chunk,
    // and 2^-k_new.
    __shared__ __attribute__((aligned(16))) float rs_s[2][kGM];
    __shared__ __attribute__((aligned(16))) float iv_s[2][kGM];

    const int n_tb = (a.n_tok + kGM - 1) / kGM;
    const int tb = blockIdx.x % n_tb, rb = blockIdx.x / n_tb;
    const int t0 = tb * kGM, r0 = rb * kGN;
    const int tid = threadIdx.x;
    const int n_chunks = a.in_dim / kGK;

    // The W-producer waves (eight for Q6_K, else four) and x-producer waves
    // (four) load, decode and stash chunk ch + 1 while the consumer waves (the
    // first kGCons) multiply chunk
    // ch: a SIMD holds waves of every kind, so the producers' VALU work issues
    // beside the consumers' MFMAs.  One barrier per chunk; every wave executes
    // the same number of barriers.
    constexpr int WPARTS = g_wparts<TY>(), WU = 4 / WPARTS;  // threads a row, units a thread
    constexpr int WT = kGN * WPARTS;                           // W-producer threads
    if (tid >= kGConsT) {
        const bool x_prod = tid >= kGConsT + WT;  // wave-uniform
        const int ptid = x_prod ? tid - kGConsT - WT : tid - kGConsT;
        // ---- register prefetch of one chunk
        // x: 64 tokens x 128 floats = 2048 float4, XU per thread; 32
        // consecutive threads read one token's 512 contiguous bytes.
        constexpr int XT = g_xthreads<TY>(), XU = kGXF / XT;  // x-producer threads, float4s a thread
        f32x4 rx[XU];
        // Running scale exponent k_t of each of this thread's tokens (100:
        // no nonzero x seen yet; any ratio applied to a zero y is exact).
        int kx[XU];
#pragma unroll
        for (int u = 0; u < XU; ++u) kx[u] = 100;
        bool ones[2] = {false, false};  // buffer b holds (1, 1) for this wave's tokens (wave-uniform)
        constexpr bool Q8PAIR = TY == kGQ8_0 && WU == 2;
        uint32_t rw[WU][Q8PAIR ? 18 : WW];
        const int w_row = ptid / WPARTS, w_part = ptid % WPARTS;
        const bool w_thread = w_row < kGN;  // threads past the tile's rows stage no W
        const bool w_live = w_thread && r0 + w_row < a.rows;
        const uint8_t* wrow = a.w + (size_t)(w_live ? r0 + w_row : 0) * a.row_bytes;
        auto load_chunk = [&](int k0) {
            if (x_prod) {
#pragma unroll
                for (int u = 0; u < XU; ++u) {
                    const int i = ptid + XT * u, tok = i >> 5, k4 = i & 31;
                    f32x4 v = {0.f, 0.f, 0.f, 0.f};
                    if (t0 + tok < a.n_tok)
                        v = *reinterpret_cast<const f32x4*>(a.x + (size_t)(t0 + tok) * a.in_dim + k0 + 4 * k4);
                    rx[u] = v;
                }
            } else if (w_thread) {
                if constexpr (Q8PAIR) {
                    load_q8_pair(wrow, k0, w_part, rw[0]);
                } else {
#pragma unroll
                    for (int u = 0; u < WU; ++u) load_w<TY>(wrow, k0, w_part * WU + u, rw[u]);
                }
            }
        };
        auto stash_chunk = [&](int k0, int b) {
            if (!x_prod) {
                if (w_thread) {
                    if constexpr (Q8PAIR) {
                        stash_q8_pair(rw[0], w_row, w_part, w_live, q_s[b], so_s[b]);
                    } else {
#pragma unroll
                        for (int u = 0; u < WU; ++u)
                            stash_w<TY>(rw[u], k0, w_row, w_part * WU + u, w_live, q_s[b], so_s[b]);
                    }
                }
                return;
            }
            // x (scaled by 2^kn) to f16 hi / lo rows, the token's ratio and
            // inverse scale, and (Q4_K) the group sums
            auto emit = [&](int u, const f32x4& xv, float ratio, int kn, bool store_scale) {
                const int i = ptid + XT * u, tok = i >> 5, k4 = i & 31;
                if (store_scale && k4 == 0) {
                    rs_s[b][tok] = ratio;
                    iv_s[b][tok] = __builtin_amdgcn_ldexpf(1.f, -kn);
                }
                f16x4 hi, lo;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    hi[j] = (f16)xv[j];
                    lo[j] = (f16)(xv[j] - (float)hi[j]);
                }
                const int off = sw(tok, k4 >> 1) + 4 * (k4 & 1);
                *reinterpret_cast<f16x4*>(&xh_s[b][off]) = hi;
                *reinterpret_cast<f16x4*>(&xl_s[b][off]) = lo;
                if constexpr (OFFSET) {
                    // the group's (scaled) x sum: eight consecutive lanes hold its 32 floats
                    float sx = (xv[0] + xv[1]) + (xv[2] + xv[3]);
                    sx = sum8(sx);
                    if ((k4 & 7) == 0) xs_s[b][(k4 >> 3) * kGM + tok] = sx;
                }
            };
            // Scale rule per (token, chunk), m the token's largest |x| in the
            // chunk: k_c = 0 for m in [2^-6, 2^14), else 15 - e(m) with
            // m < 2^e (so m 2^k_c lies in [2^14, 2^15)); no bound for m = 0
            // or m not finite; k_t = min(k_t, k_c) from k_t = 100.  Once
            // k_t = 0 and no |x| of the chunk reaches 2^14, k_t stays 0, so a
            // wave whose tokens are all there skips the reduction and the
            // scaling (the common case after the first chunk).
            float ml[XU];
            bool slow = false;
#pragma unroll
            for (int u = 0; u < XU; ++u) {
                ml[u] = fmaxf(fmaxf(fabsf(rx[u][0]), fabsf(rx[u][1])), fmaxf(fabsf(rx[u][2]), fabsf(rx[u][3])));
                slow |= !(ml[u] < 16384.f) || kx[u] != 0;
            }
            if (__builtin_amdgcn_ballot_w64(slow) == 0) {
                // the wave's tokens keep scale 1: their (ratio, 1 / scale)
                // entries need writing only if buffer b does not hold (1, 1)
                const bool store = !ones[b];
#pragma unroll
                for (int u = 0; u < XU; ++u) emit(u, rx[u], 1.f, 0, store);
                ones[b] = true;
                return;
            }
            ones[b] = false;
#pragma unroll
            for (int u = 0; u < XU; ++u) {
                // the token's 128 floats are on 32 consecutive lanes
                const float m = max32(ml[u]);
                int kn = kx[u];
                if (m > 0.f && m <= 3.402823466e38f && !(m >= 0.015625f && m < 16384.f))
                    kn = min(kn, 15 - __builtin_amdgcn_frexp_expf(m));
                else if (m >= 0.015625f && m < 16384.f)
                    kn = min(kn, 0);
                const float ratio = __builtin_amdgcn_ldexpf(1.f, kn - kx[u]);
                kx[u] = kn;
                f32x4 xv;
#pragma unroll
                for (int j = 0; j < 4; ++j) xv[j] = __builtin_amdgcn_ldexpf(rx[u][j], kn);
                emit(u, xv, ratio, kn, true);
            }
        };
        load_chunk(0);
        stash_chunk(0, 0);
        if (n_chunks > 1) load_chunk(kGK);  // in flight during chunk 0's MFMAs
        __syncthreads();
        for (int ch = 0; ch < n_chunks; ++ch) {
            // Buffer (ch + 1) & 1 was last read in iteration ch - 1, before
            // that iteration's barrier.
            if (ch + 1 < n_chunks) {
                stash_chunk((ch + 1) * kGK, (ch + 1) & 1);
                if (ch + 2 < n_chunks) load_chunk((ch + 2) * kGK);
            }
            __syncthreads();
        }
        return;
    }

    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int l32 = lane & 31, hh = lane >> 5;
    f32x16 y[kNTW];
#pragma unroll
    for (int n = 0; n < kNTW; ++n)
#pragma unroll
        for (int j = 0; j < 16; ++j) y[n][j] = 0.f;

    __syncthreads();  // chunk 0 is stashed
    // tokens of register j: 8 (j / 4) + 4 hh + j % 4 of the wave's 32
    auto token_vals = [&](const float* src, f32x4 (&v)[4]) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) v[q4] = *reinterpret_cast<const f32x4*>(src + 32 * wm + 8 * q4 + 4 * hh);
    };
    for (int ch = 0; ch < n_chunks; ++ch) {
        const int b = ch & 1;
        // y so far moves to each token's scale of this chunk (a power of two,
        // exact; 1 unless the chunk lowered it).  Unconditional: a branch on
        // a change flag costs the Q6_K consumer spills.
        {
            f32x4 rt[4];
            token_vals(rs_s[b], rt);
#pragma unroll
            for (int n = 0; n < kNTW; ++n)
#pragma unroll
                for (int j = 0; j < 16; ++j) y[n][j] *= rt[j >> 2][j & 3];
        }
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            f32x16 acc[kNTW];
#pragma unroll
            for (int n = 0; n < kNTW; ++n)
#pragma unroll
                for (int j = 0; j < 16; ++j) acc[n][j] = 0.f;
#pragma unroll
            for (int kk = 0; kk < KPG; ++kk) {
                const int c = 2 * (g * KPG + kk) + hh;
                const int xr = 32 * wm + l32;
                const f16x8 ah = *reinterpret_cast<const f16x8*>(&xh_s[b][sw(xr, c)]);
                const f16x8 al = *reinterpret_cast<const f16x8*>(&xl_s[b][sw(xr, c)]);
#pragma unroll
                for (int n = 0; n < kNTW; ++n) {
                    const f16x8 bq = *reinterpret_cast<const f16x8*>(&q_s[b][sw(32 * kNTW * wn + 32 * n + l32, c)]);
                    acc[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bq, acc[n], 0, 0, 0);
                    acc[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bq, acc[n], 0, 0, 0);
                }
            }
            // tokens of register j: 8 (j / 4) + 4 hh + j % 4 of the wave's 32
            f32x4 xs[4];
            if constexpr (OFFSET) {
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4)
                    xs[q4] = *reinterpret_cast<const f32x4*>(&xs_s[b][g * kGM + 32 * wm + 8 * q4 + 4 * hh]);
            }
#pragma unroll
            for (int n = 0; n < kNTW; ++n) {
                const f32x2 so = so_s[b][(32 * kNTW * wn + 32 * n + l32) * NG + g];
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    float v = fmaf(so[0], acc[n][j], y[n][j]);
                    if constexpr (OFFSET) v = fmaf(so[1], xs[j >> 2][j & 3], v);
                    y[n][j] = v;
                }
            }
        }
        __syncthreads();  // chunk ch's operands are read; chunk ch + 1 is stashed
    }

    // back from each token's final x scale (the last chunk's buffer is not
    // written again)
    f32x4 iv[4];
    token_vals(iv_s[(n_chunks - 1) & 1], iv);
#pragma unroll
    for (int n = 0; n < kNTW; ++n) {
        const int r = r0 + 32 * kNTW * wn + 32 * n + l32;
        if (r >= a.rows) continue;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int t = t0 + 32 * wm + 8 * (j >> 2) + 4 * hh + (j & 3);
            if (t < a.n_tok) a.y[(size_t)t * a.rows + r] = y[n][j] * iv[j >> 2][j & 3];
        }
    }
}

// y [n_tok, rows] = W x: one launch, W read once from HBM (each of the
// ceil(n_tok / 64) token blocks of a row block reads it from L2 or the
// last-level cache after the first).
lmx_status qgemm(const lmx_qmv_desc* d, const void* w, const float* x, float* y, hipStream_t st) {
    size_t bb = 0, be = 0;
    switch (d->type) {
        case kGQ4K: bb = 144; be = 256; break;
        case kGQ6K: bb = 210; be = 256; break;
        case kGQ8_0: bb = 34; be = 32; break;
        default: return LMX_E_UNSUPPORTED;
    }
    if (d->in_dim % kGK || d->in_dim % be) return LMX_E_SHAPE;
    GemmArgs a{};
    a.w = static_cast<const uint8_t*>(w);
    a.x = x;
    a.y = y;
    a.rows = (int)d->rows;
    a.in_dim = (int)d->in_dim;
    a.n_tok = (int)d->n_tok;
    a.row_bytes = (size_t)d->in_dim / be * bb;
    const long n_tb = ((long)d->n_tok + kGM - 1) / kGM, n_rb = ((long)d->rows + kGN - 1) / kGN;
    if (n_tb * n_rb > INT32_MAX) return LMX_E_SHAPE;
    const dim3 grid((unsigned)(n_tb * n_rb));
    (void)hipGetLastError();
    switch (d->type) {
        case kGQ4K: hipLaunchKernelGGL(qgemm_kernel<kGQ4K>, grid, dim3(g_threads<kGQ4K>()), 0, st, a); break;
        case kGQ6K: hipLaunchKernelGGL(qgemm_kernel<kGQ6K>, grid, dim3(g_threads<kGQ6K>()), 0, st, a); break;
        default: hipLaunchKernelGGL(qgemm_kernel<kGQ8_0>, grid, dim3(g_threads<kGQ8_0>()), 0, st, a); break;
    }
    LMX_CHECK_LAUNCH();
    return LMX_OK;
}

}  // namespace lmx
