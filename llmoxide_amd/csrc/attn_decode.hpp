// Split-K attention for few query tokens (decode) on gfx950: kernels.
//
// Instantiated per (query dtype, addressing mode) in attn_decode_*.hip;
// planning and the entry points are in attn_decode.hip.
//
// Replaces, for n_tokens small, the reference's three passes scores_pass /
// softmax_pass / weighted_v (attn.wgsl:84-232), which give decode only
// n_heads workgroups and a serial key loop (attn.wgsl:13-17).
//
// Work split.  A workgroup owns HW kv heads (one wave group per head) for a
// block of GB query heads per kv head, one query row, and split s of the
// visible keys: the contiguous 16-key tiles [s*tps, (s+1)*tps).  K/V rows
// are read once for all GB query heads of a kv head (GQA) and with
// non-temporal loads (they are streamed, never re-read).  Each wave keeps
// DEPTH tiles of K/V in registers: while it computes one, the next ones'
// loads are in flight.
//
// A workgroup is four waves, one per SIMD.  When two streaming waves share
// a SIMD, the memory pipeline serves the first one faster (measured with
// eight-wave workgroups at H 32, Hkv 8, hd 128 over 32k keys: the first wave
// of each SIMD finished its equal share at 16 us, the second at 22 us, and
// giving the first more of the tiles only slowed it without speeding the
// second).  With one wave
// per SIMD and one workgroup per CU nobody waits on a slower partner.  Row addressing is branch-free: a linear cache reads row p,
// a ring reads slot p % window (multiply-high division), and rows of the
// current batch can come from a separate k_cur/v_cur buffer.
//
// Per wave and tile:
//   S^T[16 keys x 16 cols] = K Q^T on v_mfma_f32_16x16x32_f16.  Columns
//   0..GB-1 hold the f16 high part of each query head, columns GB..2GB-1 the
//   f16 residual (q - hi) of an fp32 query, so q.k is exact to ~2^-22.
//   Lane (g, c) then holds keys 4g..4g+3 of column c.  Each 16-lane group g
//   runs its own online softmax over its four keys of every tile (fp32, exp2
//   with scale*log2(e) folded in), so no value crosses groups inside the
//   loop; the four streams are merged once at the end.  p goes through a
//   per-wave LDS slot to the P.V lanes of the same group; those read V rows
//   coalesced (16 lanes cover one 256-byte row) and accumulate in fp32.
//
// Merge.  With one split per unit the workgroup writes the output.  Else
// each split workgroup stores one partial (max, sum, o[hd]) per query head
// and a second, small kernel merges them: each of its threads folds up to
// eight partials of one float4 column (all loads issued at once), and the
// parts of a column, adjacent lanes of one wave, are combined by shuffles.
// The launch boundary orders the partial stores before the merge loads; no
// counters, so the pair can be replayed from a captured graph as is.  (A
// single-launch form, where the last split workgroup of a unit merges it,
// loses at one query row.  With device-scope fences in every workgroup
// (L2 write-back and invalidate) the kernel took 67 us instead of 24.
// Without them, a unit's splits must share one L2: workgroup b runs on XCD
// b % 8, so one kv head per workgroup and per XCD; then the merge costs
// 2.5 us instead of 4.3, but reading one head's 256-byte slice of each row
// instead of four heads' 1 KB streams 13% slower (26.8 vs 23.7 us at the
// Qwen3-8B 32k headline; 29.3 us a call against 27.4).)
#pragma once

#include <climits>
#include <cstdlib>
#include <type_traits>

#include "common.hpp"

namespace lmx {

enum DecodeMode { kModeLinear = 0, kModeGeneral = 1, kModeBatched = 2 };

// Timeline hook: a measurement build defines LMX_DECODE_MARK(i) before
// including this header (llmoxide_amd/timeline/decode_timeline.hip stores each
// wave's s_memrealtime at phase i: 0 entry, 1 query converted, 2 first tile
// done, 3 last tile done, 4 partials stored), in attn_decode_kernel and
// attn_decode_mh_kernel.  The library leaves it empty.
#ifndef LMX_DECODE_MARK
#define LMX_DECODE_MARK(i) ((void)0)
#endif

struct DecodeArgs {
    const void* q;
    const f16* k;
    const f16* v;
    const f16* const* k_ptrs;
    const f16* const* v_ptrs;
    const f16* k_cur;
    const f16* v_cur;
    const int32_t* ctx_lens;
    float* out;
    const float* gate;      // NULL, or the output gate: out *= sigmoid(gate[row * gate_stride + d])
    int q_stride;           // elements between consecutive query heads
    int gate_stride;
    float* part_o;          // [n_q][H][P][HD]  per-split partials
    float* part_ml;         // [n_q][H][P][2]   (max in log2 units, sum)
    int H, Hkv, G, kv_dim;
    int base_pos, window, n_tokens, bidi;
    int P, tps, n_hblk;
    int n_q;                // query rows (tokens, or sequences when batched)
    int n_main, n_yg;       // split workgroups; their (kv group, head block) count
    int n_merge, m_parts;   // merge workgroups; lanes per merged column
    int max_ctx;            // batched: context lengths are clamped to [1, max_ctx]
    uint32_t w_magic;       // p % window == p - window * ((p * w_magic) >> w_shift)
    int w_shift;
    float c;                // scale * log2(e)
};

constexpr int kWaves = 4;  // one wave per SIMD (see "Work split")
constexpr int kDecThreads = kWaves * 64;
constexpr int kMaxP = 512;  // splits per unit
constexpr int kTile = 16;   // keys per wave tile
constexpr int kMergePer = 8;            // partials per merge thread
#ifndef LMX_DEC_DEPTH_128
#define LMX_DEC_DEPTH_128 2  // K/V tiles in flight per wave at head_dim 128
#endif
#ifndef LMX_DEC_DEPTH_256
#define LMX_DEC_DEPTH_256 1  // at head_dim 256
#endif
#ifndef LMX_DEC_SHARED_HD
#define LMX_DEC_SHARED_HD 512  // head sizes from this one up load K/V through L2
#endif

// Visible keys [lo, hi] of query row qi (attn.wgsl:52-66 first/last_visible;
// batched: the sequence's last position).
template <int MODE>
__device__ __forceinline__ void unit_range(const DecodeArgs& a, int qi, int& lo, int& hi) {
    int pos;
    if constexpr (MODE == kModeBatched) {
        // Out-of-range lengths are clamped so every read stays in the cache
        // the caller sized for max_ctx.
        pos = min(max(a.ctx_lens[qi], 1), a.max_ctx) - 1;
        hi = pos;
    } else {
        pos = a.base_pos + qi;
        if (a.bidi) {
            const int end = a.base_pos + a.n_tokens - 1;
            hi = a.window ? min(end, pos + a.window - 1) : end;
        } else {
            hi = pos;
        }
    }
    lo = (a.window && pos + 1 > a.window) ? pos + 1 - a.window : 0;
}

// Order LDS traffic between lanes of one wave (LDS executes a wave's
// accesses in order; this keeps the compiler from reordering them).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Row rotate within a 16-lane DPP row: lane i receives lane (i + N) % 16.
template <int N>
__device__ __forceinline__ float row_rotate_down(float x) {
    return dpp<0x120 + (16 - N)>(x);  // row_ror:(16-N)
}

// Per-lane K/V registers of one 16-key tile.
//  K (MFMA A operand): lane (key c16, group g4), k-step s holds dims
//    32s + 8g4 .. +7 of key c16: each load covers 64 contiguous bytes per key.
//  V (P.V operand): load i, lane (g4, c16) holds key 4g4 + i, dims
//    128r + 8c16 .. +7 (HD >= 128, piece r) or 4c16 .. +3 (HD == 64): 16 lanes
//    cover one row, coalesced.
template <int HD>
struct KVTile {
    static constexpr int KS = HD / 32;
    static constexpr int VR = HD >= 128 ? HD / 128 : 1;
    static constexpr int VW = HD >= 128 ? 8 : 4;  // halfs per V piece
    f16x8 k[KS];
    RawF16<VW> v[4][VR];
};

template <int HD>
__device__ __forceinline__ int v_dim(int c16, int r, int j) {
    return HD >= 128 ? 128 * r + 8 * c16 + j : 4 * c16 + j;
}

// Streaming loads where the cache is read once per call (NT); plain loads
// where several head blocks of one kv head read the same rows, so that the
// XCD's L2 serves all but the first.
template <bool NT>
__device__ __forceinline__ f16x8 ld_stream8(const f16* p) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(p));
    return *reinterpret_cast<const f16x8*>(p);
}
template <bool NT>
__device__ __forceinline__ f16x4 ld_stream4(const f16* p) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const f16x4*>(p));
    return *reinterpret_cast<const f16x4*>(p);
}

// Merge: thread (column, part) folds partials part, part + m_parts, ... (at
// most kMergePer) of one float4 column of one (query row, head), issuing all
// its loads at once.  The m_parts lanes of a column are adjacent in the wave
// (m_parts is a power of two <= 64), so they combine by shuffles: no LDS and
// no barrier.  Rows with a single split were written by the split kernel and
// are skipped.
template <int HD, int MODE>
__global__ __launch_bounds__(kDecThreads) void attn_merge_kernel(DecodeArgs a) {
    constexpr int C4 = HD / 4;  // float4 columns of a head
    args_in_sgprs(a.part_o, a.part_ml, a.out, a.gate, a.gate_stride, a.m_parts, a.n_q, a.H, a.P, a.tps, a.window);
    if constexpr (MODE == kModeBatched)
        args_in_sgprs(a.ctx_lens, a.max_ctx);
    else
        args_in_sgprs(a.base_pos, a.n_tokens, a.bidi);
    const int tid = threadIdx.x;
    const int parts = a.m_parts;
    const int part = tid & (parts - 1);
    const long col = (long)blockIdx.x * (kDecThreads / parts) + tid / parts;
    const bool have = col < (long)a.n_q * a.H * C4;
    const long cc = have ? col : 0;
    const size_t row = (size_t)(cc / C4);  // qi * H + h
    const int d0 = 4 * (int)(cc % C4);
    const int qi = (int)(row / a.H);
    int lo, hi;
    unit_range<MODE>(a, qi, lo, hi);
    const int n_tiles = (hi - lo + kTile) / kTile;
    const int p_u = (n_tiles + a.tps - 1) / a.tps;
    const bool merge = have && p_u > 1;  // the same for every lane of a column
    // -1e30: a lane without partials keeps weight 0 in the combine below
    float m_run = -1e30f, l_run = 0.f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (merge) {
        const float* po = a.part_o + row * a.P * HD + d0;
        const float* pml = a.part_ml + row * a.P * 2;
        float m[kMergePer], l[kMergePer];
        f32x4 x[kMergePer];
#pragma unroll
        for (int k = 0; k < kMergePer; ++k) {
            const int s = part + k * parts;
            const int sc = s < p_u ? s : 0;  // a valid partial; weighted out below
            const f32x2 ml = *reinterpret_cast<const f32x2*>(pml + 2 * sc);
            m[k] = s < p_u ? ml[0] : -INFINITY;
            l[k] = ml[1];
            x[k] = *reinterpret_cast<const f32x4*>(po + (size_t)sc * HD);
        }
#pragma unroll
        for (int k = 0; k < kMergePer; ++k) m_run = fmaxf(m_run, m[k]);
#pragma unroll
        for (int k = 0; k < kMergePer; ++k) {
            const float w = fast_exp2(m[k] - m_run);  // 0 for the unused slots
            l_run = fmaf(l[k], w, l_run);
            acc[0] = fmaf(x[k][0], w, acc[0]);
            acc[1] = fmaf(x[k][1], w, acc[1]);
            acc[2] = fmaf(x[k][2], w, acc[2]);
            acc[3] = fmaf(x[k][3], w, acc[3]);
        }
    }
    for (int off = 1; off < parts; off <<= 1) {
        const float m2 = shfl_xor(m_run, off), l2 = shfl_xor(l_run, off);
        f32x4 y;
#pragma unroll
        for (int j = 0; j < 4; ++j) y[j] = shfl_xor(acc[j], off);
        const float mn = fmaxf(m_run, m2);
        const float c0 = fast_exp2(m_run - mn), c1 = fast_exp2(m2 - mn);
        l_run = l_run * c0 + l2 * c1;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = acc[j] * c0 + y[j] * c1;
        m_run = mn;
    }
    if (merge && part == 0) {
        const float inv = 1.f / l_run;
        f32x4 y = f32x4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
        if (a.gate) y = gate_sigmoid4(y, a.gate + row * a.gate_stride + d0);
        *reinterpret_cast<f32x4*>(a.out + row * HD + d0) = y;
    }
}

template <typename QT, int HD, int GB, int HW, int MODE, bool KR>
__global__ __launch_bounds__(kDecThreads) void attn_decode_kernel(DecodeArgs a) {
    using Tile = KVTile<HD>;
    constexpr int KS = Tile::KS, VR = Tile::VR, VW = Tile::VW;
    // KR (head_dim 128 and 256): K loaded row-major, as V, and turned into
    // MFMA operands through LDS, so that each load instruction reads four
    // whole 256-byte row pieces instead of 64 bytes of sixteen rows.  The launch picks it
    // (pick_krows); without it each lane loads its operand bytes directly.
    constexpr bool KROWS = KR && (HD == 128 || HD == 256);
    constexpr int KRP = HD >= 128 ? HD / 128 : 1;  // 128-dim pieces of a K row (as V's)
    constexpr int DPL = HD / 16;  // V dims per lane
    constexpr int WPH = kWaves / HW;  // waves per kv head
    constexpr bool SPLIT_Q = sizeof(QT) == 4;
    constexpr bool kNtLoads = HD < LMX_DEC_SHARED_HD;
    // PIPE also at head_dim 256 with DEPTH 1: the first tile's loads go out
    // with the query's, before its conversion (Gemma global decode 43.6 ->
    // 41.6 us, the 1024-key window 0.6 us shorter per workgroup).
    constexpr bool PIPE = HD <= 256;
    // Tiles in flight per wave (a 16-key tile is 16 K + 16 V registers per
    // lane at hd 128, 8 + 8 at hd 64).  At hd 128 two measured best: with
    // one wave per SIMD, deeper buffers (3, 4, 6) only lengthen the start.
    constexpr int DEPTH = !PIPE ? 1 : (HD <= 64 ? 4 : (HD == 256 ? LMX_DEC_DEPTH_256 : LMX_DEC_DEPTH_128));
    static_assert(GB * (SPLIT_Q ? 2 : 1) <= 16, "query columns");
    static_assert(VR * VW == DPL, "V lane layout");
    static_assert(kWaves % HW == 0, "waves per head");

    args_in_sgprs(a.q, a.out, a.gate, a.part_o, a.part_ml, a.q_stride, a.gate_stride, a.H, a.G, a.kv_dim, a.P,
                  a.tps, a.n_hblk, a.n_yg, a.window, a.c);
    if constexpr (MODE == kModeBatched)
        args_in_sgprs(a.k_ptrs, a.v_ptrs, a.ctx_lens, a.max_ctx);
    else
        args_in_sgprs(a.k, a.v, a.k_cur, a.v_cur, a.base_pos, a.n_tokens, a.bidi, a.w_magic, a.w_shift);
    LMX_DECODE_MARK(0);
    const int bid = blockIdx.x;
    const int split = bid % a.P;
    const int yg = (bid / a.P) % a.n_yg;
    const int qi = bid / (a.P * a.n_yg);
    const int kvg = yg / a.n_hblk;  // group of HW kv heads
    const int hb = yg - kvg * a.n_hblk;

    int lo, hi;
    unit_range<MODE>(a, qi, lo, hi);
    const int n_tiles = (hi - lo + kTile) / kTile;
    const int t_begin = split * a.tps;
    if (t_begin >= n_tiles) return;  // uniform: this unit needs fewer splits
    const int t_end = min(t_begin + a.tps, n_tiles);
    const int p_u = (n_tiles + a.tps - 1) / a.tps;  // splits this unit uses

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int hs = wave % HW, wih = wave / HW;  // head slot, wave within head
    const int kvh = kvg * HW + hs;
    const int h0 = kvh * a.G + hb * GB;  // first query head of this wave
    const int g4 = lane >> 4, c16 = lane & 15;

    const f16 *kc, *vc;
    int cur_begin = INT_MAX;
    if constexpr (MODE == kModeBatched) {
        kc = a.k_ptrs[qi];
        vc = a.v_ptrs[qi];
    } else {
        kc = a.k;
        vc = a.v;
        if (MODE == kModeGeneral && a.k_cur) cur_begin = a.base_pos;
    }

    // Key position -> row pointer (no branches: selects only).
    auto row_ptr = [&](const f16* cache, const f16* cur, int p) -> const f16* {
        if constexpr (MODE == kModeLinear) {
            return cache + (size_t)p * a.kv_dim + kvh * HD;
        } else {
            int s = p;
            if (a.window) {
                const uint32_t qd = (uint32_t)(((uint64_t)(uint32_t)p * a.w_magic) >> a.w_shift);
                s = p - (int)qd * a.window;
            }
            const f16* rc = cache + (size_t)s * a.kv_dim;
            const f16* ru = cur + (size_t)(p - a.base_pos) * a.kv_dim;
            return (p >= cur_begin ? ru : rc) + kvh * HD;
        }
    };

    // Issue the loads of tile `t` (keys lo + 16t ..); rows past hi are
    // clamped to hi (their scores are masked).
    auto load_tile = [&](int t, Tile& b) {
        const int kt = lo + kTile * t;
        if constexpr (KROWS) {
            // K as V: load (i, r), lane (g4, c16) holds key 4 g4 + i, dims
            // 128 r + 8 c16 .. + 7 (one 256-byte piece per 16 lanes)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const f16* krow = row_ptr(kc, a.k_cur, min(kt + 4 * g4 + i, hi));
#pragma unroll
                for (int r = 0; r < KRP; ++r) b.k[i * KRP + r] = ld_stream8<kNtLoads>(krow + 128 * r + 8 * c16);
            }
        } else {
            const f16* krow = row_ptr(kc, a.k_cur, min(kt + c16, hi));
#pragma unroll
            for (int s = 0; s < KS; ++s) b.k[s] = ld_stream8<kNtLoads>(krow + 32 * s + 8 * g4);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f16* vrow = row_ptr(vc, a.v_cur, min(kt + 4 * g4 + i, hi));
#pragma unroll
            for (int r = 0; r < VR; ++r) {
                const f16* vp = vrow + v_dim<HD>(c16, r, 0);
                if constexpr (VW == 8) {
                    const f16x8 x = ld_stream8<kNtLoads>(vp);
                    b.v[i][r].v[0] = f16x4{x[0], x[1], x[2], x[3]};
                    b.v[i][r].v[1] = f16x4{x[4], x[5], x[6], x[7]};
                } else {
                    b.v[i][r].v[0] = ld_stream4<kNtLoads>(vp);
                }
            }
        }
    };

    // This wave's tiles: t_begin + wih, + WPH, ... below t_end.
    const int my_n = t_begin + wih < t_end ? (t_end - t_begin - wih + WPH - 1) / WPH : 0;
    auto tile_of = [&](int j) { return t_begin + wih + j * WPH; };

    __shared__ __attribute__((aligned(16))) float sm_o[kWaves][GB][HD];
    __shared__ float sm_m[kWaves][GB];
    __shared__ float sm_l[kWaves][GB];
    // Per-wave LDS slots: p[key][head] and corr[group][head] of the tile.
    __shared__ __attribute__((aligned(16))) float P_s[kWaves][kTile][8];
    // KROWS: the K tile, rows of HD + 8 halfs (the operand reads of 16 rows
    // then fall on distinct banks).
    __shared__ __attribute__((aligned(16))) f16 K_s[KROWS ? kWaves : 1][kTile][KROWS ? HD + 8 : 8];
    __shared__ __attribute__((aligned(16))) float C_s[kWaves][4][8];

    // Combine the WPH waves of each head slot (after a workgroup barrier):
    // element (hs, g, d) of the workgroup; waves hs, hs + HW, ... hold its
    // parts.
    auto combine_waves = [&]() {
      if constexpr (WPH > 1) {  // never instantiated with one wave per head
        __syncthreads();
        for (int idx = tid; idx < HW * GB * HD; idx += kDecThreads) {
            const int e_hs = idx / (GB * HD);
            const int rem = idx - e_hs * (GB * HD);
            const int g = rem / HD, d = rem - g * HD;
            float Mw = sm_m[e_hs][g];
#pragma unroll
            for (int ww = 1; ww < WPH; ++ww) Mw = fmaxf(Mw, sm_m[e_hs + ww * HW][g]);
            float O = 0.f, Lw = 0.f;
#pragma unroll
            for (int ww = 0; ww < WPH; ++ww) {
                const int w = e_hs + ww * HW;
                const float sc = fast_exp2(sm_m[w][g] - Mw);
                O = fmaf(sm_o[w][g][d], sc, O);
                Lw = fmaf(sm_l[w][g], sc, Lw);
            }
            const int head = (kvg * HW + e_hs) * a.G + hb * GB + g;
            const size_t row = (size_t)qi * a.H + head;
            if (p_u == 1) {
                const float y = O / Lw;
                a.out[row * HD + d] = a.gate ? gate_sigmoid(y, a.gate[row * a.gate_stride + d]) : y;
            } else {
                const size_t pidx = row * a.P + split;
                a.part_o[pidx * HD + d] = O;
                if (d == 0) {
                    a.part_ml[pidx * 2] = Mw;
                    a.part_ml[pidx * 2 + 1] = Lw;
                }
            }
        }
      }
    };

    // Everything from the first load to the wave's partial sits in one
    // uniform branch: no path merges loads issued with loads not issued, so
    // the compiler's wait counts stay exact.
    if (my_n > 0) {
        // Q^T as the MFMA B operand: column c16, dims 32s + 8g4 + j.  Columns
        // past the query heads read a valid row and are zeroed (no branches).
        // The raw loads go out first, the tile prefetch next, and the f16
        // conversion waits only for the Q loads.
        const bool hi_col = c16 < GB;
        const bool lo_col = SPLIT_Q && !hi_col && c16 < 2 * GB;
        const int qhead = h0 + (hi_col ? c16 : (lo_col ? c16 - GB : 0));
        using QRaw = typename std::conditional<SPLIT_Q, f32x4, f16x8>::type;
        constexpr int QN = SPLIT_Q ? 2 : 1;
        QRaw qraw[KS][QN];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const size_t qo = ((size_t)qi * a.H + qhead) * a.q_stride + 32 * s + 8 * g4;
            if constexpr (SPLIT_Q) {
                const float* qp = reinterpret_cast<const float*>(a.q) + qo;
                qraw[s][0] = *reinterpret_cast<const f32x4*>(qp);
                qraw[s][QN - 1] = *reinterpret_cast<const f32x4*>(qp + 4);
            } else {
                qraw[s][0] = *reinterpret_cast<const f16x8*>(reinterpret_cast<const f16*>(a.q) + qo);
            }
        }
        // The DEPTH prefetches are unconditional (a wave with fewer tiles reads
        // its last one again), so every path into the loop has the same loads
        // in flight and the compiler's wait counts stay exact.
        Tile bufs[DEPTH];
        const int last_t = my_n - 1;
        if constexpr (PIPE) {
#pragma unroll
            for (int k = 0; k < DEPTH; ++k) load_tile(tile_of(min(k, last_t)), bufs[k]);
        }
        __builtin_amdgcn_sched_barrier(0);

        f16x8 qf[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            f16x8 v;
            if constexpr (SPLIT_Q) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float x = qraw[s][j / 4][j % 4];
                    const f16 hi16 = (f16)x;
                    const f16 lo16 = (f16)(x - (float)hi16);
                    v[j] = hi_col ? hi16 : (lo_col ? lo16 : (f16)0.f);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = hi_col ? qraw[s][0][j] : (f16)0.f;
            }
            qf[s] = v;
        }
        LMX_DECODE_MARK(1);

        // Online-softmax state.  Each 16-lane group g4 runs its own stream over
        // keys 4g4..4g4+3 of every tile: lane (c16 < GB, g4) holds the running
        // max and sum of head c16, lane (g4, c16) the group's o over its dims.
        float m_run = -1e30f, l_run = 0.f;
        float o[GB][DPL];
#pragma unroll
        for (int h = 0; h < GB; ++h)
#pragma unroll
            for (int d = 0; d < DPL; ++d) o[h][d] = 0.f;

        const int key_end = hi + 1;
        auto compute_tile = [&](int t, const Tile& b) {
            const int kt = lo + kTile * t;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            if constexpr (KROWS) {
                // Row-major K tile through this wave's LDS slice, read back
                // as the MFMA A operand (key c16, dims 32 s + 8 g4 .. + 7).
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int r = 0; r < KRP; ++r)
                        *reinterpret_cast<f16x8*>(&K_s[wave][4 * g4 + i][128 * r + 8 * c16]) = b.k[i * KRP + r];
                wave_lds_sync();
                f16x8 ka[KS];
#pragma unroll
                for (int s = 0; s < KS; ++s) ka[s] = *reinterpret_cast<const f16x8*>(&K_s[wave][c16][32 * s + 8 * g4]);
#pragma unroll
                for (int s = 0; s < KS; ++s)
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[s], qf[s], acc, 0, 0, 0);
            } else {
#pragma unroll
                for (int s = 0; s < KS; ++s)
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(b.k[s], qf[s], acc, 0, 0, 0);
            }
            float x[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float sv = acc[i];
                if constexpr (SPLIT_Q) sv += row_rotate_down<GB>(sv);
                x[i] = kt + 4 * g4 + i < key_end ? sv * a.c : -INFINITY;
            }
            const float tm = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
            const float mn = fmaxf(m_run, tm);
            const float corr = fast_exp2(m_run - mn);
            m_run = mn;
            float p[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) p[i] = fast_exp2(x[i] - mn);
            l_run = l_run * corr + ((p[0] + p[1]) + (p[2] + p[3]));
            if (c16 < GB) {
#pragma unroll
                for (int i = 0; i < 4; ++i) P_s[wave][4 * g4 + i][c16] = p[i];
                C_s[wave][g4][c16] = corr;
            }
            wave_lds_sync();
            float cr[GB];
#pragma unroll
            for (int h = 0; h < GB; ++h) cr[h] = C_s[wave][g4][h];
#pragma unroll
            for (int h = 0; h < GB; ++h)
#pragma unroll
                for (int d = 0; d < DPL; ++d) o[h][d] *= cr[h];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float pv[GB];
#pragma unroll
                for (int h = 0; h < GB; ++h) pv[h] = P_s[wave][4 * g4 + i][h];
#pragma unroll
                for (int r = 0; r < VR; ++r)
#pragma unroll
                    for (int j = 0; j < VW; ++j) {
                        const float vv = raw_at<VW>(b.v[i][r], j);
#pragma unroll
                        for (int h = 0; h < GB; ++h) o[h][VW * r + j] = fmaf(pv[h], vv, o[h][VW * r + j]);
                    }
            }
            wave_lds_sync();  // this tile's P/corr reads are done before the next writes
            // Keep the P.V arithmetic here: without this the compiler sinks it
            // past the next prefetch, which then has to wait for every load.
#pragma unroll
            for (int h = 0; h < GB; ++h)
#pragma unroll
                for (int d = 0; d < DPL; ++d) asm volatile("" : "+v"(o[h][d]));
            asm volatile("" : "+v"(m_run), "+v"(l_run));
            if (t == tile_of(0)) LMX_DECODE_MARK(2);
        };

        if constexpr (PIPE) {
            // Rounds of DEPTH tiles while DEPTH more remain: compute a buffer,
            // refill it with the tile DEPTH ahead (the loop body has one shape
            // and no early exit, so its wait counts are exact).  Then the last
            // 1 .. 2 DEPTH - 1 tiles on uniform paths that load nothing past
            // the wave's end.
            int j = 0;
            for (; j + 2 * DEPTH - 1 < my_n; j += DEPTH) {
#pragma unroll
                for (int k = 0; k < DEPTH; ++k) {
                    compute_tile(tile_of(j + k), bufs[k]);
                    __builtin_amdgcn_sched_barrier(0);
                    load_tile(tile_of(j + DEPTH + k), bufs[k]);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            const int rest = my_n - j;
#pragma unroll
            for (int k = 0; k < DEPTH; ++k) {
                if (k < rest) {
                    compute_tile(tile_of(j + k), bufs[k]);
                    if (DEPTH + k < rest) {
                        __builtin_amdgcn_sched_barrier(0);
                        load_tile(tile_of(j + DEPTH + k), bufs[k]);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
            }
#pragma unroll
            for (int k = 0; k + 1 < DEPTH; ++k)
                if (DEPTH + k < rest) compute_tile(tile_of(j + DEPTH + k), bufs[k]);
        } else {
            for (int j = 0; j < my_n; ++j) {
                load_tile(tile_of(j), bufs[0]);
                compute_tile(tile_of(j), bufs[0]);
            }
        }

        LMX_DECODE_MARK(3);
        // Combine the wave's four group streams: M = max of the group maxima;
        // group g is weighted by exp2(m_g - M), in l and in o.
        float M = fmaxf(m_run, shfl_xor(m_run, 16));
        M = fmaxf(M, shfl_xor(M, 32));
        const float gsc = fast_exp2(m_run - M);
        float L = l_run * gsc;
        L += shfl_xor(L, 16);
        L += shfl_xor(L, 32);
        if (c16 < GB) C_s[wave][g4][c16] = gsc;
        wave_lds_sync();
        if constexpr (WPH == 1) {
            // The wave is its head's only one here: a reduce-scatter through
            // LDS (each group writes its weighted o, then lane (g4, c16)
            // sums head g4's dims over the four groups) and the wave stores
            // its result itself, with no workgroup barrier.
            __shared__ __attribute__((aligned(16))) float red_s[kWaves][4][GB][HD];
            __shared__ float lsum_s[kWaves][GB];
#pragma unroll
            for (int h = 0; h < GB; ++h) {
                const float sc = C_s[wave][g4][h];
#pragma unroll
                for (int r = 0; r < VR; ++r)
#pragma unroll
                    for (int j = 0; j < VW; ++j)
                        red_s[wave][g4][h][v_dim<HD>(c16, r, j)] = o[h][VW * r + j] * sc;
            }
            if (c16 < GB && g4 == 0) lsum_s[wave][c16] = L;
            wave_lds_sync();
#pragma unroll
            for (int h0g = 0; h0g < GB; h0g += 4) {
                const int h = h0g + g4;
                if (h < GB) {
                    const size_t row = (size_t)qi * a.H + h0 + h;
                    const float inv = 1.f / lsum_s[wave][h];
#pragma unroll
                    for (int r = 0; r < VR; ++r) {
                        const int d0 = v_dim<HD>(c16, r, 0);
                        float acc[VW];
#pragma unroll
                        for (int j = 0; j < VW; ++j) acc[j] = red_s[wave][0][h][d0 + j];
#pragma unroll
                        for (int g = 1; g < 4; ++g)
#pragma unroll
                            for (int j = 0; j < VW; ++j) acc[j] += red_s[wave][g][h][d0 + j];
                        float* dst = p_u == 1 ? a.out + row * HD + d0
                                              : a.part_o + (row * a.P + split) * HD + d0;
#pragma unroll
                        for (int j = 0; j < VW; j += 4) {
                            f32x4 y = p_u == 1 ? f32x4{acc[j] * inv, acc[j + 1] * inv, acc[j + 2] * inv,
                                                       acc[j + 3] * inv}
                                               : f32x4{acc[j], acc[j + 1], acc[j + 2], acc[j + 3]};
                            if (p_u == 1 && a.gate) y = gate_sigmoid4(y, a.gate + row * a.gate_stride + d0 + j);
                            *reinterpret_cast<f32x4*>(dst + j) = y;
                        }
                    }
                }
            }
            if (p_u > 1 && g4 == 0 && c16 < GB) {
                const size_t pidx = ((size_t)qi * a.H + h0 + c16) * a.P + split;
                a.part_ml[pidx * 2] = M;
                a.part_ml[pidx * 2 + 1] = L;
            }
        } else {
#pragma unroll
            for (int h = 0; h < GB; ++h) {
                const float sc = C_s[wave][g4][h];
#pragma unroll
                for (int d = 0; d < DPL; ++d) {
                    float x = o[h][d] * sc;
                    x += shfl_xor(x, 16);
                    x += shfl_xor(x, 32);
                    o[h][d] = x;
                }
            }
            if (g4 == 0) {
#pragma unroll
                for (int h = 0; h < GB; ++h)
#pragma unroll
                    for (int r = 0; r < VR; ++r)
#pragma unroll
                        for (int j = 0; j < VW; ++j) sm_o[wave][h][v_dim<HD>(c16, r, j)] = o[h][VW * r + j];
                if (c16 < GB) {
                    sm_m[wave][c16] = M;
                    sm_l[wave][c16] = L;
                }
            }
        }
    } else if constexpr (WPH > 1) {
        // A wave without tiles contributes nothing: weight exp2(-1e30 - M) = 0.
        // (With one wave per head every wave has a tile: t_begin < n_tiles.)
        if (c16 < GB && g4 == 0) {
            sm_m[wave][c16] = -1e30f;
            sm_l[wave][c16] = 0.f;
            for (int d = 0; d < HD; ++d) sm_o[wave][c16][d] = 0.f;
        }
    }
    if constexpr (WPH > 1) combine_waves();
    LMX_DECODE_MARK(4);
}

// ---- Many query heads on one kv head at head_dim 512 (Gemma 4's global
// layers: 16 query heads share each kv head) --------------------------------
//
// attn_decode_kernel does P.V on the VALU, one query head's dims per lane
// set, and at head_dim 512 holds at most four heads a wave: the 16 heads of
// a kv head then stream its rows four times and spend 268 M FMAs a 32k call
// on the VALU.  Here a workgroup serves all 16 heads of a kv head and split
// s of its tiles, and both products run on the matrix cores:
//
//   S^T [16 keys x 16 heads] = K Q^T on v_mfma_f32_16x16x32_f16: A = the K
//     tile (lane (key c16, group g4) holds dims 32 s + 8 g4 .. + 7), B = Q^T
//     (column c16 = head h0 + c16; an fp32 query's f16 residual is a second
//     column block whose result adds in place).  Lane (g4, c16) then holds
//     keys 4 g4 .. + 3 of head c16: the B operand layout of
//   O^T [16 dims x 16 heads] += V^T P^T on v_mfma_f32_16x16x16_f16: A = V^T,
//     4 keys of one dim a lane, read out of the wave's row-major V tile in
//     LDS with ds_read_b64_tr_b16 (lane a + 4 j addresses key 4 g4 + j, dims
//     16 db + 4 a .. + 3; lane c16 receives keys 4 g4 .. + 3 of dim
//     16 db + c16).
//
// The four waves take the head's 512 output dims in quarters and every tile
// of the split; each forms the same scores (the matrix pipe has room: 32 or
// 16 MFMAs a 32 KB tile), so m and l agree across them and no wave merge is
// needed.  A head's running max sits in the four lanes (g4 = 0..3) of its
// column; each lane sums its own keys' p, combined at the end.  Partials
// (p_u > 1) go to the same layout attn_merge_kernel<512> reads.
constexpr int kMhHeads = 16;  // query heads a workgroup (one MFMA column block)
#ifndef LMX_MH_DEPTH
#define LMX_MH_DEPTH 2
#endif
constexpr int kMhDepth = LMX_MH_DEPTH;  // tiles in flight a wave

template <typename QT, int MODE>
__global__ __launch_bounds__(kDecThreads) void attn_decode_mh_kernel(DecodeArgs a) {
    constexpr int HD = 512, KS = HD / 32;  // score MFMA k-steps
    constexpr int DW = HD / kWaves;        // output dims a wave owns
    constexpr int NDB = DW / 16;           // its 16-dim output blocks
    constexpr int VPAD = DW + 8;           // V_s row stride (halfs)
    constexpr bool SPLIT_Q = sizeof(QT) == 4;
    args_in_sgprs(a.q, a.out, a.gate, a.part_o, a.part_ml, a.q_stride, a.gate_stride, a.H, a.G, a.kv_dim, a.P,
                  a.tps, a.n_hblk, a.n_yg, a.window, a.c);
    if constexpr (MODE == kModeBatched)
        args_in_sgprs(a.k_ptrs, a.v_ptrs, a.ctx_lens, a.max_ctx);
    else
        args_in_sgprs(a.k, a.v, a.k_cur, a.v_cur, a.base_pos, a.n_tokens, a.bidi, a.w_magic, a.w_shift);
    LMX_DECODE_MARK(0);
    const int bid = blockIdx.x;
    const int split = bid % a.P;
    const int yg = (bid / a.P) % a.n_yg;
    const int qi = bid / (a.P * a.n_yg);
    const int kvh = yg / a.n_hblk;
    const int h0 = kvh * a.G + (yg - kvh * a.n_hblk) * kMhHeads;

    int lo, hi;
    unit_range<MODE>(a, qi, lo, hi);
    const int n_tiles = (hi - lo + kTile) / kTile;
    const int t_begin = split * a.tps;
    if (t_begin >= n_tiles) return;  // uniform: this unit needs fewer splits
    const int t_end = min(t_begin + a.tps, n_tiles);
    const int p_u = (n_tiles + a.tps - 1) / a.tps;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g4 = lane >> 4, c16 = lane & 15;

    const f16 *kc, *vc;
    int cur_begin = INT_MAX;
    if constexpr (MODE == kModeBatched) {
        kc = a.k_ptrs[qi];
        vc = a.v_ptrs[qi];
    } else {
        kc = a.k;
        vc = a.v;
        if (MODE == kModeGeneral && a.k_cur) cur_begin = a.base_pos;
    }
    auto row_ptr = [&](const f16* cache, const f16* cur, int p) -> const f16* {
        if constexpr (MODE == kModeLinear) {
            return cache + (size_t)p * a.kv_dim + kvh * HD;
        } else {
            int s = p;
            if (a.window) {
                const uint32_t qd = (uint32_t)(((uint64_t)(uint32_t)p * a.w_magic) >> a.w_shift);
                s = p - (int)qd * a.window;
            }
            const f16* rc = cache + (size_t)s * a.kv_dim;
            const f16* ru = cur + (size_t)(p - a.base_pos) * a.kv_dim;
            return (p >= cur_begin ? ru : rc) + kvh * HD;
        }
    };

    // Each wave holds and loads its quarter of the head's dims: Q^T k-steps
    // (32 dims each) KQ w .. KQ w + KQ - 1, the K tile's same dims, and V's
    // dims DW w .. + DW - 1.  The partial scores of the four quarters are
    // summed through LDS; with 8 KB a tile a wave, MH_DEPTH tiles are in flight
    // (the first form, every wave loading the whole K tile with one tile
    // ahead, ran at 2.2 TB/s).
    constexpr int KQ = KS / kWaves;  // k-steps a wave owns
    struct MhTile {
        f16x8 k[KQ];  // key c16 of the tile, dims 32 (KQ w + s) + 8 g4 .. + 7
        f16x8 v[4];   // key 4 i + g4, dims DW w + 8 c16 .. + 7
    };
    // Rows past hi are clamped to hi (their scores are masked).
    auto load_tile = [&](int t, MhTile& b) {
        const int kt = lo + kTile * t;
        const f16* krow = row_ptr(kc, a.k_cur, min(kt + c16, hi)) + DW * wave;
#pragma unroll
        for (int s = 0; s < KQ; ++s) b.k[s] = ld_stream8<true>(krow + 32 * s + 8 * g4);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            b.v[i] = ld_stream8<true>(row_ptr(vc, a.v_cur, min(kt + 4 * i + g4, hi)) + DW * wave + 8 * c16);
    };

    // Q^T columns: head h0 + c16, this wave's dims (f16, and an fp32 query's
    // f16 residual).  The raw loads go out first, then the first tiles', and
    // only then the conversion waits.
    using QRaw = typename std::conditional<SPLIT_Q, f32x4, f16x8>::type;
    QRaw qraw[KQ][SPLIT_Q ? 2 : 1];
    {
        const size_t qo = ((size_t)qi * a.H + h0 + c16) * a.q_stride + DW * wave + 8 * g4;
#pragma unroll
        for (int s = 0; s < KQ; ++s) {
            if constexpr (SPLIT_Q) {
                const float* qp = reinterpret_cast<const float*>(a.q) + qo + 32 * s;
                qraw[s][0] = *reinterpret_cast<const f32x4*>(qp);
                qraw[s][SPLIT_Q ? 1 : 0] = *reinterpret_cast<const f32x4*>(qp + 4);
            } else {
                qraw[s][0] = *reinterpret_cast<const f16x8*>(reinterpret_cast<const f16*>(a.q) + qo + 32 * s);
            }
        }
    }
    const int my_n = t_end - t_begin;  // every wave takes every tile of the split
    MhTile bufs[kMhDepth];
#pragma unroll
    for (int k = 0; k < kMhDepth; ++k) load_tile(t_begin + min(k, my_n - 1), bufs[k]);
    __builtin_amdgcn_sched_barrier(0);
    f16x8 qh[KQ], ql[SPLIT_Q ? KQ : 1];
#pragma unroll
    for (int s = 0; s < KQ; ++s) {
        if constexpr (SPLIT_Q) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float x = qraw[s][j / 4][j % 4];
                const f16 h = (f16)x;
                qh[s][j] = h;
                ql[s][j] = (f16)(x - (float)h);
            }
        } else {
            qh[s] = qraw[s][0];
        }
    }
    LMX_DECODE_MARK(1);

    __shared__ __attribute__((aligned(16))) f16 V_s[kWaves][kTile][VPAD];
    // Partial scores, two sets (tile parity): [set][wave][hi / lo block][lane]
    __shared__ __attribute__((aligned(16))) f32x4 S_s[2][kWaves][2][64];
    float m_run = -1e30f, l_run = 0.f;  // head c16: running max (log2 units); this lane's keys' sum
    f32x4 o[NDB];                       // O^T block db: dims DW wave + 16 db + 4 g4 + i, head c16
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int t, const MhTile& b) {
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<f16x8*>(&V_s[wave][4 * i + g4][8 * c16]) = b.v[i];
        f32x4 sh = {0.f, 0.f, 0.f, 0.f}, sl = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KQ; ++s) {
            sh = __builtin_amdgcn_mfma_f32_16x16x32_f16(b.k[s], qh[s], sh, 0, 0, 0);
            if constexpr (SPLIT_Q) sl = __builtin_amdgcn_mfma_f32_16x16x32_f16(b.k[s], ql[s], sl, 0, 0, 0);
        }
        const int set = t & 1;
        S_s[set][wave][0][lane] = sh;
        if constexpr (SPLIT_Q) S_s[set][wave][1][lane] = sl;
        // The set written here was last read two tiles ago, before the
        // previous barrier; this barrier publishes it.
        __syncthreads();
        f32x4 sc = {0.f, 0.f, 0.f, 0.f};  // the same order in every wave: the same sums
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            sc += S_s[set][w][0][lane];
            if constexpr (SPLIT_Q) sc += S_s[set][w][1][lane];
        }
        const int kt = lo + kTile * t;
        float x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = kt + 4 * g4 + i <= hi ? sc[i] * a.c : -INFINITY;
        float tm = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
        tm = fmaxf(tm, shfl_xor(tm, 16));
        tm = fmaxf(tm, shfl_xor(tm, 32));
        const float mn = fmaxf(m_run, tm);
        const float corr = fast_exp2(m_run - mn);
        m_run = mn;
        f16x4 pf;
        float ps = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pf[i] = (f16)fast_exp2(x[i] - mn);
            ps += (float)pf[i];
        }
        l_run = l_run * corr + ps;
        typedef __fp16 tr_h4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
        typedef __attribute__((address_space(3))) tr_h4 lds_h4;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            const f16x4 va = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                (lds_h4*)&V_s[wave][4 * g4 + (c16 >> 2)][16 * db + 4 * (c16 & 3)]));
            o[db] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pf, o[db] * corr, 0, 0, 0);
        }
        wave_lds_sync();  // the V reads are done before the next tile's writes
        if (t == t_begin) LMX_DECODE_MARK(2);
    };

    // kMhDepth tiles in flight: a buffer is refilled with the tile kMhDepth
    // ahead right after it is computed.  Rounds of kMhDepth while 2 kMhDepth
    // - 1 tiles remain, then the last ones on uniform paths that load nothing
    // past the split (every wave has the same count, so the barriers match).
    int j = 0;
    for (; j + 2 * kMhDepth - 1 < my_n; j += kMhDepth) {
#pragma unroll
        for (int k = 0; k < kMhDepth; ++k) {
            compute(t_begin + j + k, bufs[k]);
            __builtin_amdgcn_sched_barrier(0);
            load_tile(t_begin + j + kMhDepth + k, bufs[k]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    const int rest = my_n - j;
#pragma unroll
    for (int k = 0; k < kMhDepth; ++k) {
        if (k < rest) {
            compute(t_begin + j + k, bufs[k]);
            if (kMhDepth + k < rest) {
                __builtin_amdgcn_sched_barrier(0);
                load_tile(t_begin + j + kMhDepth + k, bufs[k]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
#pragma unroll
    for (int k = 0; k + 1 < kMhDepth; ++k)
        if (kMhDepth + k < rest) compute(t_begin + j + kMhDepth + k, bufs[k]);

    LMX_DECODE_MARK(3);
    // The head's sum over its four lanes; every wave holds the same m and L.
    float L = l_run + shfl_xor(l_run, 16);
    L += shfl_xor(L, 32);
    const size_t row = (size_t)qi * a.H + h0 + c16;
    if (p_u == 1) {
        const float inv = 1.f / L;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            const int d = DW * wave + 16 * db + 4 * g4;
            f32x4 y = o[db] * inv;
            if (a.gate) y = gate_sigmoid4(y, a.gate + row * a.gate_stride + d);
            *reinterpret_cast<f32x4*>(a.out + row * HD + d) = y;
        }
    } else {
        const size_t pidx = row * a.P + split;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
            *reinterpret_cast<f32x4*>(a.part_o + pidx * HD + DW * wave + 16 * db + 4 * g4) = o[db];
        if (wave == 0 && g4 == 0) *reinterpret_cast<f32x2*>(a.part_ml + pidx * 2) = f32x2{m_run, L};
    }
    LMX_DECODE_MARK(4);
}

struct DecodePlan {
    int P, tps, n_hblk, gb, hw;
    int P_ws;          // splits the workspace is sized for (>= P)
    int n_main, n_yg;
    int n_merge, m_parts;
    bool krows;                // head_dim 128 / 256: K row-major through LDS (attn_decode_kernel's KR)
    bool mh;                   // head_dim 512, 16 query heads a kv head: attn_decode_mh_kernel
    size_t ml_bytes, o_bytes;  // what this launch uses
    size_t ws_bytes;           // what the workspace query reports for this shape
    size_t total() const { return ml_bytes + o_bytes; }
};

template <typename QT, int MODE, int HW>
inline lmx_status launch_decode_hw(const DecodeArgs& a, int hd, int gb, bool krows, dim3 grid, hipStream_t st) {
#define LMX_DEC_CASE(HDV, GBV)                                                                        \
    if (hd == HDV && gb == GBV) {                                                                     \
        if constexpr (HDV == 128 || HDV == 256) {                                                     \
            if (krows) {                                                                              \
                hipLaunchKernelGGL((attn_decode_kernel<QT, HDV, GBV, HW, MODE, true>), grid,          \
                                   dim3(kDecThreads), 0, st, a);                                      \
                return LMX_OK;                                                                        \
            }                                                                                         \
        }                                                                                             \
        hipLaunchKernelGGL((attn_decode_kernel<QT, HDV, GBV, HW, MODE, false>), grid, dim3(kDecThreads), \
                           0, st, a);                                                                 \
        return LMX_OK;                                                                                \
    }
    LMX_DEC_CASE(64, 1) LMX_DEC_CASE(64, 2) LMX_DEC_CASE(64, 3) LMX_DEC_CASE(64, 4)
    LMX_DEC_CASE(64, 5) LMX_DEC_CASE(64, 6) LMX_DEC_CASE(64, 7) LMX_DEC_CASE(64, 8)
    LMX_DEC_CASE(128, 1) LMX_DEC_CASE(128, 2) LMX_DEC_CASE(128, 3) LMX_DEC_CASE(128, 4)
    LMX_DEC_CASE(128, 5) LMX_DEC_CASE(128, 6)
    LMX_DEC_CASE(256, 1) LMX_DEC_CASE(256, 2)
    LMX_DEC_CASE(512, 1) LMX_DEC_CASE(512, 2) LMX_DEC_CASE(512, 4)
#undef LMX_DEC_CASE
    return LMX_E_UNSUPPORTED;
}

template <typename QT, int MODE>
inline lmx_status launch_decode(const DecodeArgs& a, int hd, int gb, int hw, bool krows, dim3 grid,
                                hipStream_t st) {
    switch (hw) {
        case 4: return launch_decode_hw<QT, MODE, 4>(a, hd, gb, krows, grid, st);
        case 2: return launch_decode_hw<QT, MODE, 2>(a, hd, gb, krows, grid, st);
        default: return launch_decode_hw<QT, MODE, 1>(a, hd, gb, krows, grid, st);
    }
}

template <int MODE>
inline lmx_status launch_merge(const DecodeArgs& a, int hd, dim3 grid, hipStream_t st) {
    switch (hd) {
        case 64: hipLaunchKernelGGL((attn_merge_kernel<64, MODE>), grid, dim3(kDecThreads), 0, st, a); break;
        case 128: hipLaunchKernelGGL((attn_merge_kernel<128, MODE>), grid, dim3(kDecThreads), 0, st, a); break;
        case 256: hipLaunchKernelGGL((attn_merge_kernel<256, MODE>), grid, dim3(kDecThreads), 0, st, a); break;
        case 512: hipLaunchKernelGGL((attn_merge_kernel<512, MODE>), grid, dim3(kDecThreads), 0, st, a); break;
        default: return LMX_E_UNSUPPORTED;
    }
    return LMX_OK;
}

// Enqueue the split kernel and, with more than one split, the merge kernel.
template <typename QT, int MODE>
lmx_status launch_mode(const DecodeArgs& a, const DecodePlan& pl, int hd, hipStream_t st) {
    lmx_status s = LMX_OK;
    if (pl.mh)
        hipLaunchKernelGGL((attn_decode_mh_kernel<QT, MODE>), dim3((unsigned)pl.n_main), dim3(kDecThreads), 0, st, a);
    else
        s = launch_decode<QT, MODE>(a, hd, pl.gb, pl.hw, pl.krows, dim3((unsigned)pl.n_main), st);
    if (s != LMX_OK || pl.P == 1) return s;
    return launch_merge<MODE>(a, hd, dim3((unsigned)pl.n_merge), st);
}

#define LMX_DECODE_MODES(X)        \
    X(float, kModeLinear)          \
    X(float, kModeGeneral)         \
    X(float, kModeBatched)         \
    X(f16, kModeLinear)            \
    X(f16, kModeGeneral)           \
    X(f16, kModeBatched)

#define LMX_DECODE_EXTERN(QT, MODE) \
    extern template lmx_status launch_mode<QT, MODE>(const DecodeArgs&, const DecodePlan&, int, hipStream_t);
LMX_DECODE_MODES(LMX_DECODE_EXTERN)
#undef LMX_DECODE_EXTERN

}  // namespace lmx
