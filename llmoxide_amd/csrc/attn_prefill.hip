// Tiled attention for long batches (prefill) on gfx950 MFMA.
//
// Replaces, for n_tokens large, the reference's scores_pass / softmax_pass /
// weighted_v (attn.wgsl:84-232), which materialize an f32 [t, H, max_vis]
// scores buffer in HBM.  Here scores stay in registers:
//
//   S^T = K Q^T   v_mfma_f32_32x32x16_f16, A = K rows from LDS, B = Q rows
//                 held in registers for the whole key loop
//   online softmax in fp32 (exp2; scale*log2e applied to the fp32 scores of
//                 an f16 query, folded into an fp32 query), P rounded to f16
//   O^T += V^T P^T  A = V^T from a transposed LDS tile, B = P straight from the
//                 S^T accumulators (no shuffle: computing the transpose makes
//                 each lane own one query column, so softmax is mostly in-lane)
//
// Three kernels share these tiles.  attn_prefill_kernel: workgroup = 4 waves x
// 32 query rows, of one query head or of 2-4 heads that share a kv head
// (head_dim >= 256), two workgroups per CU below head_dim 256.  The ping-pong
// kernel (head_dim 128, long batches): 8 waves x 32 rows, one workgroup per
// CU, the two waves of each SIMD kept half a tile apart so one's MFMAs run
// beside the other's softmax.  The key-halves kernel (short batches): 64
// query rows, two wave pairs on the two halves of the key range, merged in
// LDS.  K/V tiles of 64 keys are staged in LDS.  Key
// tiles outside a wave's visible range are skipped (causal / window), tiles
// inside every query's range skip the mask.  Workgroups are ordered so each
// XCD owns whole kv heads (its L2 serves the G query heads that share them)
// and heavy causal tiles start first.
#include <algorithm>
#include <climits>
#include <cstdlib>
#include <cstring>

#include "common.hpp"



namespace lmx {

struct PrefillArgs {
    const void* q;
    const f16* k;
    const f16* v;
    const f16* k_cur;
    const f16* v_cur;
    float* out;
    const float* gate;  // NULL, or the output gate: out *= sigmoid(gate[row * gate_stride + d])
    int q_stride, gate_stride;
    int H, Hkv, G, kv_dim;
    int base_pos, window, n_tokens, bidi;
    int n_qtiles;
    int gp;  // attn_prefill_kernel: query heads per workgroup (1, 2 or 4, dividing G)
    uint32_t w_magic;  // p % window == ring_slot(p, window, w_magic, w_shift)
    int w_shift;
    float c;  // scale * log2(e)
    // Key-range split (attn_prefill_kernel only): n_split > 1 writes each
    // split's unnormalized o and its (m, l) to part_o / part_ml for
    // prefill_merge_kernel.
    int n_split;
    float* part_o;   // [n_split][t][H][hd]
    float* part_ml;  // [n_split][t][H][2]
};

constexpr int kPfBM = 128;  // query rows per workgroup
constexpr int kPfCus = 256;  // compute units of the target (MI355X)
// Keys per LDS tile: 64, or 32 at head_dim >= 256 (the register prefetch of
// the next tile and the o accumulators share one register file).
template <int HD>
constexpr int pf_bn() { return HD >= 256 ? 32 : 64; }
// Wave pairs at head_dim 512: a wave cannot hold a 32-row block's Q and its
// 32 x 512 fp32 output in registers, so two waves share each block, one per
// half of the head's dims.  Each holds its half of Q and of the output (the
// register budget of head_dim 256), forms the partial S over its 256 dims,
// and the two partials are summed through LDS; both waves then hold the
// same scores (a + b = b + a in IEEE arithmetic), run the same softmax, and
// accumulate P V for their own half.  The MFMA work is that of one pass.
template <int HD>
constexpr bool pf_pair() { return HD >= 512; }
constexpr float kRescaleSlack = 8.f;  // log2 units a running max may lag by

// attn.wgsl:52-66
__device__ __forceinline__ int vis_lo(int pos, int w) { return (w && pos + 1 > w) ? pos + 1 - w : 0; }
__device__ __forceinline__ int vis_hi(int pos, int w, int bidi, int end) {
    if (!bidi) return pos;
    return w ? min(end, pos + w - 1) : end;
}

// S^T - mb = K Q^T - mb for KB 32-key blocks of a K tile in LDS (rows of
// KPAD halfs), Q^T in registers as the B operand.  The K operand reads run
// QK_DEPTH ahead of the MFMAs (the compiler's own schedule kept one or two
// in flight, so every MFMA waited out most of an LDS round trip); the
// (k-step, block) order alternates the KB accumulator chains.  Depth 4 at
// head_dim <= 128 (6 spills in the 128-row kernel), QK_DEPTH_HD256 at 256,
// where one wave per SIMD has the registers (measured: depth 4 +2-3% at
// S = 8192, +7% on Gemma hd 256 global 4k; depth 6 a further +2-3% there),
// and 2 at head_dim 512, whose Q alone takes 128 registers.
#ifndef LMX_QK_DEPTH_HD256
#define LMX_QK_DEPTH_HD256 8
#endif
template <int HD>
constexpr int qk_depth() { return HD >= 512 ? 2 : (HD >= 256 ? LMX_QK_DEPTH_HD256 : 4); }
// The wave pairs of head_dim 512 hold twice the K/V prefetch of head_dim 256
// in registers: shallower operand rings keep them out of scratch.
#ifndef LMX_PAIR_QK_DEPTH
#define LMX_PAIR_QK_DEPTH 2
#endif
#ifndef LMX_PAIR_PV_DEPTH
#define LMX_PAIR_PV_DEPTH 1
#endif
constexpr int kPairQkDepth = LMX_PAIR_QK_DEPTH;
constexpr int kPairPvDepth = LMX_PAIR_PV_DEPTH;
//
// EXACT: Q holds the caller's f16 values and the scores are scaled by
// c = scale * log2(e) in fp32 after the MFMAs (one FMA per score).  Else c
// was folded into Q before its one f16 rounding (an fp32 query) and the
// accumulators start at -mb.  Folding c into a query that is already f16
// would round it twice: at Gemma's scale 1.0 with unit-RMS heads of 256 the
// second rounding moves a score by ~2^-12 * c * sqrt(hd) ~ 6e-3 (log2
// units, one sigma), enough to shift the output past 2e-3.
//
// QLO (fp32 queries): the query row x, times c and a power of two 2^S chosen
// per row (its largest |x c 2^S| in [2^14, 2^15)), is carried as its f16
// rounding hi (qf) plus the f16 residual lo = f16(x c 2^S - hi), and every K
// operand also meets lo in a second MFMA; EXACT then scales the sums by
// 2^-S.  A score is exact to about 2^-22 of its products' sum instead of
// 2^-12 (at scale 1.0 on RMS-normed heads, Gemma's and the vision tower's,
// one rounding of q moves scores by ~1e-2 in log2 units).  The row scaling
// keeps hi and the residuals of all but tiny elements in f16's normal range,
// where they keep their full 11 bits.  ql(ks) returns the residual's fragment
// of k-step ks (from LDS, or recomputed from the fp32 query in memory where
// no LDS is left).
struct NoQlo {
    __device__ f16x8 operator()(int) const { return f16x8{}; }
};
template <int HD, int KB, int KPAD, bool EXACT, bool QLO = false, typename QL = NoQlo, int DEP = qk_depth<HD>()>
__device__ __forceinline__ void qk_tile(const f16* Ks, const f16x8 (&qf)[HD / 16], f32x16 (&s)[KB], float mb,
                                        float c, int l32, int hh, const QL& ql = QL{}) {
    constexpr int KSTEPS = HD / 16, NQ = KSTEPS * KB;
    constexpr int D = DEP < NQ ? DEP : NQ;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) s[kb][i] = EXACT ? 0.f : -mb;
    auto rd = [&](int q) {
        const int ks = q / KB, kb = q % KB;
        return *reinterpret_cast<const f16x8*>(&Ks[(kb * 32 + l32) * KPAD + 8 * hh + ks * 16]);
    };
    f16x8 ka[NQ];
    f16x8 qlo = {};
#pragma unroll
    for (int q = 0; q < D; ++q) ka[q] = rd(q);
    __builtin_amdgcn_sched_group_barrier(0x100, D, 0);  // the first D reads
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        if constexpr (QLO) {
            if (q % KB == 0) qlo = ql(q / KB);
        }
        if (q + D < NQ) ka[q + D] = rd(q + D);
        s[q % KB] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[q], qf[q / KB], s[q % KB], 0, 0, 0);
        if constexpr (QLO) s[q % KB] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[q], qlo, s[q % KB], 0, 0, 0);
        if (q + D < NQ) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one read
        __builtin_amdgcn_sched_group_barrier(0x008, QLO ? 2 : 1, 0);        // its MFMAs
    }
    if constexpr (EXACT) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) s[kb][i] = fmaf(s[kb][i], c, -mb);
    }
}

// Q fragments as values defined here, not the registers of their loads (an
// f16 query's conversions fold away): otherwise the waitcnt pass counts Q's
// loads as possibly pending inside the key loop and puts vmcnt(n) waits
// between the score MFMAs, which drain the K/V prefetch of later tiles.
template <int N>
__device__ __forceinline__ void settle_q(f16x8 (&qf)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("" : "+v"(qf[i]));
}

// s_waitcnt vmcnt(0) as an instruction the compiler's waitcnt pass sees
// (inline assembly it does not): every load issued before it is complete.
__device__ __forceinline__ void drain_loads() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// A raw buffer resource over p (dword 3 = 0x00020000: 32-bit data format, the
// form raw buffer loads take on gfx9 parts) with 2^31 - 1 bytes of range,
// which the rows of one K/V tile never leave.  p must be wave-uniform: it is
// moved to scalar registers first (readfirstlane), since a resource built in
// vector registers makes the compiler wrap every load in a waterfall loop.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    void* q = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(q, 0, 0x7fffffff, 0x00020000);
}

// LIN: every key row p lives at cache row p (no k_cur rows, no ring wrap),
// the common causal case; its addressing is compiled without the general
// path's branches (which cost the main loop 3-8% in registers and schedule).
template <typename QT, int HD, bool LIN>
__global__ __launch_bounds__(256, HD > 128 ? 1 : 2) void attn_prefill_kernel(PrefillArgs a) {
    constexpr bool kExact = sizeof(QT) == 2;  // f16 queries: scale applied in fp32 (qk_tile)
    constexpr int BN = pf_bn<HD>();
    constexpr bool kPair = pf_pair<HD>();
    constexpr int QD = kPair ? HD / 2 : HD;  // Q dims a wave holds (its half, kPair)
    constexpr int HDV = QD;          // output dims a wave accumulates
    constexpr int KB = BN / 32;      // 32-key MFMA blocks per tile
    constexpr int PST = BN / 16;     // 16-key P.V k-steps per tile
    constexpr int KSTEPS = QD / 16;  // MFMA k-steps over the wave's dims
    constexpr int NB = HDV / 32;     // 32-dim output blocks
    constexpr int KPAD = HD + 8;     // K_s row stride (halfs)
    constexpr int VPAD = BN + 4;     // Vt_s row stride (halfs), 8-byte aligned rows
    __shared__ __attribute__((aligned(16))) f16 K_s[2 * BN * KPAD];   // two stages
    __shared__ __attribute__((aligned(16))) f16 Vt_s[2 * HD * VPAD];
    // kPair: each wave's partial scores, 16 floats a lane as four f32x4
    // planes of 64 lanes (conflict-free 16-byte accesses)
    __shared__ __attribute__((aligned(16))) float X_s[kPair ? 4 * 16 * 64 : 4];
    // fp32 queries: the residual of q*c after its f16 rounding, one padded row
    // per query (the stride spreads a read's 32 rows over the banks as K_s's
    // does); at head_dim 512 the LDS is full and it is recomputed instead.
    constexpr bool kQlo = !kExact;
    constexpr bool kQloLds = kQlo && HD <= 256;
    constexpr int QLPAD = HD + 8;
    __shared__ __attribute__((aligned(16))) f16 QL_s[kQloLds ? 4 * 32 * QLPAD : 8];

    // ---- which (heads, query tile, key split) this workgroup owns.  The gp
    // query heads of a workgroup share kv head kvh; each takes 4 / gp waves,
    // i.e. 128 / gp query rows.  Fewer rows per head narrow the key range a
    // workgroup spans (a window's or the causal diagonal's spread) at the
    // same MFMA work per K/V tile.
    const int nblk = gridDim.x;
    const int logical = xcd_remap(blockIdx.x, nblk);
    const int n_split = a.n_split;
    const int gp = a.gp, hgroups = a.G / gp;
    const int per_kvh = a.n_qtiles * hgroups * n_split;
    const int kvh = logical / per_kvh;
    const int rem = logical - kvh * per_kvh;
    // Query tiles heaviest first (causal work grows with qt).  When the whole
    // grid is resident at once (two workgroups per CU), the second half is
    // walked lightest first, so the two workgroups a CU receives pair a heavy
    // tile with a light one instead of two of nearly the same weight.
    const int pos = rem / (hgroups * n_split);
    const int half = (a.n_qtiles + 1) / 2;
    const bool fold = HD <= 128 && nblk <= 2 * kPfCus;
    const int qt = (fold && pos >= half) ? pos - half : a.n_qtiles - 1 - pos;
    const int rem2 = rem % (hgroups * n_split);
    const int sp = rem2 % n_split;

    // wave: uniform by construction (readfirstlane), so the branches and loop
    // bounds it feeds are wave-uniform to the compiler too, and the tile
    // pointers derived from them stay scalar (no waterfall loops around
    // buffer loads)
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, hh = lane >> 5;
    // kPair: waves w and w ^ 2 share a 32-row block, dims [dh * QD, + QD)
    // each; otherwise every wave has its own block of all the dims.
    const int dh = kPair ? wave >> 1 : 0;
    const int wr = kPair ? wave & 1 : wave;  // the wave's row block
    const int wph = (kPair ? 2 : 4) / gp;    // row blocks per query head
    const int bm = 32 * wph;                 // query rows per head
    const int h = kvh * a.G + (rem2 / n_split) * gp + wr / wph;  // this wave's head
    const int t = a.n_tokens, base = a.base_pos, w = a.window;
    const int end = base + t - 1;
    const int q0 = qt * bm;
    const int qw0 = q0 + (wr % wph) * 32;

    // ---- this lane's query (column l32 of the wave's S^T tiles)
    const int qrow = qw0 + l32;
    const bool qvalid = qrow < t;
    const int qpos = base + qrow;
    const int my_lo = qvalid ? vis_lo(qpos, w) : 1;
    const int my_hi = qvalid ? vis_hi(qpos, w, a.bidi, end) : 0;

    // Q as the B operand: lane holds Q[qrow][ks*16 + 8*hh + j], j < 8.  An fp32
    // query has c = scale * log2(e) folded in before its f16 rounding, and its
    // residual is the second operand (kQlo); an f16 query is used as given and
    // qk_tile scales its scores.
    f16x8 qf[KSTEPS];
    const size_t qoff = ((size_t)(qvalid ? qrow : 0) * a.H + h) * a.q_stride + dh * QD + 8 * hh;
    const float* qrow32 = reinterpret_cast<const float*>(a.q) + qoff;
    f16* ql_row = &QL_s[kQloLds ? (wave * 32 + l32) * QLPAD + 8 * hh : 0];
    // fp32 queries: c 2^S folded into Q (the row's largest |x c 2^S| in
    // [2^14, 2^15); 2^S = 1 for an all-zero or non-finite row), and the
    // scores scaled back by c_sc = 2^-S; f16 queries: Q as given, c_sc = c.
    float qs = 1.f, c_sc = a.c;
    if constexpr (kQlo) {
        float m = 0.f;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            const f32x4 x0 = *reinterpret_cast<const f32x4*>(qrow32 + ks * 16);
            const f32x4 x1 = *reinterpret_cast<const f32x4*>(qrow32 + ks * 16 + 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) m = fmaxf(m, fmaxf(fabsf(x0[j]), fabsf(x1[j])));
        }
        m = fmaxf(m, shfl_xor(m, 32)) * a.c;  // the row's two halves
        const int S = (m > 0.f && m <= 3.402823466e38f) ? 15 - __builtin_amdgcn_frexp_expf(m) : 0;
        qs = __builtin_amdgcn_ldexpf(1.f, S);
        c_sc = __builtin_amdgcn_ldexpf(1.f, -S);
    }
    const float qc = a.c * qs;  // fp32 queries: x c 2^S
    {
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            float x[8];
            if constexpr (sizeof(QT) == 2) {
                const f16x8 q8 = *reinterpret_cast<const f16x8*>(reinterpret_cast<const f16*>(a.q) + qoff + ks * 16);
#pragma unroll
                for (int j = 0; j < 8; ++j) x[j] = (float)q8[j];
            } else {
                const f32x4 x0 = *reinterpret_cast<const f32x4*>(qrow32 + ks * 16);
                const f32x4 x1 = *reinterpret_cast<const f32x4*>(qrow32 + ks * 16 + 4);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    x[j] = x0[j];
                    x[4 + j] = x1[j];
                }
            }
            if constexpr (kExact) {
#pragma unroll
                for (int j = 0; j < 8; ++j) qf[ks][j] = (f16)x[j];
            } else {
                // y = x c 2^S once, and the residual taken against the very
                // registers the MFMA reads: with contraction on, the compiler
                // otherwise forms the residual's hi as one fused
                // multiply-convert (one rounding) and the MFMA operand's as
                // multiply then convert (two), which differ by an f16 ulp
                // where the fp32 product is a tie.
                float y[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    y[j] = x[j] * qc;
                    asm volatile("" : "+v"(y[j]));
                    qf[ks][j] = (f16)y[j];
                }
                asm volatile("" : "+v"(qf[ks]));
                if constexpr (kQloLds) {
                    f16x8 lo;
#pragma unroll
                    for (int j = 0; j < 8; ++j) lo[j] = (f16)(y[j] - (float)qf[ks][j]);
                    *reinterpret_cast<f16x8*>(ql_row + ks * 16) = lo;
                }
            }
        }
        settle_q(qf);
    }
    // The residual's fragment of k-step ks (read after the first barrier of
    // the key loop, which orders the stores above before it).
    auto ql = [&](int ks) -> f16x8 {
        if constexpr (kQloLds) {
            return *reinterpret_cast<const f16x8*>(ql_row + ks * 16);
        } else if constexpr (kQlo) {
            const f32x4 x0 = *reinterpret_cast<const f32x4*>(qrow32 + ks * 16);
            const f32x4 x1 = *reinterpret_cast<const f32x4*>(qrow32 + ks * 16 + 4);
            f16x8 lo;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                lo[j] = (f16)(x0[j] * qc - (float)qf[ks][j]);
                lo[4 + j] = (f16)(x1[j] * qc - (float)qf[ks][4 + j]);
            }
            return lo;
        } else {
            return f16x8{};
        }
    };

    // ---- key ranges: the workgroup's, and this wave's
    const int q_last = min(q0 + bm, t) - 1;
    const int wg_lo = vis_lo(base + q0, w);
    const int wg_hi = vis_hi(base + q_last, w, a.bidi, end);
    const int wq_last = min(qw0 + 31, t - 1);
    const bool wave_live = qw0 < t;
    const int wv_lo = wave_live ? vis_lo(base + qw0, w) : 1;                    // smallest lo
    const int wv_hi = wave_live ? vis_hi(base + wq_last, w, a.bidi, end) : 0;  // largest hi
    const int wv_lo_max = wave_live ? vis_lo(base + wq_last, w) : 0;          // largest lo
    const int wv_hi_min = wave_live ? vis_hi(base + qw0, w, a.bidi, end) : -1; // smallest hi

    const int cur_begin = (!LIN && a.k_cur) ? base : INT_MAX;

    float m_run = -1e30f, l_run = 0.f;
    f32x16 o[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[nb][i] = 0.f;

    // ---- K/V tiles: global -> registers (the next tile's loads are in
    // flight while the current tile is computed) -> one of two LDS stages.
    // Rows outside [wg_lo, wg_hi] are zero.  V is stored transposed; its
    // copy gives consecutive lanes consecutive 4-key groups (kg) of one 8-dim
    // chunk (dc), so the 8-byte transposed stores of 16 lanes fill all 32
    // banks once.  Consecutive dims would put lanes 8 rows apart, on two
    // banks (the row stride is 16 banks mod 32).
    constexpr int KCH = HD / 8;                   // 16-byte chunks per key row
    constexpr int KCHV = HD / 8;                  // 16-byte chunks of a V row
    constexpr int KPT = BN * KCH / 256;           // K chunks per thread
    constexpr int VPT = (KCHV * (BN / 4) + 255) / 256;  // V 4-key groups per thread
    static_assert(BN * KCH % 256 == 0, "K tile split");
    f16x8 rk[KPT];
    f16x8 rv[VPT][4];
    // kBufFetch: the fast path's per-thread byte offsets from a tile's first
    // row (thread tid takes K chunk tid % KCH of row tid / KCH, and V dims
    // 8 (tid / (BN / 4)) of rows 4 (tid % (BN / 4)) + u; each later load adds
    // a whole number of rows or chunks)
    constexpr bool kBufFetch = true;
    static_assert(256 % KCH == 0 && 256 % (BN / 4) == 0, "uniform load strides");
    const int k_voff = (tid / KCH) * a.kv_dim * 2 + (tid % KCH) * 16;
    const int v_voff = 4 * (tid % (BN / 4)) * a.kv_dim * 2 + (tid / (BN / 4)) * 16;
    // Row of position p: a k_cur row for p >= cur_begin, else cache slot
    // p % w (a multiply-high, not a division).
    auto row_src = [&](const f16* cache, const f16* cur, int p) -> const f16* {
        if constexpr (LIN) return cache + (size_t)p * a.kv_dim;
        if (p >= cur_begin) return cur + (size_t)(p - base) * a.kv_dim;
        const int sl = w ? ring_slot(p, w, a.w_magic, a.w_shift) : p;
        return cache + (size_t)sl * a.kv_dim;
    };
    // Fast path for a tile whose rows are all visible to the workgroup and
    // lie in consecutive rows of one buffer: all in k_cur, or all in the
    // cache without a ring wrap inside the tile.  One base pointer, no
    // per-row checks.
    auto fetch_fast = [&](int kt) -> bool {
        if (kt < wg_lo || kt + BN - 1 > wg_hi) return false;
        const f16 *kb, *vb;
        if (LIN) {
            kb = a.k + (size_t)kt * a.kv_dim;
            vb = a.v + (size_t)kt * a.kv_dim;
        } else if (kt >= cur_begin) {
            kb = a.k_cur + (size_t)(kt - base) * a.kv_dim;
            vb = a.v_cur + (size_t)(kt - base) * a.kv_dim;
        } else {
            if (kt + BN - 1 >= cur_begin) return false;
            int s0 = kt;
            if (w) {
                s0 = ring_slot(kt, w, a.w_magic, a.w_shift);
                if (s0 + BN > w) return false;
            }
            kb = a.k + (size_t)s0 * a.kv_dim;
            vb = a.v + (size_t)s0 * a.kv_dim;
        }
        kb += kvh * HD;
        vb += kvh * HD;
        if constexpr (kBufFetch) {
            // Buffer loads from the tile's first row: the per-load strides go
            // in the scalar offset and the immediate, so a thread keeps one
            // 32-bit offset for K and one for V, not a 64-bit address a load.
            const int kvb = a.kv_dim * 2;  // bytes per row
            const __amdgpu_buffer_rsrc_t rk_src = make_rsrc(kb), rv_src = make_rsrc(vb);
#pragma unroll
            for (int i = 0; i < KPT; ++i)
                rk[i] = __builtin_bit_cast(
                    f16x8, __builtin_amdgcn_raw_buffer_load_b128(rk_src, k_voff, i * (256 / KCH) * kvb, 0));
#pragma unroll
            for (int i = 0; i < VPT; ++i) {
                if (tid + 256 * i < KCHV * (BN / 4))
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        rv[i][u] = __builtin_bit_cast(
                            f16x8, __builtin_amdgcn_raw_buffer_load_b128(rv_src, v_voff + i * (256 / (BN / 4)) * 16,
                                                                          u * kvb, 0));
            }
            return true;
        }
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int c = tid + 256 * i;
            const int key = c / KCH, col = c - key * KCH;
            rk[i] = *reinterpret_cast<const f16x8*>(kb + (size_t)key * a.kv_dim + col * 8);
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int pr = tid + 256 * i;
            const int kg = pr % (BN / 4), dc = pr / (BN / 4);
            if (pr < KCHV * (BN / 4))
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    rv[i][u] = *reinterpret_cast<const f16x8*>(vb + (size_t)(4 * kg + u) * a.kv_dim + dc * 8);
        }
        return true;
    };
    // Edge tiles: rows outside the workgroup's range are zero.  (Loading a
    // clamped row and selecting zero instead of branching around each load
    // measured 13-29% slower: the longer loop body cost the common path.)
    auto fetch = [&](int kt) {
        if (fetch_fast(kt)) return;
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int c = tid + 256 * i;
            const int key = c / KCH, col = c - key * KCH;
            const int p = kt + key;
            f16x8 val = {};
            if (p >= wg_lo && p <= wg_hi)
                val = *reinterpret_cast<const f16x8*>(row_src(a.k, a.k_cur, p) + kvh * HD + col * 8);
            rk[i] = val;
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int pr = tid + 256 * i;
            const int kg = pr % (BN / 4), dc = pr / (BN / 4);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int p = kt + 4 * kg + u;
                f16x8 val = {};
                if (pr < KCHV * (BN / 4) && p >= wg_lo && p <= wg_hi)
                    val = *reinterpret_cast<const f16x8*>(row_src(a.v, a.v_cur, p) + kvh * HD + dc * 8);
                rv[i][u] = val;
            }
        }
    };
    auto stash = [&](int stage) {
        f16* Ks = K_s + stage * (BN * KPAD);
        f16* Vts = Vt_s + stage * (HD * VPAD);
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int c = tid + 256 * i;
            const int key = c / KCH, col = c - key * KCH;
            *reinterpret_cast<f16x8*>(&Ks[key * KPAD + col * 8]) = rk[i];
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int pr = tid + 256 * i;
            if (pr >= KCHV * (BN / 4)) continue;
            const int kg = pr % (BN / 4), dc = pr / (BN / 4);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                *reinterpret_cast<f16x4*>(&Vts[(dc * 8 + j) * VPAD + 4 * kg]) =
                    f16x4{rv[i][0][j], rv[i][1][j], rv[i][2][j], rv[i][3][j]};
        }
    };

    // This workgroup's split: chunk sp of the tiles covering [wg_lo, wg_hi].
    const int kt_all = (wg_lo / BN) * BN;
    const int n_t_all = wg_lo <= wg_hi ? (wg_hi - kt_all) / BN + 1 : 0;
    const int cs = (n_t_all + n_split - 1) / n_split;
    const int kt_begin = kt_all + sp * cs * BN;
    const int kt_stop = min(wg_hi, kt_begin + cs * BN - 1);
    if (kt_begin <= kt_stop) fetch(kt_begin);
    int stage = 0;
    for (int kt = kt_begin; kt <= kt_stop; kt += BN, stage ^= 1) {
        // Stage `stage` was last read two tiles ago, before the barrier of
        // the previous iteration: writing it now needs no extra barrier.
        stash(stage);
        __syncthreads();
        if (kt + BN <= kt_stop) fetch(kt + BN);
        // wave-uniform, and the same for both waves of a kPair block
        const bool live = wave_live && kt <= wv_hi && kt + BN - 1 >= wv_lo;
        if (!kPair && !live) continue;
        const bool need_mask = !(kt >= wv_lo_max && kt + BN - 1 <= wv_hi_min);
        const f16* Ks = K_s + stage * (BN * KPAD);
        const f16* Vts = Vt_s + stage * (HD * VPAD) + dh * HDV * VPAD;

        // ---- S^T - m = K Q^T - m, two 32-key blocks.  The accumulators start
        //      at -mb (mb = the running max once one is set), so the scores
        //      come out already shifted for exp2.  kPair: each wave's partial
        //      over its dims, scaled (c_sc), goes through X_s; every wave
        //      meets the barrier, live or not; the sum is then shifted by mb.
        float mb = m_run > -1e29f ? m_run : 0.f;
        f32x16 s[KB];
        if constexpr (kPair) {
            static_assert(KB == 1, "one 32-key block per tile in the pair exchange");
            if (live) {
                qk_tile<QD, KB, KPAD, true, kQlo, decltype(ql), kPairQkDepth>(Ks + dh * QD, qf, s, 0.f, c_sc, l32,
                                                                              hh, ql);
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    *reinterpret_cast<f32x4*>(&X_s[((wave * 4 + g) * 64 + lane) * 4]) =
                        f32x4{s[0][4 * g], s[0][4 * g + 1], s[0][4 * g + 2], s[0][4 * g + 3]};
            }
            __syncthreads();
            if (!live) continue;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 o4 = *reinterpret_cast<const f32x4*>(&X_s[(((wave ^ 2) * 4 + g) * 64 + lane) * 4]);
#pragma unroll
                for (int j = 0; j < 4; ++j) s[0][4 * g + j] = (s[0][4 * g + j] + o4[j]) - mb;
            }
        } else {
            qk_tile<HD, KB, KPAD, true, kQlo>(Ks, qf, s, mb, c_sc, l32, hh, ql);
        }

        // ---- mask, online softmax.  s[kb][i] is key
        //      kt + 32*kb + 8*(i/4) + 4*hh + i%4 for query qrow, minus mb.
        if (need_mask) {
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int key = kt + 32 * kb + 8 * (i / 4) + 4 * hh + (i % 4);
                    if (key < my_lo || key > my_hi) s[kb][i] = -INFINITY;
                }
        }
        // The tile in two halves of 32 keys (kb), each with its own softmax
        // step, so that the P.V MFMAs of half 0 can run while half 1's p is
        // formed.  P^T of a half is the B operand of two 16-key k-steps,
        // registers 0..7 and 8..15 of s[kb].  p = exp2(s) is formed first; the
        // lazy rescale then only asks whether some p exceeds 2^slack (a score
        // above m_run + slack), which a packed f16 max over the rounded p
        // answers with a quarter of the instructions of a float max over the
        // scores.  Such a half, and a query's first one (m_run not set yet),
        // take the exact path: the float max, the rescale of o and l, and p
        // again.
        constexpr float kSlackP = 256.f;  // 2^kRescaleSlack
        static_assert(kRescaleSlack == 8.f, "kSlackP is 2^kRescaleSlack");
        const f16x2 one2 = {(f16)1.f, (f16)1.f};
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            f16x8 pf[2];
            auto make_p = [&]() {
#pragma unroll
                for (int st = 0; st < 2; ++st)
#pragma unroll
                    for (int j = 0; j < 8; ++j) pf[st][j] = (f16)fast_exp2(s[kb][8 * st + j]);
            };
            make_p();
            f16x2 pm = {pf[0][0], pf[0][1]};
#pragma unroll
            for (int st = 0; st < 2; ++st)
#pragma unroll
                for (int j = 0; j < 8; j += 2) pm = __builtin_elementwise_max(pm, f16x2{pf[st][j], pf[st][j + 1]});
            // The test is "some p of the wave exceeds 2^slack": a ballot over
            // each lane's own p, no combine of a query's two half-columns.
            const float pmax = fmaxf((float)pm[0], (float)pm[1]);
            if (__builtin_amdgcn_ballot_w64(!(pmax <= kSlackP) || m_run < -1e29f) != 0) {
                float mt = -INFINITY;
#pragma unroll
                for (int i = 0; i < 16; ++i) mt = fmaxf(mt, s[kb][i]);
                mt = fmaxf(mt, shfl_xor(mt, 32)) + mb;  // the half's largest score
                const float mn = fmaxf(m_run, mt);
                const float corr = fast_exp2(m_run - mn);
                m_run = mn;
                l_run *= corr;
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) o[nb][i] *= corr;
                // The scores still to come in this tile become relative to
                // mn; while a query has seen no key (a masked half, m_run
                // still unset) they stay relative to 0.
                const float nmb = mn > -1e29f ? mn : 0.f;
                const float shift = nmb - mb;
#pragma unroll
                for (int k2 = kb; k2 < KB; ++k2)
#pragma unroll
                    for (int i = 0; i < 16; ++i) s[k2][i] -= shift;
                mb = nmb;
                make_p();
            }
            // The row sum takes the f16-rounded p, as the P.V product does,
            // two at a time (v_dot2_f32_f16 against 1).
#pragma unroll
            for (int st = 0; st < 2; ++st)
#pragma unroll
                for (int j = 0; j < 8; j += 2)
                    l_run = __builtin_amdgcn_fdot2(f16x2{pf[st][j], pf[st][j + 1]}, one2, l_run, false);

            // ---- O^T += V^T P^T.  A operand row = dim nb*32 + l32; keys
            //      32*kb + 16*st + 4*hh + {0..3} and + 8 + 4*hh + {0..3}.
            //      Later blocks' operands are read while block nb's MFMAs run.
            auto load = [&](int nb, f16x8 (&va)[2]) {
                const f16* vrow = &Vts[(nb * 32 + l32) * VPAD + 32 * kb + 4 * hh];
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const f16x4 v0 = *reinterpret_cast<const f16x4*>(vrow + 16 * st);
                    const f16x4 v1 = *reinterpret_cast<const f16x4*>(vrow + 16 * st + 8);
                    va[st] = f16x8{v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                }
            };
            // Operands PVD blocks ahead: 2 at head_dim >= 256, where one wave
            // per SIMD waits out each LDS round trip (+1.2% on Gemma's 4k
            // prefill; 3 measured the same), 1 below.
            constexpr int PVD = kPair ? kPairPvDepth : (HD >= 256 ? 2 : 1);
            static_assert(PVD < NB, "operand ring");
            f16x8 va[PVD + 1][2];
#pragma unroll
            for (int d0 = 0; d0 < PVD; ++d0) load(d0, va[d0]);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                if (nb + PVD < NB) load(nb + PVD, va[(nb + PVD) % (PVD + 1)]);
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    o[nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[nb % (PVD + 1)][st], pf[st], o[nb], 0, 0, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // then two LDS reads
                }
            }
        }
    }

    // ---- normalize and store: o[nb][i] is dim nb*32 + 8*(i/4) + 4*hh + i%4
    const float l_tot = l_run + shfl_xor(l_run, 32);
    if (!qvalid) return;
    if (n_split > 1) {
        // the split's partial: o as accumulated, and (m, l); an empty split
        // leaves m = -1e30, l = 0, o = 0
        const size_t row = ((size_t)sp * t + qrow) * a.H + h;
        if (hh == 0 && dh == 0) *reinterpret_cast<f32x2*>(a.part_ml + 2 * row) = f32x2{m_run, l_tot};
        float* prow = a.part_o + row * HD + dh * HDV;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4)
                *reinterpret_cast<f32x4*>(prow + nb * 32 + 8 * g4 + 4 * hh) =
                    f32x4{o[nb][4 * g4], o[nb][4 * g4 + 1], o[nb][4 * g4 + 2], o[nb][4 * g4 + 3]};
        return;
    }
    const float inv = 1.f / l_tot;
    float* orow = a.out + ((size_t)qrow * a.H + h) * HD + dh * HDV;
    const float* grow = a.gate ? a.gate + ((size_t)qrow * a.H + h) * a.gate_stride + dh * HDV : nullptr;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
            const int d = nb * 32 + 8 * g4 + 4 * hh;
            f32x4 y = f32x4{o[nb][4 * g4] * inv, o[nb][4 * g4 + 1] * inv, o[nb][4 * g4 + 2] * inv,
                            o[nb][4 * g4 + 3] * inv};
            if (grow) y = gate_sigmoid4(y, grow + d);
            *reinterpret_cast<f32x4*>(orow + d) = y;
        }
}

// Short batches from linear caches (a grid of 128-row tiles would leave
// half the CUs idle, as S = 512 at 32 heads does): a workgroup takes 64
// query rows of one head, and its two wave pairs walk the two halves of the
// workgroup's key tiles at once, each pair with its own two-stage K/V ring
// (128 threads copy a pair's tile), then merge through LDS.  The heaviest
// workgroup's serial chain of key tiles is halved (S = 512: 256 workgroups,
// at most 4 tiles each).  Wave w: rows 32 (w & 1) .. + 31, key half w >> 1.
// The per-tile step (scores, mask, online softmax, P.V) is attn_prefill_kernel's.
template <typename QT, int HD>
__global__ __launch_bounds__(256, 1) void attn_prefill_kh_kernel(PrefillArgs a) {
    static_assert(HD <= 128, "head_dim <= 128");
    constexpr bool kExact = sizeof(QT) == 2;
    constexpr int BN = 64;
    constexpr int HDV = HD;
    constexpr int KB = BN / 32;      // 32-key MFMA blocks per tile
    constexpr int KSTEPS = HD / 16;  // MFMA k-steps over head_dim
    constexpr int NB = HD / 32;      // 32-dim output blocks
    constexpr int KPAD = HD + 8;
    constexpr int VPAD = BN + 4;
    constexpr int KCH = HD / 8;                         // 16-byte chunks per key row
    constexpr int KPT = BN * KCH / 128;                 // K chunks per thread of a pair
    constexpr int VPT = (KCH * (BN / 4) + 127) / 128;   // V 4-key groups per thread of a pair
    static_assert(BN * KCH % 128 == 0, "K tile split");
    __shared__ __attribute__((aligned(16))) f16 K_s[2][2][BN * KPAD];   // [pair][stage]
    __shared__ __attribute__((aligned(16))) f16 Vt_s[2][2][HD * VPAD];

    const int nblk = gridDim.x;
    const int logical = xcd_remap(blockIdx.x, nblk);
    const int per_kvh = a.n_qtiles * a.G;
    const int kvh = logical / per_kvh;
    const int rem = logical - kvh * per_kvh;
    const int qt = a.n_qtiles - 1 - rem / a.G;  // heaviest first
    const int h = kvh * a.G + rem % a.G;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pair = wave >> 1, rb = wave & 1;  // key half, row block
    const int ptid = tid & 127;                 // thread within the pair
    const int l32 = lane & 31, hh = lane >> 5;
    const int t = a.n_tokens, base = a.base_pos, w = a.window;
    const int end = base + t - 1;
    const int q0 = qt * 64;
    const int qw0 = q0 + 32 * rb;

    const int qrow = qw0 + l32;
    const bool qvalid = qrow < t;
    const int qpos = base + qrow;
    const int my_lo = qvalid ? vis_lo(qpos, w) : 1;
    const int my_hi = qvalid ? vis_hi(qpos, w, a.bidi, end) : 0;

    f16x8 qf[KSTEPS];
    {
        const size_t qoff = ((size_t)(qvalid ? qrow : 0) * a.H + h) * a.q_stride + 8 * hh;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            float x[8];
            if constexpr (sizeof(QT) == 2) {
                const f16x8 q8 = *reinterpret_cast<const f16x8*>(reinterpret_cast<const f16*>(a.q) + qoff + ks * 16);
#pragma unroll
                for (int j = 0; j < 8; ++j) x[j] = (float)q8[j];
            } else {
                const float* qp = reinterpret_cast<const float*>(a.q) + qoff + ks * 16;
                const f32x4 x0 = *reinterpret_cast<const f32x4*>(qp);
                const f32x4 x1 = *reinterpret_cast<const f32x4*>(qp + 4);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    x[j] = x0[j];
                    x[4 + j] = x1[j];
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) qf[ks][j] = (f16)(kExact ? x[j] : x[j] * a.c);
        }
        settle_q(qf);
    }

    // ---- key ranges: the workgroup's, and this wave's
    const int q_last = min(q0 + 64, t) - 1;
    const int wg_lo = vis_lo(base + q0, w);
    const int wg_hi = vis_hi(base + q_last, w, a.bidi, end);
    const int wq_last = min(qw0 + 31, t - 1);
    const bool wave_live = qw0 < t;
    const int wv_lo = wave_live ? vis_lo(base + qw0, w) : 1;                    // smallest lo
    const int wv_hi = wave_live ? vis_hi(base + wq_last, w, a.bidi, end) : 0;  // largest hi
    const int wv_lo_max = wave_live ? vis_lo(base + wq_last, w) : 0;          // largest lo
    const int wv_hi_min = wave_live ? vis_hi(base + qw0, w, a.bidi, end) : -1; // smallest hi

    float m_run = -1e30f, l_run = 0.f;
    f32x16 o[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[nb][i] = 0.f;

    // ---- this pair's K/V tiles (linear addressing: key p is row p); rows
    // outside [wg_lo, wg_hi] are zero.  Same layouts as attn_prefill_kernel.
    f16x8 rk[KPT];
    f16x8 rv[VPT][4];
    auto fetch = [&](int kt) {
        const bool inside = kt >= wg_lo && kt + BN - 1 <= wg_hi;
        const f16* kb = a.k + (size_t)kvh * HD;
        const f16* vb = a.v + (size_t)kvh * HD;
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int c = ptid + 128 * i;
            const int key = c / KCH, col = c - key * KCH;
            const int p = kt + key;
            f16x8 val = {};
            if (inside || (p >= wg_lo && p <= wg_hi))
                val = *reinterpret_cast<const f16x8*>(kb + (size_t)p * a.kv_dim + col * 8);
            rk[i] = val;
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int pr = ptid + 128 * i;
            const int kg = pr % (BN / 4), dc = pr / (BN / 4);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int p = kt + 4 * kg + u;
                f16x8 val = {};
                if (pr < KCH * (BN / 4) && (inside || (p >= wg_lo && p <= wg_hi)))
                    val = *reinterpret_cast<const f16x8*>(vb + (size_t)p * a.kv_dim + dc * 8);
                rv[i][u] = val;
            }
        }
    };
    auto stash = [&](int stage) {
        f16* Ks = K_s[pair][stage];
        f16* Vts = Vt_s[pair][stage];
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int c = ptid + 128 * i;
            const int key = c / KCH, col = c - key * KCH;
            *reinterpret_cast<f16x8*>(&Ks[key * KPAD + col * 8]) = rk[i];
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int pr = ptid + 128 * i;
            if (pr >= KCH * (BN / 4)) continue;
            const int kg = pr % (BN / 4), dc = pr / (BN / 4);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                *reinterpret_cast<f16x4*>(&Vts[(dc * 8 + j) * VPAD + 4 * kg]) =
                    f16x4{rv[i][0][j], rv[i][1][j], rv[i][2][j], rv[i][3][j]};
        }
    };

    // The workgroup's tiles, first half to pair 0 and second to pair 1; both
    // pairs take `half` steps (the second may idle on its last), one
    // workgroup barrier each.
    const int kt_all = (wg_lo / BN) * BN;
    const int n_t_all = wg_lo <= wg_hi ? (wg_hi - kt_all) / BN + 1 : 0;
    const int half = (n_t_all + 1) / 2;
    const int first = pair * half;
    const int my_n = min(n_t_all, first + half) - first;  // tiles of this pair (>= 0)
    if (my_n > 0) fetch(kt_all + first * BN);
    for (int st = 0; st < half; ++st) {
        const int stage = st & 1;
        const int kt = kt_all + (first + st) * BN;
        const bool live = st < my_n;  // pair-uniform
        // Stage `stage` was last read two steps ago, before the barrier of
        // the previous step: writing it now needs no extra barrier.
        if (live) stash(stage);
        __syncthreads();
        if (st + 1 < my_n) fetch(kt + BN);
        if (!live || !wave_live || kt > wv_hi || kt + BN - 1 < wv_lo) continue;  // wave-uniform
        const bool need_mask = !(kt >= wv_lo_max && kt + BN - 1 <= wv_hi_min);
        const f16* Ks = K_s[pair][stage];
        const f16* Vts = Vt_s[pair][stage];

        // ---- S^T - m = K Q^T - m, two 32-key blocks.  The accumulators start
        //      at -mb (mb = the running max once one is set), so the scores
        //      come out already shifted for exp2.
        float mb = m_run > -1e29f ? m_run : 0.f;
        f32x16 s[KB];
        qk_tile<HD, KB, KPAD, kExact>(Ks, qf, s, mb, a.c, l32, hh);

        // ---- mask, online softmax.  s[kb][i] is key
        //      kt + 32*kb + 8*(i/4) + 4*hh + i%4 for query qrow, minus mb.
        if (need_mask) {
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int key = kt + 32 * kb + 8 * (i / 4) + 4 * hh + (i % 4);
                    if (key < my_lo || key > my_hi) s[kb][i] = -INFINITY;
                }
        }
        // The tile in two halves of 32 keys (kb), each with its own softmax
        // step, so that the P.V MFMAs of half 0 can run while half 1's p is
        // formed.  P^T of a half is the B operand of two 16-key k-steps,
        // registers 0..7 and 8..15 of s[kb].  p = exp2(s) is formed first; the
        // lazy rescale then only asks whether some p exceeds 2^slack (a score
        // above m_run + slack), which a packed f16 max over the rounded p
        // answers with a quarter of the instructions of a float max over the
        // scores.  Such a half, and a query's first one (m_run not set yet),
        // take the exact path: the float max, the rescale of o and l, and p
        // again.
        constexpr float kSlackP = 256.f;  // 2^kRescaleSlack
        static_assert(kRescaleSlack == 8.f, "kSlackP is 2^kRescaleSlack");
        const f16x2 one2 = {(f16)1.f, (f16)1.f};
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            f16x8 pf[2];
            auto make_p = [&]() {
#pragma unroll
                for (int st = 0; st < 2; ++st)
#pragma unroll
                    for (int j = 0; j < 8; ++j) pf[st][j] = (f16)fast_exp2(s[kb][8 * st + j]);
            };
            make_p();
            f16x2 pm = {pf[0][0], pf[0][1]};
#pragma unroll
            for (int st = 0; st < 2; ++st)
#pragma unroll
                for (int j = 0; j < 8; j += 2) pm = __builtin_elementwise_max(pm, f16x2{pf[st][j], pf[st][j + 1]});
            // The test is "some p of the wave exceeds 2^slack": a ballot over
            // each lane's own p, no combine of a query's two half-columns.
            const float pmax = fmaxf((float)pm[0], (float)pm[1]);
            if (__builtin_amdgcn_ballot_w64(!(pmax <= kSlackP) || m_run < -1e29f) != 0) {
                float mt = -INFINITY;
#pragma unroll
                for (int i = 0; i < 16; ++i) mt = fmaxf(mt, s[kb][i]);
                mt = fmaxf(mt, shfl_xor(mt, 32)) + mb;  // the half's largest score
                const float mn = fmaxf(m_run, mt);
                const float corr = fast_exp2(m_run - mn);
                m_run = mn;
                l_run *= corr;
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) o[nb][i] *= corr;
                // The scores still to come in this tile become relative to
                // mn; while a query has seen no key (a masked half, m_run
                // still unset) they stay relative to 0.
                const float nmb = mn > -1e29f ? mn : 0.f;
                const float shift = nmb - mb;
#pragma unroll
                for (int k2 = kb; k2 < KB; ++k2)
#pragma unroll
                    for (int i = 0; i < 16; ++i) s[k2][i] -= shift;
                mb = nmb;
                make_p();
            }
            // The row sum takes the f16-rounded p, as the P.V product does,
            // two at a time (v_dot2_f32_f16 against 1).
#pragma unroll
            for (int st = 0; st < 2; ++st)
#pragma unroll
                for (int j = 0; j < 8; j += 2)
                    l_run = __builtin_amdgcn_fdot2(f16x2{pf[st][j], pf[st][j + 1]}, one2, l_run, false);

            // ---- O^T += V^T P^T.  A operand row = dim nb*32 + l32; keys
            //      32*kb + 16*st + 4*hh + {0..3} and + 8 + 4*hh + {0..3}.
            //      Later blocks' operands are read while block nb's MFMAs run.
            auto load = [&](int nb, f16x8 (&va)[2]) {
                const f16* vrow = &Vts[(nb * 32 + l32) * VPAD + 32 * kb + 4 * hh];
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const f16x4 v0 = *reinterpret_cast<const f16x4*>(vrow + 16 * st);
                    const f16x4 v1 = *reinterpret_cast<const f16x4*>(vrow + 16 * st + 8);
                    va[st] = f16x8{v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                }
            };
            // Operands PVD blocks ahead: 2 at head_dim >= 256, where one wave
            // per SIMD waits out each LDS round trip (+1.2% on Gemma's 4k
            // prefill; 3 measured the same), 1 below.
            constexpr int PVD = HD >= 256 ? 2 : 1;
            static_assert(PVD < NB, "operand ring");
            f16x8 va[PVD + 1][2];
#pragma unroll
            for (int d0 = 0; d0 < PVD; ++d0) load(d0, va[d0]);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                if (nb + PVD < NB) load(nb + PVD, va[(nb + PVD) % (PVD + 1)]);
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    o[nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[nb % (PVD + 1)][st], pf[st], o[nb], 0, 0, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // then two LDS reads
                }
            }
        }
    }

    // ---- merge the two key halves of each row block through LDS (the K
    // stages, free after this barrier): pair 1 writes its o, max and row sum
    // lane-contiguous; pair 0 rescales both to the larger max and stores.
    const float l_tot = l_run + shfl_xor(l_run, 32);
    __syncthreads();
    constexpr int MW = NB * 16 + 2;  // floats a lane hands over
    static_assert(2 * MW * 64 * 4 <= (int)sizeof(K_s), "merge space");
    float* xs = reinterpret_cast<float*>(&K_s[0][0][0]) + rb * MW * 64;
    if (pair == 1) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int i = 0; i < 16; ++i) xs[(nb * 16 + i) * 64 + lane] = o[nb][i];
        xs[(NB * 16) * 64 + lane] = m_run;
        xs[(NB * 16 + 1) * 64 + lane] = l_tot;
    }
    __syncthreads();
    if (pair == 1 || !qvalid) return;
    const float m2 = xs[(NB * 16) * 64 + lane], l2 = xs[(NB * 16 + 1) * 64 + lane];
    const float mn = fmaxf(m_run, m2);
    const float c0 = fast_exp2(m_run - mn), c1 = fast_exp2(m2 - mn);
    const float inv = 1.f / (l_tot * c0 + l2 * c1);
    float* orow = a.out + ((size_t)qrow * a.H + h) * HD;
    const float* grow = a.gate ? a.gate + ((size_t)qrow * a.H + h) * a.gate_stride : nullptr;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
            const int d = nb * 32 + 8 * g4 + 4 * hh;
            f32x4 y;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = 4 * g4 + j;
                y[j] = (o[nb][i] * c0 + xs[(nb * 16 + i) * 64 + lane] * c1) * inv;
            }
            if (grow) y = gate_sigmoid4(y, grow + d);
            *reinterpret_cast<f32x4*>(orow + d) = y;
        }
}

// Combines the n_split partials of each (query row, head): with M the largest
// split max, out = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s, splits in
// order, then the output gate.  One thread per 4 output dims.
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillArgs a, int hd) {
    const int n_rows = a.n_tokens * a.H;
    const int c4n = hd / 4;
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long)n_rows * c4n) return;
    const int row = (int)(idx / c4n), c4 = (int)(idx % c4n);
    float M = -INFINITY;
    for (int sp = 0; sp < a.n_split; ++sp) M = fmaxf(M, a.part_ml[2 * ((size_t)sp * n_rows + row)]);
    float L = 0.f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int sp = 0; sp < a.n_split; ++sp) {
        const size_t r = (size_t)sp * n_rows + row;
        const f32x2 ml = *reinterpret_cast<const f32x2*>(a.part_ml + 2 * r);
        const float wgt = fast_exp2(ml[0] - M);
        L += wgt * ml[1];
        const f32x4 ov = *reinterpret_cast<const f32x4*>(a.part_o + r * hd + 4 * c4);
        acc += wgt * ov;
    }
    f32x4 y = acc * (1.f / L);
    if (a.gate) {
        const int qrow = row / a.H, h = row % a.H;
        y = gate_sigmoid4(y, a.gate + ((size_t)qrow * a.H + h) * a.gate_stride + 4 * c4);
    }
    *reinterpret_cast<f32x4*>(a.out + (size_t)row * hd + 4 * c4) = y;
}

// ---- Ping-pong variant (head_dim <= 128) -----------------------------------
//
// Eight waves, two per SIMD, each owning 32 query rows of a 256-row block
// (the same S^T = K Q^T, O^T += V^T P^T tiles as above).  A wave's work on key
// tile i is split into an MFMA phase, QK(i) and PV(i-1), and a VALU phase,
// mask + softmax(i) plus a share of the K/V copy.  Two barriers per tile keep
// group 0 (waves 0-3) and group 1 (waves 4-7) a phase apart, so on each SIMD
// one wave's MFMAs run while the other wave's exponentials issue:
//
//              phase 1                      phase 2
//   group 0    QK(i), PV(i-1)               softmax(i), copy K(i+1)
//   group 1    softmax(i-1), copy V(i)      QK(i), PV(i-1)
//
// K tile i and V tile i-1 are read in iteration i; the stages written in
// iteration i (K(i+1), V(i)) were last read in iteration i-1.  The MFMA
// phase runs at wave priority 1, so the SIMD issues the next MFMA as soon as
// the matrix pipe takes it and fills the gaps with the other wave's VALU.
constexpr int kPpBM = 256;  // query rows per workgroup: 8 waves x 32

template <typename QT, int HD, bool LIN>
__global__ __launch_bounds__(512, 1) void attn_prefill_pp_kernel(PrefillArgs a) {
    constexpr bool kExact = sizeof(QT) == 2;  // f16 queries: scale applied in fp32 (qk_tile)
    constexpr int BN = 64;
    constexpr int KB = BN / 32;      // 32-key MFMA blocks per tile
    constexpr int PST = BN / 16;     // 16-key P.V k-steps per tile
    constexpr int KSTEPS = HD / 16;  // MFMA k-steps over head_dim
    constexpr int NB = HD / 32;      // 32-dim output blocks
    constexpr int KPAD = HD + 8;
    constexpr int VPAD = BN + 4;
    static_assert(HD <= 128, "two waves per SIMD");
    __shared__ __attribute__((aligned(16))) f16 K_s[2 * BN * KPAD];
    __shared__ __attribute__((aligned(16))) f16 Vt_s[2 * HD * VPAD];

    // The workgroup's gp query heads share kv head kvh, 256 / gp rows each.
    const int nblk = gridDim.x;
    const int logical = xcd_remap(blockIdx.x, nblk);
    const int gp = a.gp, hgroups = a.G / gp;
    const int per_kvh = a.n_qtiles * hgroups;
    const int kvh = logical / per_kvh;
    const int rem = logical - kvh * per_kvh;
    const int qt = a.n_qtiles - 1 - rem / hgroups;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 2;
    const int ctid = tid & 255;  // thread index within the group (the copy split)
    const int l32 = lane & 31, hh = lane >> 5;
    const int t = a.n_tokens, base = a.base_pos, w = a.window;
    const int end = base + t - 1;
    const int bm = kPpBM / gp;  // query rows per head
    const int q0 = qt * bm;
    // The groups take alternate 32-row blocks, so the two waves of a SIMD
    // have nearly the same causal key range (and, with gp = 4, one head).
    const int blk = 2 * (wave & 3) + grp, bph = 8 / gp;  // 32-row blocks per head
    const int h = kvh * a.G + (rem % hgroups) * gp + blk / bph;
    const int qw0 = q0 + 32 * (blk % bph);

    const int qrow = qw0 + l32;
    const bool qvalid = qrow < t;
    const int qpos = base + qrow;
    const int my_lo = qvalid ? vis_lo(qpos, w) : 1;
    const int my_hi = qvalid ? vis_hi(qpos, w, a.bidi, end) : 0;

    f16x8 qf[KSTEPS];
    {
        const size_t qoff = ((size_t)(qvalid ? qrow : 0) * a.H + h) * a.q_stride + 8 * hh;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            float x[8];
            if constexpr (sizeof(QT) == 2) {
                const f16x8 q8 = *reinterpret_cast<const f16x8*>(reinterpret_cast<const f16*>(a.q) + qoff + ks * 16);
#pragma unroll
                for (int j = 0; j < 8; ++j) x[j] = (float)q8[j];
            } else {
                const float* qp = reinterpret_cast<const float*>(a.q) + qoff + ks * 16;
                const f32x4 x0 = *reinterpret_cast<const f32x4*>(qp);
                const f32x4 x1 = *reinterpret_cast<const f32x4*>(qp + 4);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    x[j] = x0[j];
                    x[4 + j] = x1[j];
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) qf[ks][j] = (f16)(kExact ? x[j] : x[j] * a.c);
        }
        settle_q(qf);
    }

    // ---- key tiles of the workgroup, and the wave's own run of them
    const int q_last = min(q0 + bm, t) - 1;
    const int wg_lo = vis_lo(base + q0, w);
    const int wg_hi = vis_hi(base + q_last, w, a.bidi, end);
    const int kt_begin = (wg_lo / BN) * BN;
    const int n_t = wg_lo <= wg_hi ? (wg_hi - kt_begin) / BN + 1 : 0;
    const bool wave_live = qw0 < t;
    const int wq_last = min(qw0 + 31, t - 1);
    const int wv_lo_max = wave_live ? vis_lo(base + wq_last, w) : 0;           // largest lo
    const int wv_hi_min = wave_live ? vis_hi(base + qw0, w, a.bidi, end) : -1;  // smallest hi
    int wi0 = 1, wi1 = 0;  // empty
    if (wave_live) {
        const int wv_lo = vis_lo(base + qw0, w);
        const int wv_hi = min(vis_hi(base + wq_last, w, a.bidi, end), wg_hi);
        if (wv_lo <= wv_hi) {
            wi0 = (wv_lo - kt_begin) / BN;
            wi1 = (wv_hi - kt_begin) / BN;
        }
    }
    const int cur_begin = (!LIN && a.k_cur) ? base : INT_MAX;

    float m_run = -1e30f, l_run = 0.f, mb = 0.f;
    f32x16 o[NB];
    f32x16 s[KB];
    f16x8 P[PST];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[nb][i] = 0.f;

    // ---- K/V copies, as in the kernel above; group 0 copies K, group 1 V,
    //      each with its 256 threads (ctid).
    constexpr int KCH = HD / 8;
    constexpr int KPT = BN * KCH / 256;
    constexpr int VPT = (KCH * (BN / 4) + 255) / 256;
    static_assert(BN * KCH % 256 == 0, "K tile split");
    f16x8 rk[KPT];
    f16x8 rv[VPT][4];
    auto row_src = [&](const f16* cache, const f16* cur, int p) -> const f16* {
        if constexpr (LIN) return cache + (size_t)p * a.kv_dim;
        if (p >= cur_begin) return cur + (size_t)(p - base) * a.kv_dim;
        const int sl = w ? ring_slot(p, w, a.w_magic, a.w_shift) : p;
        return cache + (size_t)sl * a.kv_dim;
    };
    // The base of a tile whose rows are all visible to the workgroup and lie
    // in consecutive rows of one buffer (all in k_cur, or all in the cache
    // without a ring wrap inside the tile), else NULL.
    auto fast_base = [&](const f16* cache, const f16* cur, int kt) -> const f16* {
        if (kt < wg_lo || kt + BN - 1 > wg_hi) return nullptr;
        if (LIN) return cache + (size_t)kt * a.kv_dim + kvh * HD;
        if (kt >= cur_begin) return cur + (size_t)(kt - base) * a.kv_dim + kvh * HD;
        if (kt + BN - 1 >= cur_begin) return nullptr;
        int s0 = kt;
        if (w) {
            s0 = ring_slot(kt, w, a.w_magic, a.w_shift);
            if (s0 + BN > w) return nullptr;
        }
        return cache + (size_t)s0 * a.kv_dim + kvh * HD;
    };
    // Interior tiles by buffer loads from the tile's first row (one 32-bit
    // offset a thread; the per-load strides in the scalar offset), as in
    // attn_prefill_kernel.
    static_assert(256 % KCH == 0 && 256 % (BN / 4) == 0, "uniform load strides");
    const int kvb = a.kv_dim * 2;  // bytes per row
    const int k_voff = (ctid / KCH) * kvb + (ctid % KCH) * 16;
    const int v_voff = 4 * (ctid % (BN / 4)) * kvb + (ctid / (BN / 4)) * 16;
    auto fetch_k = [&](int kt) {
        if (const f16* kb = fast_base(a.k, a.k_cur, kt)) {
            const __amdgpu_buffer_rsrc_t src = make_rsrc(kb);
#pragma unroll
            for (int i = 0; i < KPT; ++i)
                rk[i] = __builtin_bit_cast(
                    f16x8, __builtin_amdgcn_raw_buffer_load_b128(src, k_voff, i * (256 / KCH) * kvb, 0));
            return;
        }
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int c = ctid + 256 * i;
            const int key = c / KCH, col = c - key * KCH;
            const int p = kt + key;
            f16x8 val = {};
            if (p >= wg_lo && p <= wg_hi)
                val = *reinterpret_cast<const f16x8*>(row_src(a.k, a.k_cur, p) + kvh * HD + col * 8);
            rk[i] = val;
        }
    };
    auto fetch_v = [&](int kt) {
        if (const f16* vb = fast_base(a.v, a.v_cur, kt)) {
            const __amdgpu_buffer_rsrc_t src = make_rsrc(vb);
#pragma unroll
            for (int i = 0; i < VPT; ++i)
                if (ctid + 256 * i < KCH * (BN / 4))
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        rv[i][u] = __builtin_bit_cast(
                            f16x8, __builtin_amdgcn_raw_buffer_load_b128(src, v_voff + i * (256 / (BN / 4)) * 16,
                                                                          u * kvb, 0));
            return;
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int pr = ctid + 256 * i;
            const int kg = pr % (BN / 4), dc = pr / (BN / 4);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int p = kt + 4 * kg + u;
                f16x8 val = {};
                if (pr < KCH * (BN / 4) && p >= wg_lo && p <= wg_hi)
                    val = *reinterpret_cast<const f16x8*>(row_src(a.v, a.v_cur, p) + kvh * HD + dc * 8);
                rv[i][u] = val;
            }
        }
    };
    auto stash_k = [&](int stage) {
        f16* Ks = K_s + stage * (BN * KPAD);
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int c = ctid + 256 * i;
            const int key = c / KCH, col = c - key * KCH;
            *reinterpret_cast<f16x8*>(&Ks[key * KPAD + col * 8]) = rk[i];
        }
    };
    auto stash_v = [&](int stage) {
        f16* Vts = Vt_s + stage * (HD * VPAD);
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int pr = ctid + 256 * i;
            if (pr >= KCH * (BN / 4)) continue;
            const int kg = pr % (BN / 4), dc = pr / (BN / 4);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                *reinterpret_cast<f16x4*>(&Vts[(dc * 8 + j) * VPAD + 4 * kg]) =
                    f16x4{rv[i][0][j], rv[i][1][j], rv[i][2][j], rv[i][3][j]};
        }
    };

    // ---- the wave's steps
    // S^T - mb = K Q^T - mb; mb is the running max once one is set.
    auto qk = [&](const f16* Ks) {
        mb = m_run > -1e29f ? m_run : 0.f;
        qk_tile<HD, KB, KPAD, kExact>(Ks, qf, s, mb, a.c, l32, hh);
    };
    // s[kb][i] is key kt + 32*kb + 8*(i/4) + 4*hh + i%4 of query qrow.
    auto mask = [&](int kt) {
        if (kt >= wv_lo_max && kt + BN - 1 <= wv_hi_min) return;  // wave-uniform
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int key = kt + 32 * kb + 8 * (i / 4) + 4 * hh + (i % 4);
                if (key < my_lo || key > my_hi) s[kb][i] = -INFINITY;
            }
    };
    // p = exp2(s) into P (the B operands of the PST k-steps: step st is
    // registers 8*(st%2) .. +7 of s[st/2]); the lazy-rescale test on the f16
    // p as in the kernel above; l from the rounded p.
    constexpr float kSlackP = 256.f;  // 2^kRescaleSlack
    static_assert(kRescaleSlack == 8.f, "kSlackP is 2^kRescaleSlack");
    const f16x2 one2 = {(f16)1.f, (f16)1.f};
    auto softmax = [&]() {
        auto make_p = [&]() {
#pragma unroll
            for (int st = 0; st < PST; ++st)
#pragma unroll
                for (int j = 0; j < 8; ++j) P[st][j] = (f16)fast_exp2(s[st / 2][8 * (st % 2) + j]);
        };
        make_p();
        f16x2 pm = {P[0][0], P[0][1]};
#pragma unroll
        for (int st = 0; st < PST; ++st)
#pragma unroll
            for (int j = 0; j < 8; j += 2) pm = __builtin_elementwise_max(pm, f16x2{P[st][j], P[st][j + 1]});
        const float pmax = fmaxf((float)pm[0], (float)pm[1]);
        if (__builtin_amdgcn_ballot_w64(!(pmax <= kSlackP) || m_run < -1e29f) != 0) {
            float mt = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int i = 0; i < 16; ++i) mt = fmaxf(mt, s[kb][i]);
            mt = fmaxf(mt, shfl_xor(mt, 32)) + mb;  // the tile's largest score
            const float mn = fmaxf(m_run, mt);
            const float corr = fast_exp2(m_run - mn);
            m_run = mn;
            l_run *= corr;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[nb][i] *= corr;
            // no key seen yet (a masked tile): the scores stay relative to 0
            const float nmb = mn > -1e29f ? mn : 0.f;
            const float shift = nmb - mb;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int i = 0; i < 16; ++i) s[kb][i] -= shift;
            mb = nmb;
            make_p();
        }
#pragma unroll
        for (int st = 0; st < PST; ++st)
#pragma unroll
            for (int j = 0; j < 8; j += 2)
                l_run = __builtin_amdgcn_fdot2(f16x2{P[st][j], P[st][j + 1]}, one2, l_run, false);
    };
    // O^T += V^T P^T.  A operand row = dim nb*32 + l32; keys 16*st + 4*hh
    // + {0..3} and 16*st + 8 + 4*hh + {0..3} of the tile.
    // The A operands of output block nb+1 are read from LDS while block nb's
    // MFMAs run (one read in flight per MFMA would wait out the LDS latency
    // every time).
    auto pv = [&](const f16* Vts) {
        auto load = [&](int nb, f16x8 (&va)[PST]) {
            const f16* vrow = &Vts[(nb * 32 + l32) * VPAD + 4 * hh];
#pragma unroll
            for (int st = 0; st < PST; ++st) {
                const f16x4 v0 = *reinterpret_cast<const f16x4*>(vrow + 16 * st);
                const f16x4 v1 = *reinterpret_cast<const f16x4*>(vrow + 16 * st + 8);
                va[st] = f16x8{v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
            }
        };
        f16x8 va[2][PST];
        load(0, va[0]);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            if (nb + 1 < NB) load(nb + 1, va[(nb + 1) & 1]);
#pragma unroll
            for (int st = 0; st < PST; ++st) {
                o[nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[nb & 1][st], P[st], o[nb], 0, 0, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // then two LDS reads
            }
        }
    };

    // ---- prologue: K(0) staged, K(1) and V(0) in registers
    if (n_t > 0) {
        if (grp == 0) {
            fetch_k(kt_begin);
            stash_k(0);
            if (n_t > 1) fetch_k(kt_begin + BN);
        } else {
            fetch_v(kt_begin);
        }
    }
    // One loop per group (the group is fixed per wave); both run n_t + 1
    // iterations of two barriers each.  The compiler joins the groups' paths
    // (after the prologue, and from group 1's loop exit into group 0's
    // preheader, never taken), so its waitcnt pass would see group 1's V
    // fetch registers, which hold group 0's P, as pending in group 0's loop
    // and wait for group 0's own K fetch before every P.V and exponential.
    // Draining the loads before group 0's loop and after group 1's removes
    // those waits.
    if (grp == 0) {
        drain_loads();
        for (int i = 0; i <= n_t; ++i) {
            const int kt = kt_begin + i * BN;
            const bool k_in = i >= wi0 && i <= wi1;  // K tile i is the wave's (uniform)
            const bool v_in = i - 1 >= wi0 && i - 1 <= wi1;
            __syncthreads();
            __builtin_amdgcn_s_setprio(1);
            if (k_in) qk(K_s + (i & 1) * (BN * KPAD));
            if (v_in) pv(Vt_s + ((i + 1) & 1) * (HD * VPAD));
            __builtin_amdgcn_s_setprio(0);
            __syncthreads();
            if (k_in) {
                mask(kt);
                softmax();
            }
            if (i + 1 < n_t) stash_k((i + 1) & 1);
            if (i + 2 < n_t) fetch_k(kt + 2 * BN);
        }
    } else {
        for (int i = 0; i <= n_t; ++i) {
            const int kt = kt_begin + i * BN;
            const bool k_in = i >= wi0 && i <= wi1;
            const bool v_in = i - 1 >= wi0 && i - 1 <= wi1;
            __syncthreads();
            if (v_in) {
                mask(kt - BN);
                softmax();
            }
            if (i < n_t) stash_v(i & 1);
            if (i + 1 < n_t) fetch_v(kt + BN);
            __syncthreads();
            __builtin_amdgcn_s_setprio(1);
            if (k_in) qk(K_s + (i & 1) * (BN * KPAD));
            if (v_in) pv(Vt_s + ((i + 1) & 1) * (HD * VPAD));
            __builtin_amdgcn_s_setprio(0);
        }
        drain_loads();
    }

    // ---- normalize and store: o[nb][i] is dim nb*32 + 8*(i/4) + 4*hh + i%4
    const float l_tot = l_run + shfl_xor(l_run, 32);
    if (!qvalid) return;
    const float inv = 1.f / l_tot;
    float* orow = a.out + ((size_t)qrow * a.H + h) * HD;
    const float* grow = a.gate ? a.gate + ((size_t)qrow * a.H + h) * a.gate_stride : nullptr;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
            const int d = nb * 32 + 8 * g4 + 4 * hh;
            f32x4 y = f32x4{o[nb][4 * g4] * inv, o[nb][4 * g4 + 1] * inv, o[nb][4 * g4 + 2] * inv,
                            o[nb][4 * g4 + 3] * inv};
            if (grow) y = gate_sigmoid4(y, grow + d);
            *reinterpret_cast<f32x4*>(orow + d) = y;
        }
}

// The ping-pong kernel takes 256 query rows per workgroup and one workgroup
// per CU: it pays when there are at least two workgroups per CU (S >= 4096 at
// 32 heads; at S = 2048 a single round of unequal causal workgroups leaves
// CUs idle, and the 128-row kernel is faster).  LMX_PREFILL_KERNEL=pp|tile
// forces one of them (tuning overrides, for tests and sweeps).  fp32 queries
// take the 128-row kernel, which carries their f16 residual (qk_tile).
static bool use_ping_pong(int hd, long n_tokens, long n_heads, lmx_dtype q_dt) {
    if (hd != 128 || q_dt != LMX_F16) return false;
    if (const int f = tuning().prefill_kernel; f >= 0) return f == 1;
    return (n_tokens + kPpBM - 1) / kPpBM * n_heads >= 512;
}

// Query heads per prefill workgroup (they share one kv head).  At head_dim
// 256 two heads of a kv group share a workgroup (64 rows each): a 1024-key
// window then spans fewer key tiles per workgroup at the same MFMA work per
// tile.  At head_dim 512 (wave pairs, two 32-row blocks a workgroup) one.
// LMX_PREFILL_GP=1|2|4 overrides it (tuning overrides, for tests and sweeps)
// where it divides G and the workgroup has that many row blocks.
static int prefill_gp(int hd, int G, bool pp) {
    const int blocks = hd >= 512 ? 2 : 4;
    if (const int v = tuning().prefill_gp; v > 0 && G % v == 0 && v <= blocks) return v;
    if (pp || hd >= 512) return 1;
    return hd >= 256 && G % 2 == 0 ? 2 : 1;
}

// Query rows per attn_prefill_kernel workgroup and head: 32 per row block.
static int prefill_rows(int hd, int gp) { return (hd >= 512 ? kPfBM / 2 : kPfBM) / gp; }

// Key splits for attn_prefill_kernel.  When the query tiles give fewer
// workgroups than the CUs hold at once (two per CU, one at head_dim 256), as
// for a short chunk on a long cache, each tile's key range is cut into splits
// until that many are in flight, keeping at least kMinSplitTiles tiles per
// split; a merge kernel combines them.
constexpr int kMinSplitTiles = 8;
constexpr int kMaxSplits = 16;
constexpr int kCus = 256;
int decode_max_vis(const lmx_attn_params* p);
static int prefill_splits(const lmx_attn_params* p, lmx_dtype q_dt) {
    const int hd = (int)p->head_dim;
    if (use_ping_pong(hd, (long)p->n_tokens, (long)p->n_heads, q_dt)) return 1;
    const int gp = prefill_gp(hd, (int)(p->n_heads / p->n_kv_heads), false);
    const long bm = prefill_rows(hd, gp);
    const long n_wg = (long)((p->n_tokens + bm - 1) / bm) * (p->n_heads / gp);
    const long slots = (long)kCus * (hd > 128 ? 1 : 2);
    if (n_wg >= slots) return 1;
    const int bn = hd >= 256 ? 32 : 64;
    // the longest key range a workgroup covers: one query's range plus the
    // spread of the tile's positions
    const long tiles = ((long)decode_max_vis(p) + bm + bn - 1) / bn + 1;
    long sp = (slots + n_wg - 1) / n_wg;
    if (sp > tiles / kMinSplitTiles) sp = tiles / kMinSplitTiles;
    if (sp > kMaxSplits) sp = kMaxSplits;
    return sp < 2 ? 1 : (int)sp;
}

static size_t round_up256(size_t x) { return (x + 255) / 256 * 256; }

size_t prefill_workspace_bytes(const lmx_attn_params* p) {
    const int sp = std::max(prefill_splits(p, LMX_F16), prefill_splits(p, LMX_F32));
    if (sp == 1) return 0;
    const size_t rows = (size_t)sp * p->n_tokens * p->n_heads;
    return round_up256(rows * 2 * sizeof(float)) + round_up256(rows * p->head_dim * sizeof(float));
}

bool prefill_supported(const lmx_attn_params* p, lmx_dtype q_dt) {
    (void)q_dt;
    return p->head_dim == 64 || p->head_dim == 128 || p->head_dim == 256 || p->head_dim == 512;
}

lmx_status prefill_fwd(const lmx_attn_params* p, const AttnIo& io, const void* q, lmx_dtype q_dt,
                       const void* k_cache, const void* v_cache, const void* k_cur, const void* v_cur,
                       float* out, void* ws, size_t ws_bytes, hipStream_t st) {
    PrefillArgs a{};
    a.n_split = prefill_splits(p, q_dt);
    if (a.n_split > 1) {
        if (!ws || ws_bytes < prefill_workspace_bytes(p)) return LMX_E_WORKSPACE;
        if (((uintptr_t)ws & 255) != 0) return LMX_E_ALIGN;
        const size_t rows = (size_t)a.n_split * p->n_tokens * p->n_heads;
        a.part_ml = static_cast<float*>(ws);
        a.part_o = reinterpret_cast<float*>(static_cast<char*>(ws) + round_up256(rows * 2 * sizeof(float)));
    }
    a.q = q;
    a.q_stride = io.q_stride;
    a.gate = io.gate;
    a.gate_stride = io.gate_stride;
    a.k = static_cast<const f16*>(k_cache);
    a.v = static_cast<const f16*>(v_cache);
    a.k_cur = static_cast<const f16*>(k_cur);
    a.v_cur = static_cast<const f16*>(v_cur);
    a.out = out;
    a.H = (int)p->n_heads;
    a.Hkv = (int)p->n_kv_heads;
    a.G = a.H / a.Hkv;
    a.kv_dim = (int)p->kv_dim;
    a.base_pos = (int)p->base_pos;
    a.window = (int)p->window;
    a.n_tokens = (int)p->n_tokens;
    a.bidi = (int)p->bidi;
    a.c = p->scale * kLog2e;
    window_magic((uint32_t)a.window, &a.w_magic, &a.w_shift);
    const int hd = (int)p->head_dim;
    const bool pp = use_ping_pong(hd, (long)p->n_tokens, (long)p->n_heads, q_dt);
    a.gp = prefill_gp(hd, a.G, pp);
    const int bm = pp ? kPpBM / a.gp : prefill_rows(hd, a.gp);
    a.n_qtiles = (a.n_tokens + bm - 1) / bm;
    long nblk = (long)a.n_qtiles * (a.H / a.gp) * a.n_split;
    // Linear addressing: no k_cur rows and every position below the window;
    // or a batch at base 0 whose every key is a k_cur row (row p of k_cur is
    // position p), as a first windowed prefill chunk is.
    bool lin = !k_cur && (p->window == 0 || (uint64_t)p->base_pos + p->n_tokens <= p->window);
    if (k_cur && p->base_pos == 0) {
        a.k = static_cast<const f16*>(k_cur);
        a.v = static_cast<const f16*>(v_cur);
        lin = true;
    }
    // Key halves in one workgroup (attn_prefill_kh_kernel) when the 128-row
    // grid would fill at most half the CUs.  LMX_PREFILL_KH=0 turns it off
    // (tuning overrides, for tests and A/B timing).
    const bool kh = !pp && hd <= 128 && lin && a.n_split == 1 && a.gp == 1 && 2 * nblk <= kPfCus &&
                    q_dt == LMX_F16 && tuning().prefill_kh != 0;
    if (kh) {
        a.n_qtiles = (a.n_tokens + 63) / 64;
        nblk = (long)a.n_qtiles * a.H;
    }
    if (nblk > INT_MAX) return LMX_E_SHAPE;
    dim3 grid((unsigned)nblk);
    (void)hipGetLastError();
#define LMX_PF(QT, HDV)                                                                           \
    do {                                                                                          \
        if (lin) hipLaunchKernelGGL((attn_prefill_kernel<QT, HDV, true>), grid, dim3(256), 0, st, a); \
        else hipLaunchKernelGGL((attn_prefill_kernel<QT, HDV, false>), grid, dim3(256), 0, st, a);   \
    } while (0)
#define LMX_PP(QT)                                                                                \
    do {                                                                                          \
        if (lin) hipLaunchKernelGGL((attn_prefill_pp_kernel<QT, 128, true>), grid, dim3(512), 0, st, a); \
        else hipLaunchKernelGGL((attn_prefill_pp_kernel<QT, 128, false>), grid, dim3(512), 0, st, a);   \
    } while (0)
    if (kh) {  // f16 queries only
        if (hd == 64) hipLaunchKernelGGL((attn_prefill_kh_kernel<f16, 64>), grid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((attn_prefill_kh_kernel<f16, 128>), grid, dim3(256), 0, st, a);
    } else if (pp) {  // f16 queries only
        LMX_PP(f16);
    } else if (q_dt == LMX_F16) {
        if (hd == 64) LMX_PF(f16, 64);
        else if (hd == 128) LMX_PF(f16, 128);
        else if (hd == 256) LMX_PF(f16, 256);
        else if (hd == 512) LMX_PF(f16, 512);
        else return LMX_E_UNSUPPORTED;
    } else {
        if (hd == 64) LMX_PF(float, 64);
        else if (hd == 128) LMX_PF(float, 128);
        else if (hd == 256) LMX_PF(float, 256);
        else if (hd == 512) LMX_PF(float, 512);
        else return LMX_E_UNSUPPORTED;
    }
#undef LMX_PF
#undef LMX_PP
    if (a.n_split > 1) {
        const long items = (long)a.n_tokens * a.H * (hd / 4);
        hipLaunchKernelGGL(prefill_merge_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, st, a, hd);
    }
    LMX_CHECK_LAUNCH();
    return LMX_OK;
}

}  // namespace lmx
