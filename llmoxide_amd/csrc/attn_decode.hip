// Split-K attention for few query tokens (decode) on gfx950.
//
// Replaces, for n_tokens small, the reference's three passes scores_pass /
// softmax_pass / weighted_v (attn.wgsl:84-232), which give decode only
// n_heads workgroups and a serial key loop (attn.wgsl:13-17).
//
// Work split.  A "unit" is one (query, kv head, block of GB query heads that
// share the kv head); K/V of a unit are read once for all GB heads (GQA).  A
// unit's visible key range is cut into chunks of kWaves*kTU*16 keys; P
// workgroups serve each unit, workgroup w taking chunks w, w+P, w+2P, ...
// (a static, deterministic split).  Every wave streams its share of those
// chunks with the next chunk's K/V loads in flight while it computes the
// current one.  Each workgroup leaves one partial (max, sum, o[hd]) per head;
// the last workgroup to arrive merges the unit's partials.  Partials cross workgroups with
// agent-coherent (sc1) stores and loads and a counter atomic issued after the
// stores are acknowledged, so no L2 writeback is needed.
//
// Per wave, 16-key tiles:
//   S^T[16 keys x 16 cols] = K Q^T on v_mfma_f32_16x16x32_f16.  Columns
//   0..GB-1 hold the f16 high part of each query head, columns GB..2GB-1 the
//   f16 residual (q - hi) of an fp32 query, so q.k is exact to ~2^-22.
//   Lane (g, c) then holds keys 4g..4g+3 of column c: the online softmax runs
//   once per (key, head), in fp32, with exp2 and scale*log2(e) folded in.
//   p goes through a small per-wave LDS slot to the P.V lanes, which own
//   hd/16 dims of one key in four and accumulate in fp32 VALU (each lane reads
//   a contiguous hd/16-element slice of a V row).
#include <climits>
#include <cstdlib>

#include "common.hpp"

namespace lmx {

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
    float* part_o;          // [n_q][H][P][HD]   per-workgroup partials
    float* part_ml;         // [n_q][H][P][2]    (max in log2 units, sum)
    uint32_t* ctr_arrive;   // [units]  workgroups finished
    int H, Hkv, G, kv_dim;
    int base_pos, window, n_tokens, bidi;
    int P, n_hblk;
    int max_ctx;  // batched: context lengths are clamped to [1, max_ctx]
    float c;      // scale * log2(e)
};

constexpr int kWaves = 8;
constexpr int kDecThreads = kWaves * 64;
constexpr int kMaxP = 64;  // workgroups per unit

// Register budget per lane (of 256 at two waves per SIMD) for the K/V tile
// buffers: each 16-key tile holds hd/8 VGPRs of K and hd/8 of V per lane.
// Two tiles per wave per chunk, double-buffered, when they fit; else one tile,
// double-buffered; else one tile, loaded and used in turn.
__host__ __device__ constexpr int dec_base_regs(int hd, int gb) { return hd / 8 + gb * hd / 16 + 48; }
__host__ __device__ constexpr int dec_tile_regs(int hd) { return hd / 8 + hd / 8; }
__host__ __device__ constexpr int tiles_per_wave(int hd, int gb) {
    return dec_base_regs(hd, gb) + 4 * dec_tile_regs(hd) <= 232 ? 2 : 1;
}
__host__ __device__ constexpr bool dec_pipelined(int hd, int gb) {
    return dec_base_regs(hd, gb) + 2 * tiles_per_wave(hd, gb) * dec_tile_regs(hd) <= 232;
}
__host__ __device__ constexpr int chunk_keys(int hd, int gb) { return kWaves * tiles_per_wave(hd, gb) * 16; }

// Agent-coherent accesses (global_store/load ... sc1): visible across XCDs
// without an L2 writeback.
__device__ __forceinline__ void st_co(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_co(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

template <typename QT, int HD, int GB, bool BATCHED>
__global__ __launch_bounds__(kDecThreads) void attn_decode_kernel(DecodeArgs a) {
    constexpr int KD = HD / 4;      // K dims per lane (contiguous)
    constexpr int KSTEP = HD / 32;  // MFMA k-steps
    constexpr int DPL = HD / 16;    // V dims per lane
    constexpr bool SPLIT_Q = sizeof(QT) == 4;
    constexpr int kTU = tiles_per_wave(HD, GB);
    constexpr int CH = chunk_keys(HD, GB);
    constexpr bool PIPE = dec_pipelined(HD, GB);
    static_assert(GB * (SPLIT_Q ? 2 : 1) <= 16, "query columns");
    const int wg = blockIdx.x;
    const int kvh = blockIdx.y / a.n_hblk;
    const int hb = blockIdx.y - kvh * a.n_hblk;
    const int qi = blockIdx.z;
    const int h0 = kvh * a.G + hb * GB;
    const size_t unit = ((size_t)qi * a.Hkv + kvh) * a.n_hblk + hb;

    int lo, hi, cur_begin;
    const f16 *kc, *vc;
    if constexpr (BATCHED) {
        // Out-of-range lengths are clamped so every read stays in the cache
        // the caller sized for max_ctx.
        const int pos = min(max(a.ctx_lens[qi], 1), a.max_ctx) - 1;
        lo = (a.window && pos + 1 > a.window) ? pos + 1 - a.window : 0;
        hi = pos;
        kc = a.k_ptrs[qi];
        vc = a.v_ptrs[qi];
        cur_begin = INT_MAX;
    } else {
        // attn.wgsl:52-66 (first_visible / last_visible)
        const int pos = a.base_pos + qi;
        lo = (a.window && pos + 1 > a.window) ? pos + 1 - a.window : 0;
        if (a.bidi) {
            const int end = a.base_pos + a.n_tokens - 1;
            hi = a.window ? min(end, pos + a.window - 1) : end;
        } else {
            hi = pos;
        }
        kc = a.k;
        vc = a.v;
        cur_begin = a.k_cur ? a.base_pos : INT_MAX;
    }
    const int n_chunks = (hi - lo + 1 + CH - 1) / CH;
    if (wg >= n_chunks) return;  // uniform: more workgroups than chunks
    const int P = a.P;
    const int p_eff = min(P, n_chunks);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g4 = lane >> 4, c16 = lane & 15;
    const int w = a.window;

    // Q^T as the MFMA B operand: column c16, dims KD*g4 + 8*s + j.
    f16x8 qf[KSTEP];
    {
        int head = -1;
        bool lo_part = false;
        if (c16 < GB) {
            head = h0 + c16;
        } else if (SPLIT_Q && c16 < 2 * GB) {
            head = h0 + c16 - GB;
            lo_part = true;
        }
#pragma unroll
        for (int s = 0; s < KSTEP; ++s) {
            f16x8 v = {};
            if (head >= 0) {
                const size_t qo = ((size_t)qi * a.H + head) * HD + KD * g4 + 8 * s;
                if constexpr (SPLIT_Q) {
                    const float* qp = reinterpret_cast<const float*>(a.q) + qo;
                    const f32x4 x0 = *reinterpret_cast<const f32x4*>(qp);
                    const f32x4 x1 = *reinterpret_cast<const f32x4*>(qp + 4);
                    const float xs[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const f16 hi16 = (f16)xs[j];
                        v[j] = lo_part ? (f16)(xs[j] - (float)hi16) : hi16;
                    }
                } else {
                    v = *reinterpret_cast<const f16x8*>(reinterpret_cast<const f16*>(a.q) + qo);
                }
            }
            qf[s] = v;
        }
    }

    // Softmax state of column c16 (meaningful for c16 < GB).
    float m_run = -1e30f, l_run = 0.f;
    float o[GB][DPL];
#pragma unroll
    for (int h = 0; h < GB; ++h)
#pragma unroll
        for (int d = 0; d < DPL; ++d) o[h][d] = 0.f;

    // Per-wave LDS slots: p[tile][key][head] and corr[tile][head].
    __shared__ float P_s[kWaves][kTU][16][8];
    __shared__ float C_s[kWaves][kTU][8];

    // This wave's work: group j is chunk wg + j*P, of which the wave takes
    // the kTU tiles starting at key wave*16*kTU.  Groups are double-buffered
    // in registers: group j+1 is loaded while group j is computed.
    struct Tiles {
        f16x8 k[kTU][KSTEP];
        RawF16<DPL> v[kTU][4];
    };
    auto row_of = [&](const f16* cache, const f16* cur, int p, int k0, int s_base) -> const f16* {
        if (p >= cur_begin) return cur + (size_t)(p - a.base_pos) * a.kv_dim + kvh * HD;
        int s = p;
        if (w) {
            s = s_base + (p - k0);
            if (s >= w) s -= w;
            if (s >= w) s %= w;
        }
        return cache + (size_t)s * a.kv_dim + kvh * HD;
    };
    auto load_group = [&](int j, Tiles& b) {
        const int k0 = lo + (wg + j * P) * CH;
        const int k1 = min(k0 + CH, hi + 1);
        const int tb = k0 + wave * 16 * kTU;
        if (tb >= k1) return;
        const int s_base = w ? k0 % w : 0;
#pragma unroll
        for (int t = 0; t < kTU; ++t) {
            const int base_t = tb + 16 * t;
            const int pk = min(base_t + c16, k1 - 1);
            const f16* krow = row_of(kc, a.k_cur, pk, k0, s_base) + KD * g4;
#pragma unroll
            for (int s = 0; s < KSTEP; ++s) b.k[t][s] = *reinterpret_cast<const f16x8*>(krow + 8 * s);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int pv = min(base_t + 4 * i + g4, k1 - 1);
                load_raw<DPL>(row_of(vc, a.v_cur, pv, k0, s_base) + DPL * c16, b.v[t][i]);
            }
        }
    };
    auto compute_group = [&](int j, const Tiles& b) {
        const int k0 = lo + (wg + j * P) * CH;
        const int k1 = min(k0 + CH, hi + 1);
        const int tb = k0 + wave * 16 * kTU;
        if (tb >= k1) return;
        wave_lds_sync();  // the previous group's P.V reads are done
#pragma unroll
        for (int t = 0; t < kTU; ++t) {
            const int base_t = tb + 16 * t;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < KSTEP; ++s)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(b.k[t][s], qf[s], acc, 0, 0, 0);
            float x[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float sv = acc[i];
                if constexpr (SPLIT_Q) sv += row_rotate_down<GB>(sv);
                const int key = base_t + 4 * g4 + i;
                x[i] = key < k1 ? sv * a.c : -INFINITY;
            }
            float tm = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
            tm = fmaxf(tm, shfl_xor(tm, 16));
            tm = fmaxf(tm, shfl_xor(tm, 32));
            const float mn = fmaxf(m_run, tm);
            const float corr = fast_exp2(m_run - mn);
            m_run = mn;
            float ps = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float p = fast_exp2(x[i] - mn);
                ps += p;
                if (c16 < GB) P_s[wave][t][4 * g4 + i][c16] = p;
            }
            l_run = l_run * corr + ps;
            if (c16 < GB && g4 == 0) C_s[wave][t][c16] = corr;
        }
        wave_lds_sync();
#pragma unroll
        for (int t = 0; t < kTU; ++t) {
            float corr[GB];
#pragma unroll
            for (int h = 0; h < GB; ++h) corr[h] = C_s[wave][t][h];
#pragma unroll
            for (int h = 0; h < GB; ++h)
#pragma unroll
                for (int d = 0; d < DPL; ++d) o[h][d] *= corr[h];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int kk = 4 * i + g4;
#pragma unroll
                for (int h = 0; h < GB; ++h) {
                    const float p = P_s[wave][t][kk][h];
#pragma unroll
                    for (int d = 0; d < DPL; ++d) o[h][d] = fmaf(p, raw_at<DPL>(b.v[t][i], d), o[h][d]);
                }
            }
        }
    };

    const int n_groups = (n_chunks - wg + P - 1) / P;  // chunks wg, wg+P, ... below n_chunks
    if constexpr (PIPE) {
        Tiles buf0, buf1;
        load_group(0, buf0);
        for (int j = 0; j < n_groups; j += 2) {
            if (j + 1 < n_groups) load_group(j + 1, buf1);
            compute_group(j, buf0);
            if (j + 1 >= n_groups) break;
            if (j + 2 < n_groups) load_group(j + 2, buf0);
            compute_group(j + 1, buf1);
        }
    } else {
        Tiles buf;
        for (int j = 0; j < n_groups; ++j) {
            load_group(j, buf);
            compute_group(j, buf);
        }
    }

    // Reduce the wave: l over the four lanes of each column, o over the four
    // key groups (all share the column's running max).
    l_run += shfl_xor(l_run, 16);
    l_run += shfl_xor(l_run, 32);
#pragma unroll
    for (int h = 0; h < GB; ++h)
#pragma unroll
        for (int d = 0; d < DPL; ++d) {
            float x = o[h][d];
            x += shfl_xor(x, 16);
            x += shfl_xor(x, 32);
            o[h][d] = x;
        }

    __shared__ float sm_o[kWaves][GB][HD];
    __shared__ float sm_m[kWaves][GB];
    __shared__ float sm_l[kWaves][GB];
    if (g4 == 0) {
#pragma unroll
        for (int h = 0; h < GB; ++h)
#pragma unroll
            for (int d = 0; d < DPL; ++d) sm_o[wave][h][DPL * c16 + d] = o[h][d];
        if (c16 < GB) {
            sm_m[wave][c16] = m_run;
            sm_l[wave][c16] = l_run;
        }
    }
    __syncthreads();

    const size_t qh0 = (size_t)qi * a.H + h0;  // first (query, head) row of this unit
    for (int idx = tid; idx < GB * HD; idx += kDecThreads) {
        const int g = idx / HD, d = idx - g * HD;
        float M = sm_m[0][g];
#pragma unroll
        for (int ww = 1; ww < kWaves; ++ww) M = fmaxf(M, sm_m[ww][g]);
        float O = 0.f, L = 0.f;
#pragma unroll
        for (int ww = 0; ww < kWaves; ++ww) {
            const float sc = fast_exp2(sm_m[ww][g] - M);
            O = fmaf(sm_o[ww][g][d], sc, O);
            L = fmaf(sm_l[ww][g], sc, L);
        }
        if (p_eff == 1) {
            a.out[(qh0 + g) * HD + d] = O / L;
        } else {
            const size_t pidx = (qh0 + g) * P + wg;
            st_co(a.part_o + pidx * HD + d, O);
            if (d == 0) {
                st_co(a.part_ml + pidx * 2, M);
                st_co(a.part_ml + pidx * 2 + 1, L);
            }
        }
    }
    if (p_eff == 1) return;

    // Count this workgroup in once its sc1 stores are acknowledged; the last
    // one merges the unit's partials and resets the unit's counter.
    __shared__ int s_last;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(a.ctr_arrive + unit, 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        const bool last = old == (uint32_t)p_eff - 1;
        if (last) __hip_atomic_store(a.ctr_arrive + unit, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = last;
    }
    __syncthreads();
    if (!s_last) return;

    // Merge: wave g < GB computes head g's weights over the partials
    // (lane s); then thread (part, column) sums every SP-th partial of one
    // float4 column and the parts are added in LDS.
    __shared__ float s_w[GB][kMaxP];
    __shared__ float s_L[GB];
    if (wave < GB) {
        const int g = wave;
        const float* ml = a.part_ml + (qh0 + g) * P * 2;
        float m = -1e30f, l = 0.f;
        if (lane < p_eff) {
            m = ld_co(ml + lane * 2);
            l = ld_co(ml + lane * 2 + 1);
        }
        float M = m;
#pragma unroll
        for (int x = 1; x < 64; x <<= 1) M = fmaxf(M, shfl_xor(M, x));
        const float wgt = lane < p_eff ? fast_exp2(m - M) : 0.f;
        float L = wgt * l;
#pragma unroll
        for (int x = 1; x < 64; x <<= 1) L += shfl_xor(L, x);
        s_w[g][lane] = wgt;
        if (lane == 0) s_L[g] = L;
    }
    __syncthreads();
    constexpr int NCOL = GB * HD / 4;
    constexpr int SP = kDecThreads / NCOL >= 1 ? kDecThreads / NCOL : 1;
    __shared__ f32x4 s_red[SP][NCOL];
    for (int idx = tid; idx < SP * NCOL; idx += kDecThreads) {
        const int part = idx / NCOL, col = idx % NCOL;
        const int g = col / (HD / 4), d4 = col % (HD / 4);
        const float* src = a.part_o + (qh0 + g) * P * HD + 4 * d4;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int s = part; s < p_eff; s += SP) {
            const float wgt = s_w[g][s];
            const float* p = src + (size_t)s * HD;
            acc[0] = fmaf(wgt, ld_co(p), acc[0]);
            acc[1] = fmaf(wgt, ld_co(p + 1), acc[1]);
            acc[2] = fmaf(wgt, ld_co(p + 2), acc[2]);
            acc[3] = fmaf(wgt, ld_co(p + 3), acc[3]);
        }
        s_red[part][col] = acc;
    }
    __syncthreads();
    for (int col = tid; col < NCOL; col += kDecThreads) {
        const int g = col / (HD / 4), d4 = col % (HD / 4);
        f32x4 acc = s_red[0][col];
#pragma unroll
        for (int part = 1; part < SP; ++part) {
            const f32x4 x = s_red[part][col];
            acc[0] += x[0];
            acc[1] += x[1];
            acc[2] += x[2];
            acc[3] += x[3];
        }
        const float inv = 1.f / s_L[g];
        *reinterpret_cast<f32x4*>(a.out + (qh0 + g) * HD + 4 * d4) =
            f32x4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
    }
}

// ------------------------------------------------------------------ host --

struct DecodePlan {
    int P, n_hblk, gb;
    size_t ctr_bytes, ml_bytes, o_bytes;
    size_t total() const { return ctr_bytes + ml_bytes + o_bytes; }
};

// Query heads per workgroup: the largest divisor of G within the register
// budget (o holds gb * hd/16 floats per lane) and the 16 MFMA columns (an
// fp32 query takes two columns per head).
static int pick_gb(int G, int hd) {
    const int cap = hd >= 512 ? 1 : (hd == 256 ? 4 : 8);
    for (int gb = cap; gb >= 1; --gb)
        if (G % gb == 0) return gb;
    return 1;
}

static size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Workgroups the heuristic aims for: one 8-wave workgroup per CU on 256 CUs.
// LMX_DECODE_TARGET_WGS overrides it for tuning sweeps.
static long target_wgs() {
    static long v = [] {
        const char* e = std::getenv("LMX_DECODE_TARGET_WGS");
        long x = e ? std::atol(e) : 0;
        return x > 0 ? x : 256L;
    }();
    return v;
}

// n_q query rows (tokens or sequences), longest visible range max_vis.
static DecodePlan plan_decode(int n_q, int H, int Hkv, int hd, int max_vis) {
    DecodePlan pl{};
    const int G = H / Hkv;
    pl.gb = pick_gb(G, hd);
    pl.n_hblk = G / pl.gb;
    const long units = (long)n_q * Hkv * pl.n_hblk;
    const long n_chunks = (max_vis + chunk_keys(hd, pl.gb) - 1) / chunk_keys(hd, pl.gb);
    long P = (target_wgs() + units - 1) / units;
    if (P > n_chunks) P = n_chunks;
    if (P > kMaxP) P = kMaxP;
    if (P < 1) P = 1;
    pl.P = (int)P;
    if (P > 1) {
        pl.ctr_bytes = round_up((size_t)units * 4, 256);
        pl.ml_bytes = round_up((size_t)n_q * H * P * 2 * 4, 256);
        pl.o_bytes = round_up((size_t)n_q * H * P * hd * 4, 256);
    }
    return pl;
}

template <typename QT, bool BATCHED>
static lmx_status launch_decode(const DecodeArgs& a, int hd, int gb, dim3 grid, hipStream_t st) {
#define LMX_DEC_CASE(HDV, GBV)                                                                   \
    if (hd == HDV && gb == GBV) {                                                                \
        hipLaunchKernelGGL((attn_decode_kernel<QT, HDV, GBV, BATCHED>), grid, dim3(kDecThreads), \
                           0, st, a);                                                            \
        return LMX_OK;                                                                           \
    }
    LMX_DEC_CASE(64, 1) LMX_DEC_CASE(64, 2) LMX_DEC_CASE(64, 3) LMX_DEC_CASE(64, 4)
    LMX_DEC_CASE(64, 5) LMX_DEC_CASE(64, 6) LMX_DEC_CASE(64, 7) LMX_DEC_CASE(64, 8)
    LMX_DEC_CASE(128, 1) LMX_DEC_CASE(128, 2) LMX_DEC_CASE(128, 3) LMX_DEC_CASE(128, 4)
    LMX_DEC_CASE(128, 5) LMX_DEC_CASE(128, 6) LMX_DEC_CASE(128, 7) LMX_DEC_CASE(128, 8)
    LMX_DEC_CASE(256, 1) LMX_DEC_CASE(256, 2) LMX_DEC_CASE(256, 3) LMX_DEC_CASE(256, 4)
    LMX_DEC_CASE(512, 1)
#undef LMX_DEC_CASE
    return LMX_E_UNSUPPORTED;
}

// Longest visible range over the batch's queries (attn.wgsl:52-66 maximized
// over the tokens; O(t) and t is small on this path).
int decode_max_vis(const lmx_attn_params* p) {
    long best = 0;
    const long t = p->n_tokens, base = p->base_pos, w = p->window;
    for (long i = 0; i < t; ++i) {
        const long pos = base + i;
        const long lo = (w && pos + 1 > w) ? pos + 1 - w : 0;
        long hi = pos;
        if (p->bidi) {
            const long end = base + t - 1;
            hi = w ? (end < pos + w - 1 ? end : pos + w - 1) : end;
        }
        if (hi - lo + 1 > best) best = hi - lo + 1;
    }
    return (int)best;
}

size_t decode_workspace_bytes(const lmx_attn_params* p) {
    const DecodePlan pl = plan_decode((int)p->n_tokens, (int)p->n_heads, (int)p->n_kv_heads,
                                      (int)p->head_dim, decode_max_vis(p));
    return pl.total();
}

size_t decode_batched_workspace_bytes(const lmx_attn_params* p, int n_seq, int max_ctx) {
    int mv = max_ctx;
    if (p->window && (int)p->window < mv) mv = (int)p->window;
    const DecodePlan pl = plan_decode(n_seq, (int)p->n_heads, (int)p->n_kv_heads,
                                      (int)p->head_dim, mv);
    return pl.total();
}

static lmx_status run(DecodeArgs a, const DecodePlan& pl, int n_q, int hd, lmx_dtype q_dt,
                      bool batched, void* ws, size_t ws_bytes, hipStream_t st) {
    if (pl.total() > 0) {
        if (!ws || ws_bytes < pl.total()) return LMX_E_WORKSPACE;
        if (((uintptr_t)ws & 255) != 0) return LMX_E_ALIGN;
        char* b = static_cast<char*>(ws);
        a.ctr_arrive = reinterpret_cast<uint32_t*>(b);
        b += pl.ctr_bytes;
        a.part_ml = reinterpret_cast<float*>(b);
        b += pl.ml_bytes;
        a.part_o = reinterpret_cast<float*>(b);
    }
    a.P = pl.P;
    a.n_hblk = pl.n_hblk;
    dim3 grid(pl.P, a.Hkv * pl.n_hblk, n_q);
    (void)hipGetLastError();
    lmx_status s;
    if (q_dt == LMX_F32)
        s = batched ? launch_decode<float, true>(a, hd, pl.gb, grid, st)
                    : launch_decode<float, false>(a, hd, pl.gb, grid, st);
    else
        s = batched ? launch_decode<f16, true>(a, hd, pl.gb, grid, st)
                    : launch_decode<f16, false>(a, hd, pl.gb, grid, st);
    if (s != LMX_OK) return s;
    LMX_CHECK_LAUNCH();
    return LMX_OK;
}

lmx_status decode_fwd(const lmx_attn_params* p, const void* q, lmx_dtype q_dt, const void* k_cache,
                      const void* v_cache, const void* k_cur, const void* v_cur, float* out,
                      void* ws, size_t ws_bytes, hipStream_t st) {
    DecodeArgs a{};
    a.q = q;
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
    const DecodePlan pl = plan_decode(a.n_tokens, a.H, a.Hkv, (int)p->head_dim, decode_max_vis(p));
    return run(a, pl, a.n_tokens, (int)p->head_dim, q_dt, false, ws, ws_bytes, st);
}

lmx_status decode_batched(const lmx_attn_params* p, int n_seq, int max_ctx, const int32_t* ctx_lens,
                          const void* const* k_ptrs, const void* const* v_ptrs, const void* q,
                          lmx_dtype q_dt, float* out, void* ws, size_t ws_bytes, hipStream_t st) {
    DecodeArgs a{};
    a.q = q;
    a.k_ptrs = reinterpret_cast<const f16* const*>(k_ptrs);
    a.v_ptrs = reinterpret_cast<const f16* const*>(v_ptrs);
    a.ctx_lens = ctx_lens;
    a.out = out;
    a.H = (int)p->n_heads;
    a.Hkv = (int)p->n_kv_heads;
    a.G = a.H / a.Hkv;
    a.kv_dim = (int)p->kv_dim;
    a.window = (int)p->window;
    a.n_tokens = 1;
    a.max_ctx = max_ctx;
    a.c = p->scale * kLog2e;
    int mv = max_ctx;
    if (a.window && a.window < mv) mv = a.window;
    const DecodePlan pl = plan_decode(n_seq, a.H, a.Hkv, (int)p->head_dim, mv);
    return run(a, pl, n_seq, (int)p->head_dim, q_dt, true, ws, ws_bytes, st);
}

}  // namespace lmx
