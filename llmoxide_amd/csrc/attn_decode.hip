// Split-K attention for few query tokens (decode) on gfx950.
//
// Replaces, for n_tokens small, the reference's three passes scores_pass /
// softmax_pass / weighted_v (attn.wgsl:84-232), which give decode only
// n_heads workgroups and a serial key loop (attn.wgsl:13-17).  Here the key
// range of every (query, kv-head) is split over many workgroups; each reads
// its K/V slice once for all GB query heads that share the kv head (GQA), so
// K/V bytes cross HBM once.  Scores never leave registers: an online softmax
// keeps (max, sum, o[hd]) per head, partials are merged in LDS, and the last
// workgroup to finish a (query, kv-head) merges the split partials.
//
// Lane layout (wave64 = four 16-lane DPP rows): lane (row r, col c) of wave w
// owns key slot rs = 4w + r and dims [c*hd/16, (c+1)*hd/16).  One vector load
// per lane fetches hd/16 f16, so a row reads one key's contiguous hd*2-byte
// head slice and a wave reads four such slices per instruction.  The q.k dot
// is finished with four DPP row adds (row_sum16).
#include <climits>

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
    float* part_o;       // [n_q][H][n_splits][HD]
    float* part_ml;      // [n_q][H][n_splits][2]  (max in log2 units, sum)
    uint32_t* counters;  // [n_q][Hkv][n_hblk]
    int H, Hkv, G, kv_dim;
    int base_pos, window, n_tokens, bidi;
    int n_splits, chunk, n_hblk;
    int max_ctx;  // batched: context lengths are clamped to [1, max_ctx]
    float c;      // scale * log2(e)
};

constexpr int kDecThreads = 256;
constexpr int kMaxSplits = 1024;

__device__ __forceinline__ float block_max256(float x, float* red) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) x = fmaxf(x, shfl_xor(x, m));
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = x;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__device__ __forceinline__ float block_sum256(float x, float* red) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) x += shfl_xor(x, m);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = x;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

template <typename QT, int HD, int GB, int U, bool BATCHED>
__global__ __launch_bounds__(kDecThreads) void attn_decode_kernel(DecodeArgs a) {
    constexpr int DPL = HD / 16;
    const int split = blockIdx.x;
    const int kvh = blockIdx.y / a.n_hblk;
    const int hb = blockIdx.y - kvh * a.n_hblk;
    const int qi = blockIdx.z;
    const int h0 = kvh * a.G + hb * GB;

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
    const int n_vis = hi - lo + 1;
    const int ns = (n_vis + a.chunk - 1) / a.chunk;
    if (split >= ns) return;  // uniform: this split lies past the visible range
    const int k0 = lo + split * a.chunk;
    const int k1 = min(k0 + a.chunk, hi + 1);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row = lane >> 4, col = lane & 15;
    const int rs = wave * 4 + row;
    const int hoff = kvh * HD + col * DPL;

    float q[GB][DPL];
#pragma unroll
    for (int g = 0; g < GB; ++g) {
        const size_t qo = ((size_t)qi * a.H + h0 + g) * HD + col * DPL;
        if constexpr (sizeof(QT) == 4)
            load_f32<DPL>(reinterpret_cast<const float*>(a.q) + qo, q[g]);
        else
            load_f16_as_f32<DPL>(reinterpret_cast<const f16*>(a.q) + qo, q[g]);
    }

    float m[GB], l[GB], o[GB][DPL];
#pragma unroll
    for (int g = 0; g < GB; ++g) {
        m[g] = -1e30f;
        l[g] = 0.f;
#pragma unroll
        for (int d = 0; d < DPL; ++d) o[g][d] = 0.f;
    }

    const int w = a.window;
    const int s_base = w ? k0 % w : 0;

    for (int j0 = 0; k0 + 16 * j0 < k1; j0 += U) {
        RawF16<DPL> kr[U], vr[U];
        bool valid[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int off = rs + 16 * (j0 + u);
            valid[u] = k0 + off < k1;
            const int o_c = valid[u] ? off : 0;
            const int p = k0 + o_c;
            const f16 *kp, *vp;
            if (p >= cur_begin) {
                const size_t r = (size_t)(p - a.base_pos) * a.kv_dim + hoff;
                kp = a.k_cur + r;
                vp = a.v_cur + r;
            } else {
                int s = p;
                if (w) {
                    s = s_base + o_c;
                    if (s >= w) s -= w;
                    if (s >= w) s %= w;
                }
                const size_t r = (size_t)s * a.kv_dim + hoff;
                kp = kc + r;
                vp = vc + r;
            }
            load_raw<DPL>(kp, kr[u]);
            load_raw<DPL>(vp, vr[u]);
        }

        float s[GB][U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int g = 0; g < GB; ++g) {
                float acc = 0.f;
#pragma unroll
                for (int d = 0; d < DPL; ++d) acc = fmaf(q[g][d], raw_at<DPL>(kr[u], d), acc);
                acc = row_sum16(acc) * a.c;
                s[g][u] = valid[u] ? acc : -INFINITY;
            }
        }
#pragma unroll
        for (int g = 0; g < GB; ++g) {
            float mb = s[g][0];
#pragma unroll
            for (int u = 1; u < U; ++u) mb = fmaxf(mb, s[g][u]);
            const float mn = fmaxf(m[g], mb);
            const float corr = fast_exp2(m[g] - mn);
            m[g] = mn;
            l[g] *= corr;
#pragma unroll
            for (int d = 0; d < DPL; ++d) o[g][d] *= corr;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float p = fast_exp2(s[g][u] - mn);
                l[g] += p;
#pragma unroll
                for (int d = 0; d < DPL; ++d) o[g][d] = fmaf(p, raw_at<DPL>(vr[u], d), o[g][d]);
            }
        }
    }

    // Merge the four rows of each wave (lanes c, c+16, c+32, c+48 hold the
    // same dims for different key slots).
#pragma unroll
    for (int g = 0; g < GB; ++g) {
        float M = fmaxf(m[g], shfl_xor(m[g], 16));
        M = fmaxf(M, shfl_xor(M, 32));
        const float sc = fast_exp2(m[g] - M);
        float L = l[g] * sc;
        L += shfl_xor(L, 16);
        L += shfl_xor(L, 32);
#pragma unroll
        for (int d = 0; d < DPL; ++d) {
            float x = o[g][d] * sc;
            x += shfl_xor(x, 16);
            x += shfl_xor(x, 32);
            o[g][d] = x;
        }
        m[g] = M;
        l[g] = L;
    }

    __shared__ float sm_o[4][GB][HD];
    __shared__ float sm_m[4][GB];
    __shared__ float sm_l[4][GB];
    if (row == 0) {
#pragma unroll
        for (int g = 0; g < GB; ++g) {
#pragma unroll
            for (int d = 0; d < DPL; ++d) sm_o[wave][g][col * DPL + d] = o[g][d];
            if (col == 0) {
                sm_m[wave][g] = m[g];
                sm_l[wave][g] = l[g];
            }
        }
    }
    __syncthreads();

    const int n_q_heads = a.H;
    for (int idx = tid; idx < GB * HD; idx += kDecThreads) {
        const int g = idx / HD, d = idx - g * HD;
        const float M = fmaxf(fmaxf(sm_m[0][g], sm_m[1][g]), fmaxf(sm_m[2][g], sm_m[3][g]));
        float O = 0.f, L = 0.f;
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {
            const float sc = fast_exp2(sm_m[ww][g] - M);
            O = fmaf(sm_o[ww][g][d], sc, O);
            L = fmaf(sm_l[ww][g], sc, L);
        }
        const size_t qh = (size_t)qi * n_q_heads + h0 + g;
        if (ns == 1) {
            a.out[qh * HD + d] = O / L;
        } else {
            const size_t pidx = qh * a.n_splits + split;
            a.part_o[pidx * HD + d] = O;
            if (d == 0) {
                a.part_ml[pidx * 2] = M;
                a.part_ml[pidx * 2 + 1] = L;
            }
        }
    }
    if (ns == 1) return;

    // Publish the partial, then let the last workgroup of this (query,
    // kv-head, head-block) merge all splits.
    __threadfence();
    __syncthreads();
    __shared__ int s_last;
    uint32_t* ctr = a.counters + ((size_t)qi * a.Hkv + kvh) * a.n_hblk + hb;
    if (tid == 0) {
        const uint32_t old =
            __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (old == (uint32_t)(ns - 1));
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    __shared__ float sw[GB][kMaxSplits];
    __shared__ float sM[GB], sL[GB];
    __shared__ float red[4];
#pragma unroll
    for (int g = 0; g < GB; ++g) {
        const size_t qh = (size_t)qi * n_q_heads + h0 + g;
        const float* ml = a.part_ml + qh * a.n_splits * 2;
        float mx = -1e30f;
        for (int s2 = tid; s2 < ns; s2 += kDecThreads) mx = fmaxf(mx, ml[s2 * 2]);
        const float M = block_max256(mx, red);
        float lsum = 0.f;
        for (int s2 = tid; s2 < ns; s2 += kDecThreads) {
            const float wgt = fast_exp2(ml[s2 * 2] - M);
            sw[g][s2] = wgt;
            lsum = fmaf(wgt, ml[s2 * 2 + 1], lsum);
        }
        const float L = block_sum256(lsum, red);
        if (tid == 0) {
            sM[g] = M;
            sL[g] = L;
        }
    }
    __syncthreads();
    for (int idx = tid; idx < GB * HD; idx += kDecThreads) {
        const int g = idx / HD, d = idx - g * HD;
        const size_t qh = (size_t)qi * n_q_heads + h0 + g;
        const float* po = a.part_o + qh * a.n_splits * HD + d;
        float acc = 0.f;
        for (int s2 = 0; s2 < ns; ++s2) acc = fmaf(sw[g][s2], po[(size_t)s2 * HD], acc);
        a.out[qh * HD + d] = acc / sL[g];
    }
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------ host --

struct DecodePlan {
    int n_splits, chunk, n_hblk, gb;
    size_t ctr_bytes, ml_bytes, o_bytes;
    size_t total() const { return ctr_bytes + ml_bytes + o_bytes; }
};

static int pick_gb(int G, int hd) {
    const int cap = hd >= 512 ? 2 : 4;
    for (int gb = cap; gb >= 1; --gb)
        if (G % gb == 0) return gb;
    return 1;
}

static size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// n_q query rows (tokens or sequences), longest visible range max_vis.
static DecodePlan plan_decode(int n_q, int H, int Hkv, int hd, int max_vis) {
    DecodePlan pl{};
    const int G = H / Hkv;
    pl.gb = pick_gb(G, hd);
    pl.n_hblk = G / pl.gb;
    const long par = (long)n_q * Hkv * pl.n_hblk;
    const long target = 1024;  // about four workgroups per CU on 256 CUs
    long ns = (target + par - 1) / par;
    const long max_ns = (max_vis + 63) / 64;
    if (ns > max_ns) ns = max_ns;
    if (ns > kMaxSplits) ns = kMaxSplits;
    if (ns < 1) ns = 1;
    long chunk = (max_vis + ns - 1) / ns;
    chunk = (chunk + 63) / 64 * 64;
    ns = (max_vis + chunk - 1) / chunk;
    pl.n_splits = (int)ns;
    pl.chunk = (int)chunk;
    if (pl.n_splits > 1) {
        pl.ctr_bytes = round_up((size_t)n_q * Hkv * pl.n_hblk * 4, 256);
        pl.ml_bytes = round_up((size_t)n_q * H * pl.n_splits * 2 * 4, 256);
        pl.o_bytes = round_up((size_t)n_q * H * pl.n_splits * hd * 4, 256);
    }
    return pl;
}

template <typename QT, int HD, int GB, bool BATCHED>
static void launch_hd(const DecodeArgs& a, dim3 grid, hipStream_t st) {
    constexpr int U = HD <= 128 ? 8 : (HD == 256 ? 4 : 2);
    hipLaunchKernelGGL((attn_decode_kernel<QT, HD, GB, U, BATCHED>), grid, dim3(kDecThreads), 0, st, a);
}

template <typename QT, bool BATCHED>
static lmx_status launch_decode(const DecodeArgs& a, int hd, int gb, dim3 grid, hipStream_t st) {
#define LMX_DEC_CASE(HDV, GBV)                                       \
    if (hd == HDV && gb == GBV) {                                    \
        launch_hd<QT, HDV, GBV, BATCHED>(a, grid, st);               \
        return LMX_OK;                                               \
    }
    LMX_DEC_CASE(64, 1) LMX_DEC_CASE(64, 2) LMX_DEC_CASE(64, 3) LMX_DEC_CASE(64, 4)
    LMX_DEC_CASE(128, 1) LMX_DEC_CASE(128, 2) LMX_DEC_CASE(128, 3) LMX_DEC_CASE(128, 4)
    LMX_DEC_CASE(256, 1) LMX_DEC_CASE(256, 2) LMX_DEC_CASE(256, 3) LMX_DEC_CASE(256, 4)
    LMX_DEC_CASE(512, 1) LMX_DEC_CASE(512, 2)
#undef LMX_DEC_CASE
    return LMX_E_UNSUPPORTED;
}

// Longest visible range over the batch's queries (closed form of
// attn.wgsl:52-66 maximized over the tokens).
int decode_max_vis(const lmx_attn_params* p) {
    long best = 0;
    const long t = p->n_tokens, base = p->base_pos, w = p->window;
    // The longest range belongs to the last token causally, but with bidi a
    // middle token can see further; scanning is O(t) and t is small here.
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
        if (!ws) return LMX_E_WORKSPACE;
        if (ws_bytes < pl.total()) return LMX_E_WORKSPACE;
        if (((uintptr_t)ws & 255) != 0) return LMX_E_ALIGN;
        char* b = static_cast<char*>(ws);
        a.counters = reinterpret_cast<uint32_t*>(b);
        a.part_ml = reinterpret_cast<float*>(b + pl.ctr_bytes);
        a.part_o = reinterpret_cast<float*>(b + pl.ctr_bytes + pl.ml_bytes);
    }
    a.n_splits = pl.n_splits;
    a.chunk = pl.chunk;
    a.n_hblk = pl.n_hblk;
    dim3 grid(pl.n_splits, a.Hkv * pl.n_hblk, n_q);
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
