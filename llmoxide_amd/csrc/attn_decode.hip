// Split-K attention for few query tokens (decode): planning and entry points.
// The kernels and their design notes are in attn_decode.hpp.
#include <algorithm>

#include "attn_decode.hpp"

namespace lmx {

// Query heads per wave: the largest divisor of G within the register budget
// (o holds gb * hd/16 floats per lane, K/V tiles grow with hd) and the 16
// MFMA columns (an fp32 query takes two columns per head).  Each head block
// (G / gb of them per kv head) streams the kv head's rows again; at head_dim
// 512 four heads a wave still fit (256 VGPRs + 64 AGPRs, no spills): Gemma 4's
// global layers (16 query heads on one kv head, 32k keys) went from 102 us a
// call at gb 1 to 42 us at gb 4 (55 at gb 2), with the K/V loads cached
// (LMX_DEC_SHARED_HD) so that the XCD's L2 serves part of the repeats.
#ifndef LMX_DEC_GB512
#define LMX_DEC_GB512 4
#endif
static int pick_gb(int G, int hd) {
    const int cap = hd >= 512 ? LMX_DEC_GB512 : (hd == 256 ? 2 : (hd == 128 ? 6 : 8));
    for (int gb = cap; gb >= 1; --gb)
        if (G % gb == 0) return gb;
    return 1;
}

// kv heads per workgroup: the largest power of two <= kWaves dividing Hkv
// (kWaves / hw waves share a head's tiles).  LMX_DECODE_HW = 1, 2 or 4
// overrides it where it divides Hkv, for tuning sweeps.
static int pick_hw(int Hkv) {
    static const int env = [] {
        const char* e = std::getenv("LMX_DECODE_HW");
        const int v = e ? std::atoi(e) : 0;
        return (v == 1 || v == 2 || v == 4) ? v : 0;
    }();
    if (env && Hkv % env == 0) return env;
    for (int hw = kWaves; hw > 1; hw >>= 1)
        if (Hkv % hw == 0) return hw;
    return 1;
}

static size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

constexpr long kCusPerGpu = 256;  // compute units of the target (MI355X)

static long env_long(const char* name, long dflt) {
    const char* e = std::getenv(name);
    const long x = e ? std::atol(e) : 0;
    return x > 0 ? x : dflt;
}

// Workgroups the heuristic aims for, and the fewest tiles a wave should get
// before a unit is split further.  One query row: one 4-wave workgroup per
// CU on 256 CUs, all of them streaming at once.  Several rows (a batch of
// sequences of unequal length): 256 per row and at least eight per CU, so
// that CUs whose workgroups end early pick up queued ones.  Measured on
// ragged 1k-32k batches of Qwen3-8B shape: at B = 8, 2048 beats 256 by 20%
// and 4096 by 6%; at B = 32, 8192 beats 2048 by 28% (500 -> 359 us) and
// 16384 by 5%.  Both optima give a 32k sequence 16-tile waves, as B = 1
// has.  The target stops growing at 16384 (B = 64), which bounds the split
// partials, and so the workspace, for large batches (B = 256 at 32k: 136 MB
// rather than 545 MB).  LMX_DECODE_TARGET_WGS / LMX_DECODE_MIN_TILES
// override them for tuning sweeps.
static long target_wgs(int n_q) {
    static long v = env_long("LMX_DECODE_TARGET_WGS", 0);
    if (v > 0) return v;
    return n_q > 1 ? std::max(2048L, std::min(16384L, 256L * n_q)) : 256;
}
static long min_tiles_per_wave(int hd) {
    static long v = env_long("LMX_DECODE_MIN_TILES", 0);
    if (v > 0) return v;
    // A 16-key tile at head_dim >= 256 is 16 KB of K and V: one per wave puts
    // a short window's whole read in flight at once (Gemma's 1024-key SWA
    // layers: 128 workgroups instead of 64; 11.9 -> 10.5 us a call).  At 128
    // two tiles a wave measured better for the 512-key C1 decode.
    return hd >= 256 ? 1 : 2;
}

// K row-major through LDS (head_dim 128 and 256), or each lane's operand bytes
// loaded directly.  Rows pay wherever the LDS round trip it adds to a tile is
// hidden: by other workgroups on the CU (ragged batches: B=8 116 -> 108 us,
// B=32 358 -> 336 us) or by a short stream (the 512-key C1 decode, 2 tiles a
// wave: 8.05 -> 7.73 us).  One workgroup per CU streaming 16 tiles a wave
// (B=1 at 32k) keeps the direct loads, 1% faster there (27.1 against 27.5 us
// a call).  LMX_DECODE_KROWS=0|1 forces it (tuning overrides, for tests).
static bool pick_krows(int hd, int mode, const DecodePlan& pl) {
    if (hd != 128 && hd != 256) return false;
    if (const int f = tuning().decode_krows; f >= 0) return f == 1;
    const int tiles_per_wave = (pl.tps + kWaves / pl.hw - 1) / (kWaves / pl.hw);
    return mode == kModeBatched || pl.n_main > kCusPerGpu || tiles_per_wave <= 4;
}

// Head_dim 512 with 16 query heads a kv head (Gemma 4's global layers) takes
// attn_decode_mh_kernel: a workgroup serves the 16 heads and every tile of its
// split, each wave a quarter of the output dims.  Splits of at least
// kMhMinTiles tiles (32 KB of K and V each) amortise its Q load.
// LMX_DECODE_MH=0 keeps attn_decode_kernel (tuning overrides, for tests).
constexpr long kMhMinTiles = 4;
static bool use_mh(int G, int hd) { return hd == 512 && G % kMhHeads == 0 && tuning().decode_mh != 0; }

// n_q query rows (tokens or sequences), longest visible range max_vis.
static DecodePlan plan_decode(int n_q, int H, int Hkv, int hd, int max_vis, int mode) {
    DecodePlan pl{};
    const int G = H / Hkv;
    pl.mh = use_mh(G, hd);
    pl.gb = pl.mh ? kMhHeads : pick_gb(G, hd);
    pl.n_hblk = G / pl.gb;
    pl.hw = pl.mh ? 1 : pick_hw(Hkv);
    pl.n_yg = (Hkv / pl.hw) * pl.n_hblk;
    const long units = (long)n_q * pl.n_yg;
    const long n_tiles = (max_vis + kTile - 1) / kTile;
    const long wph = pl.mh ? 1 : kWaves / pl.hw;  // the mh kernel's waves all take every tile
    long P = (target_wgs(n_q) + units - 1) / units;
    const long cap = n_tiles / (wph * (pl.mh ? kMhMinTiles : min_tiles_per_wave(hd)));
    if (P > cap) P = cap;
    if (P > kMaxP) P = kMaxP;
    if (P < 1) P = 1;
    const long tps = (n_tiles + P - 1) / P;
    // The workspace is sized for P before empty splits are dropped: that
    // count grows with the context, the count after dropping does not (12
    // tiles in 5 splits of 3 use 4 splits, 10 tiles in 5 splits of 2 use 5).
    pl.P_ws = (int)P;
    P = (n_tiles + tps - 1) / tps;  // drop splits that would be empty
    pl.P = (int)P;
    pl.tps = (int)tps;
    pl.n_main = (int)(P * units);
    if (P > 1) {
        // Merge layout: parts (a power of two <= 64) lanes per float4 column,
        // so that each folds at most kMergePer partials.
        static const long parts_env = env_long("LMX_DECODE_MERGE_PARTS", 0);
        int parts = 1;
        while (parts * kMergePer < P) parts <<= 1;
        if (parts_env >= parts && parts_env <= 64 && (parts_env & (parts_env - 1)) == 0)
            parts = (int)parts_env;
        pl.m_parts = parts;
        const long cols = (long)n_q * H * (hd / 4);
        pl.n_merge = (int)((cols * parts + kDecThreads - 1) / kDecThreads);
        pl.ml_bytes = round_up((size_t)n_q * H * P * 2 * 4, 256);
        pl.o_bytes = round_up((size_t)n_q * H * P * hd * 4, 256);
    }
    pl.krows = !pl.mh && pick_krows(hd, mode, pl);
    if (pl.P_ws > 1)
        pl.ws_bytes = round_up((size_t)n_q * H * pl.P_ws * 2 * 4, 256) +
                      round_up((size_t)n_q * H * pl.P_ws * hd * 4, 256);
    return pl;
}

// Workspace for up to n_q query rows whose visible ranges are at most
// max_vis keys: the largest need over 1..n_q rows, so that a workspace sized
// for a batch also serves every smaller one (the split count per row falls
// as rows are added, and n_q * P can dip when it does).
static size_t decode_ws_upto(int n_q, int H, int Hkv, int hd, int max_vis) {
    size_t need = 0;
    for (int n = 1; n <= n_q; ++n) need = std::max(need, plan_decode(n, H, Hkv, hd, max_vis, kModeGeneral).ws_bytes);
    return need;
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
    return decode_ws_upto((int)p->n_tokens, (int)p->n_heads, (int)p->n_kv_heads, (int)p->head_dim,
                          decode_max_vis(p));
}

size_t decode_batched_workspace_bytes(const lmx_attn_params* p, int n_seq, int max_ctx) {
    int mv = max_ctx;
    if (p->window && (int)p->window < mv) mv = (int)p->window;
    return decode_ws_upto(n_seq, (int)p->n_heads, (int)p->n_kv_heads, (int)p->head_dim, mv);
}

static lmx_status run(DecodeArgs a, const DecodePlan& pl, int n_q, int hd, lmx_dtype q_dt,
                      int mode, void* ws, size_t ws_bytes, hipStream_t st) {
    if (pl.total() > 0) {
        if (!ws || ws_bytes < pl.total()) return LMX_E_WORKSPACE;
        if (((uintptr_t)ws & 255) != 0) return LMX_E_ALIGN;
        char* b = static_cast<char*>(ws);
        a.part_ml = reinterpret_cast<float*>(b);
        b += pl.ml_bytes;
        a.part_o = reinterpret_cast<float*>(b);
    }
    a.n_q = n_q;
    a.P = pl.P;
    a.tps = pl.tps;
    a.n_hblk = pl.n_hblk;
    a.n_main = pl.n_main;
    a.n_yg = pl.n_yg;
    a.n_merge = pl.n_merge;
    a.m_parts = pl.m_parts;
    window_magic((uint32_t)a.window, &a.w_magic, &a.w_shift);
    (void)hipGetLastError();
    lmx_status s;
    if (q_dt == LMX_F32)
        s = mode == kModeLinear    ? launch_mode<float, kModeLinear>(a, pl, hd, st)
            : mode == kModeGeneral ? launch_mode<float, kModeGeneral>(a, pl, hd, st)
                                   : launch_mode<float, kModeBatched>(a, pl, hd, st);
    else
        s = mode == kModeLinear    ? launch_mode<f16, kModeLinear>(a, pl, hd, st)
            : mode == kModeGeneral ? launch_mode<f16, kModeGeneral>(a, pl, hd, st)
                                   : launch_mode<f16, kModeBatched>(a, pl, hd, st);
    if (s != LMX_OK) return s;
    LMX_CHECK_LAUNCH();
    return LMX_OK;
}

lmx_status decode_fwd(const lmx_attn_params* p, const AttnIo& io, const void* q, lmx_dtype q_dt,
                      const void* k_cache, const void* v_cache, const void* k_cur, const void* v_cur,
                      float* out, void* ws, size_t ws_bytes, hipStream_t st) {
    DecodeArgs a{};
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
    const int mv = decode_max_vis(p);
    // Linear addressing reads row p for every visible p: no k_cur rows and no
    // ring wrap (every visible position is below the window).
    const long last = (long)p->base_pos + p->n_tokens - 1;
    const bool linear = !k_cur && (p->window == 0 || last < (long)p->window);
    const int mode = linear ? kModeLinear : kModeGeneral;
    const DecodePlan pl = plan_decode(a.n_tokens, a.H, a.Hkv, (int)p->head_dim, mv, mode);
    return run(a, pl, a.n_tokens, (int)p->head_dim, q_dt, mode, ws, ws_bytes, st);
}

lmx_status decode_batched(const lmx_attn_params* p, int n_seq, int max_ctx, const int32_t* ctx_lens,
                          const void* const* k_ptrs, const void* const* v_ptrs, const void* q,
                          lmx_dtype q_dt, float* out, void* ws, size_t ws_bytes, hipStream_t st) {
    DecodeArgs a{};
    a.q = q;
    a.q_stride = (int)p->head_dim;
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
    const DecodePlan pl = plan_decode(n_seq, a.H, a.Hkv, (int)p->head_dim, mv, kModeBatched);
    return run(a, pl, n_seq, (int)p->head_dim, q_dt, kModeBatched, ws, ws_bytes, st);
}

}  // namespace lmx
