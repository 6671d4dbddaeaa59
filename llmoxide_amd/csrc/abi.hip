// extern "C" entry points of libllmoxide_amd.so (declared in include/lmx/attn.h).
//
// Every entry point validates its arguments on the host before it enqueues
// anything and reports failures as lmx_status codes, mirroring the reference's
// host-side checks (ensure! on batch and context, qwen35.rs:1212-1222;
// forward.rs:1385-1395) and its error enum (llmoxide/src/error.rs:9-47).
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "common.hpp"

namespace lmx {

// attn_decode.hip
size_t decode_workspace_bytes(const lmx_attn_params* p);
size_t decode_batched_workspace_bytes(const lmx_attn_params* p, int n_seq, int max_ctx);
lmx_status decode_fwd(const lmx_attn_params* p, const AttnIo& io, const void* q, lmx_dtype q_dt,
                      const void* k_cache, const void* v_cache, const void* k_cur, const void* v_cur,
                      float* out, void* ws, size_t ws_bytes, hipStream_t st);
lmx_status decode_batched(const lmx_attn_params* p, int n_seq, int max_ctx, const int32_t* ctx_lens,
                          const void* const* k_ptrs, const void* const* v_ptrs, const void* q,
                          lmx_dtype q_dt, float* out, void* ws, size_t ws_bytes, hipStream_t st);
// attn_prefill.hip
bool prefill_supported(const lmx_attn_params* p, lmx_dtype q_dt);
size_t prefill_workspace_bytes(const lmx_attn_params* p);
lmx_status prefill_fwd(const lmx_attn_params* p, const AttnIo& io, const void* q, lmx_dtype q_dt,
                       const void* k_cache, const void* v_cache, const void* k_cur, const void* v_cur,
                       float* out, void* ws, size_t ws_bytes, hipStream_t st);
// qmatvec.hip
lmx_status qmatvec(const lmx_qmv_desc* d, const void* w, const float* x, float* y, hipStream_t st);
// deltanet.hip
lmx_status deltanet_recur(const lmx_dop* op, const float* ssm_a, const float* dt_bias,
                          const float* alpha, const float* beta, const float* conv, float* state,
                          float* out, hipStream_t st);
size_t deltanet_chunked_ws(const lmx_dop* op, int chunk);
lmx_status deltanet_chunked(const lmx_dop* op, const float* ssm_a, const float* dt_bias,
                            const float* alpha, const float* beta, const float* conv,
                            float* state, float* out, int chunk, void* ws, size_t ws_bytes,
                            hipStream_t st);

// prologue.hip
lmx_status attn_prologue(const lmx_prologue_desc* d, float* q, const float* k_new,
                         const float* v_new, const float* q_gain, const float* k_gain,
                         const float* rope_factors, void* k_cache, void* v_cache,
                         hipStream_t st);

// deltanet_io.hip
lmx_status deltanet_front(const lmx_delta_front_desc* d, const float* x, const float* taps,
                          float* conv_state, float* conv_out, hipStream_t st);
lmx_status deltanet_back(const lmx_delta_back_desc* d, float* o, const float* z, const float* w,
                         hipStream_t st);

// Queries with at most this many tokens take the split-K path; longer
// batches take the MFMA tile path.
constexpr uint32_t kSplitKMaxTokens = 8;

static bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// [a, a + na) and [b, b + nb) share a byte.
static bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
    const char *ca = static_cast<const char*>(a), *cb = static_cast<const char*>(b);
    return ca < cb + nb && cb < ca + na;
}

// attn_pad.hip: head sizes outside the kernels' set, through padded copies
bool native_head_dim(uint32_t hd);
size_t padded_workspace_bytes(const lmx_attn_params* p);
lmx_status padded_attn(const lmx_attn_params* p, const AttnIo& io, const void* q, lmx_dtype q_dt,
                       const void* k_cache, const void* v_cache, const void* k_cur, const void* v_cur,
                       float* out, void* ws, size_t ws_bytes, hipStream_t st);

// head_dim: a multiple of 4 up to 512, the reference's domain (vec4 rows,
// attn.wgsl:36-46).  64, 128, 256 and 512 run natively; the others through
// zero-padded copies at the next of those sizes.  Cache rows are a multiple
// of 8 elements (16-byte loads) at native sizes, of 4 otherwise.
static lmx_status check_attn_params(const lmx_attn_params* p) {
    if (!p) return LMX_E_NULL;
    if (p->n_tokens == 0 || p->n_heads == 0 || p->n_kv_heads == 0) return LMX_E_SHAPE;
    if (p->n_heads % p->n_kv_heads) return LMX_E_SHAPE;
    if (p->head_dim == 0 || p->head_dim > 512 || p->head_dim % 4) return LMX_E_UNSUPPORTED;
    const uint32_t row_align = native_head_dim(p->head_dim) ? 8 : 4;
    if ((uint64_t)p->kv_dim < (uint64_t)p->n_kv_heads * p->head_dim || p->kv_dim % row_align)
        return LMX_E_SHAPE;
    if (!std::isfinite(p->scale)) return LMX_E_SHAPE;
    if (p->bidi > 1) return LMX_E_SHAPE;
    const uint64_t end = (uint64_t)p->base_pos + p->n_tokens;
    if (end >= (1ull << 31)) return LMX_E_CONTEXT;
    if (p->window == 0) {
        if (end > p->n_slots) return LMX_E_CONTEXT;
    } else {
        if (p->n_slots < p->window) return LMX_E_SHAPE;
    }
    return LMX_OK;
}

bool use_split_k(const lmx_attn_params* p, lmx_dtype q_dt) {
    return p->n_tokens <= kSplitKMaxTokens || !prefill_supported(p, q_dt);
}

// Fill kernel for the workspace (a kernel rather than hipMemsetAsync, so it
// can be recorded into a graph).
__global__ void zero_words(uint32_t* p, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

// The same for 16-byte aligned buffers of whole 16-byte words (a KV slab).
// Workgroups run round-robin over the 8 XCDs, so XCD x's workgroups
// (b % 8 == x) take the x-th eighth of the buffer between them, rather than
// the x-th 4 KB of every 32 KB; the grid is a multiple of 8.
__global__ void zero_quads(uint4* p, size_t n) {
    const unsigned per = gridDim.x / 8, xcd = blockIdx.x % 8, local = blockIdx.x / 8;
    const size_t part = (n + 7) / 8, lo = xcd * part, hi = lo + part < n ? lo + part : n;
    for (size_t i = lo + (size_t)local * blockDim.x + threadIdx.x; i < hi; i += (size_t)per * blockDim.x)
        p[i] = uint4{0u, 0u, 0u, 0u};
}

// write_cache (ops.wgsl:323-346): four elements per thread, f32 -> f16 RNE.
// Row i is skipped when row i + window of the same call maps to the same ring
// slot, so the latest position wins as in the reference's in-order store.
__global__ void kv_append_kernel(const float* __restrict__ src, f16* __restrict__ cache,
                                 uint32_t n_tokens, uint32_t kv_dim, uint32_t base_pos,
                                 uint32_t window) {
    const uint32_t per_row = kv_dim / 4;
    const size_t n = (size_t)n_tokens * per_row;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        const uint32_t row = (uint32_t)(i / per_row);
        const uint32_t c4 = (uint32_t)(i - (size_t)row * per_row);
        if (window && row + window < n_tokens) continue;
        const uint32_t pos = base_pos + row;
        const uint32_t slot = window ? pos % window : pos;
        const f32x4 x = *reinterpret_cast<const f32x4*>(src + (size_t)row * kv_dim + 4 * c4);
        f16x4 h;
        h[0] = (f16)x[0];
        h[1] = (f16)x[1];
        h[2] = (f16)x[2];
        h[3] = (f16)x[3];
        *reinterpret_cast<f16x4*>(cache + (size_t)slot * kv_dim + 4 * c4) = h;
    }
}

// Scratch of lmx_attn_fwd_noalloc: the split partials of decode and of a
// key-split prefill, for callers that cannot allocate.  Each GPU the library
// runs on holds one copy for the life of the process.  In host code the name
// `scratch` is only a handle: kernels get the device address that
// hipGetSymbolAddress returns for the current device.
constexpr size_t kScratchBytes = (size_t)LMX_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device

// The copy of `scratch` on the device that `stream` belongs to (the null
// stream: the current device), looked up once per device with that device
// current.  The kernels run on the stream's device, so its copy is the one
// they may touch.
static lmx_status scratch_of_stream_device(hipStream_t stream, void** out) {
    int cur = -1, dev = -1;
    if (hipGetDevice(&cur) != hipSuccess || cur < 0) return LMX_E_DEVICE;
    if (hipStreamGetDevice(stream, &dev) != hipSuccess) return LMX_E_DEVICE;
    if (dev < 0 || dev >= kMaxDevices) return LMX_E_DEVICE;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        if (dev != cur && hipSetDevice(dev) != hipSuccess) return LMX_E_DEVICE;
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch));
        if (dev != cur) (void)hipSetDevice(cur);
        if (e != hipSuccess || !ptr) return LMX_E_DEVICE;
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return LMX_OK;
}

// ---- tuning overrides (see Tuning in common.hpp)
static std::atomic<int> g_tune_kernel{-1}, g_tune_gp{0}, g_tune_kh{-1}, g_tune_krows{-1}, g_tune_mh{-1},
    g_tune_dfused{-1};
static std::once_flag g_tune_once;

static void read_tuning_env() {
    auto choice = [](const char* name, const char* a, int va, const char* b, int vb) {
        const char* e = std::getenv(name);
        if (e && !std::strcmp(e, a)) return va;
        if (e && !std::strcmp(e, b)) return vb;
        return -1;
    };
    g_tune_kernel.store(choice("LMX_PREFILL_KERNEL", "pp", 1, "tile", 0));
    const char* gp = std::getenv("LMX_PREFILL_GP");
    const int g = gp ? std::atoi(gp) : 0;
    g_tune_gp.store((g == 1 || g == 2 || g == 4) ? g : 0);
    const char* kh = std::getenv("LMX_PREFILL_KH");
    g_tune_kh.store(kh && kh[0] == '0' ? 0 : -1);
    g_tune_krows.store(choice("LMX_DECODE_KROWS", "1", 1, "0", 0));
    const char* mh = std::getenv("LMX_DECODE_MH");
    g_tune_mh.store(mh && mh[0] == '0' ? 0 : -1);
    g_tune_dfused.store(choice("LMX_DELTA_FUSED", "0", 0, "starve", 2));
}

Tuning tuning() {
    std::call_once(g_tune_once, read_tuning_env);
    return Tuning{g_tune_kernel.load(), g_tune_gp.load(), g_tune_kh.load(), g_tune_krows.load(), g_tune_mh.load(),
                  g_tune_dfused.load()};
}

}  // namespace lmx

using namespace lmx;

extern "C" {

const char* lmx_status_str(lmx_status s) {
    switch (s) {
        case LMX_OK: return "ok";
        case LMX_E_NULL: return "required pointer is NULL";
        case LMX_E_SHAPE: return "inconsistent or out-of-range geometry";
        case LMX_E_UNSUPPORTED: return "unsupported dtype or head_dim";
        case LMX_E_WORKSPACE: return "workspace missing or too small";
        case LMX_E_CONTEXT: return "positions exceed the cache (context overflow)";
        case LMX_E_RING_HAZARD: return "windowed batch would read ring slots it overwrites; pass k_cur/v_cur";
        case LMX_E_ALIGN: return "pointer misaligned for its layout";
        case LMX_E_LAUNCH: return "HIP launch failed";
        case LMX_E_DEVICE: return "no usable gfx950 device";
        case LMX_E_FULL: return "no free sequence slot";
        case LMX_E_HOST: return "host memory exhausted";
    }
    return "unknown status";
}

int lmx_version(void) { return 106; }

void lmx_tuning_reload(void) {
    std::call_once(g_tune_once, [] {});
    read_tuning_env();
}

lmx_status lmx_workspace_init(void* ws, size_t ws_bytes, lmx_stream stream) {
    if (ws_bytes == 0) return LMX_OK;
    if (!ws) return LMX_E_NULL;
    if (!aligned(ws, 4) || ws_bytes % 4) return LMX_E_ALIGN;
    const bool quads = aligned(ws, 16) && ws_bytes % 16 == 0;
    const size_t n = ws_bytes / (quads ? 16 : 4);
    size_t blocks = (n + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (quads) blocks = (blocks + 7) / 8 * 8;  // zero_quads splits the grid by XCD
    (void)hipGetLastError();
    if (quads)
        hipLaunchKernelGGL(zero_quads, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                           static_cast<uint4*>(ws), n);
    else
        hipLaunchKernelGGL(zero_words, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                           static_cast<uint32_t*>(ws), n);
    LMX_CHECK_LAUNCH();
    return LMX_OK;
}

lmx_status lmx_kv_append(const lmx_kv_desc* d, const float* k_new, const float* v_new,
                         void* k_cache, void* v_cache, lmx_dtype cache_dt, lmx_stream stream) {
    if (!d) return LMX_E_NULL;
    if (cache_dt != LMX_F16) return LMX_E_UNSUPPORTED;
    if ((k_new == nullptr) != (k_cache == nullptr) || (v_new == nullptr) != (v_cache == nullptr))
        return LMX_E_NULL;
    if (!k_new && !v_new) return LMX_E_NULL;
    if (d->n_tokens == 0 || d->kv_dim == 0 || d->kv_dim % 4) return LMX_E_SHAPE;
    const uint64_t end = (uint64_t)d->base_pos + d->n_tokens;
    if (end >= (1ull << 32)) return LMX_E_CONTEXT;
    if (d->window == 0) {
        if (end > d->n_slots) return LMX_E_CONTEXT;
    } else if (d->n_slots < d->window) {
        return LMX_E_SHAPE;
    }
    for (const void* p : {(const void*)k_new, (const void*)v_new})
        if (p && !aligned(p, 16)) return LMX_E_ALIGN;
    for (const void* p : {(const void*)k_cache, (const void*)v_cache})
        if (p && !aligned(p, 8)) return LMX_E_ALIGN;
    const size_t n = (size_t)d->n_tokens * (d->kv_dim / 4);
    size_t blocks = (n + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    (void)hipGetLastError();
    if (k_new)
        hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                           k_new, static_cast<f16*>(k_cache), d->n_tokens, d->kv_dim, d->base_pos,
                           d->window);
    if (v_new)
        hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                           v_new, static_cast<f16*>(v_cache), d->n_tokens, d->kv_dim, d->base_pos,
                           d->window);
    LMX_CHECK_LAUNCH();
    return LMX_OK;
}

lmx_status lmx_attn_prologue(const lmx_prologue_desc* d, float* q, const float* k_new,
                             const float* v_new, const float* q_gain, const float* k_gain,
                             const float* rope_factors, void* k_cache, void* v_cache,
                             lmx_dtype cache_dt, lmx_stream stream) {
    if (!d || !q || !k_new || !v_new || !k_cache || !v_cache) return LMX_E_NULL;
    if (cache_dt != LMX_F16) return LMX_E_UNSUPPORTED;
    if (d->n_tokens == 0 || d->n_heads == 0 || d->n_kv_heads == 0) return LMX_E_SHAPE;
    const uint32_t hd = d->head_dim;
    if (hd != 64 && hd != 128 && hd != 256 && hd != 512) return LMX_E_UNSUPPORTED;
    if (d->n_rot % 2 || d->n_rot > hd || d->q_stride < hd) return LMX_E_SHAPE;
    if (d->n_rot && !(d->rope_base > 0.f)) return LMX_E_SHAPE;
    if (!(d->rms_eps >= 0.f)) return LMX_E_SHAPE;
    const uint64_t end = (uint64_t)d->base_pos + d->n_tokens;
    if (end >= (1ull << 31)) return LMX_E_CONTEXT;
    if (d->window == 0) {
        if (end > d->n_slots) return LMX_E_CONTEXT;
    } else if (d->n_slots < d->window) {
        return LMX_E_SHAPE;
    }
    if ((uint64_t)d->n_heads * d->q_stride * d->n_tokens >= (1ull << 31) ||
        (uint64_t)d->n_kv_heads * hd * (end > d->n_slots ? end : d->n_slots) >= (1ull << 31))
        return LMX_E_SHAPE;
    for (const void* p : {(const void*)q, (const void*)k_new, (const void*)v_new,
                          (const void*)q_gain, (const void*)k_gain, (const void*)rope_factors})
        if (p && !aligned(p, 4)) return LMX_E_ALIGN;
    for (const void* p : {(const void*)k_cache, (const void*)v_cache})
        if (!aligned(p, 2)) return LMX_E_ALIGN;
    return attn_prologue(d, q, k_new, v_new, q_gain, k_gain, rope_factors, k_cache, v_cache,
                         (hipStream_t)stream);
}

size_t lmx_attn_workspace_bytes(const lmx_attn_params* p) {
    if (check_attn_params(p) != LMX_OK) return 0;
    if (!native_head_dim(p->head_dim)) return padded_workspace_bytes(p);
    // The split-K decode path and a key-split prefill use a workspace; the
    // size covers whichever path either query dtype takes.
    size_t need = 0;
    for (lmx_dtype dt : {LMX_F32, LMX_F16}) {
        const size_t b = use_split_k(p, dt) ? decode_workspace_bytes(p) : prefill_workspace_bytes(p);
        if (b > need) need = b;
    }
    return need;
}

lmx_status lmx_attn_fwd(const lmx_attn_params* p, const void* q, lmx_dtype q_dt,
                        const void* k_cache, const void* v_cache, lmx_dtype kv_dt,
                        const void* k_cur, const void* v_cur, float* out, void* ws,
                        size_t ws_bytes, lmx_stream stream) {
    return lmx_attn_fwd_ext(p, nullptr, q, q_dt, k_cache, v_cache, kv_dt, k_cur, v_cur, out, ws,
                            ws_bytes, stream);
}

lmx_status lmx_attn_fwd_ext(const lmx_attn_params* p, const lmx_attn_ext* x, const void* q,
                            lmx_dtype q_dt, const void* k_cache, const void* v_cache,
                            lmx_dtype kv_dt, const void* k_cur, const void* v_cur, float* out,
                            void* ws, size_t ws_bytes, lmx_stream stream) {
    lmx_status s = check_attn_params(p);
    if (s != LMX_OK) return s;
    if (q_dt != LMX_F32 && q_dt != LMX_F16) return LMX_E_UNSUPPORTED;
    if (kv_dt != LMX_F16) return LMX_E_UNSUPPORTED;
    if (!q || !k_cache || !v_cache || !out) return LMX_E_NULL;
    if ((k_cur == nullptr) != (v_cur == nullptr)) return LMX_E_NULL;
    if (p->window && p->n_tokens > 1 && (uint64_t)p->base_pos + p->n_tokens > p->window && !k_cur)
        return LMX_E_RING_HAZARD;
    // native sizes: 16-byte rows; padded ones are copied in 4-element pieces
    const bool native = native_head_dim(p->head_dim);
    const size_t qa = native || q_dt == LMX_F32 ? 16 : 8, ca = native ? 16 : 8;
    if (!aligned(q, qa) || !aligned(k_cache, ca) || !aligned(v_cache, ca) || !aligned(out, 16))
        return LMX_E_ALIGN;
    if (k_cur && (!aligned(k_cur, ca) || !aligned(v_cur, ca))) return LMX_E_ALIGN;
    const uint32_t hd = p->head_dim;
    const uint32_t qs = x && x->q_stride ? x->q_stride : hd;
    const uint32_t gs = x && x->gate_stride ? x->gate_stride : hd;
    const float* gate = x ? x->gate : nullptr;
    if (qs < hd || qs % (native ? 8 : 4) || gs < hd || gs % 4) return LMX_E_SHAPE;
    if ((uint64_t)p->n_tokens * p->n_heads * qs > INT32_MAX ||
        (uint64_t)p->n_tokens * p->n_heads * gs > INT32_MAX)
        return LMX_E_SHAPE;
    if (gate && !aligned(gate, 16)) return LMX_E_ALIGN;
    // out must not overlap what the kernels read after another workgroup
    // may have written it: the queries and the gate
    const size_t q_bytes = ((size_t)p->n_tokens * p->n_heads - 1) * qs * (q_dt == LMX_F32 ? 4 : 2) +
                           (size_t)hd * (q_dt == LMX_F32 ? 4 : 2);
    const size_t o_bytes = (size_t)p->n_tokens * p->n_heads * hd * 4;
    if (overlaps(out, o_bytes, q, q_bytes)) return LMX_E_SHAPE;
    if (gate && overlaps(out, o_bytes, gate, (((size_t)p->n_tokens * p->n_heads - 1) * gs + hd) * 4))
        return LMX_E_SHAPE;
    const AttnIo io{(int)qs, (int)gs, gate};
    if (!native)
        return padded_attn(p, io, q, q_dt, k_cache, v_cache, k_cur, v_cur, out, ws, ws_bytes,
                           (hipStream_t)stream);
    if (use_split_k(p, q_dt))
        return decode_fwd(p, io, q, q_dt, k_cache, v_cache, k_cur, v_cur, out, ws, ws_bytes,
                          (hipStream_t)stream);
    return prefill_fwd(p, io, q, q_dt, k_cache, v_cache, k_cur, v_cur, out, ws, ws_bytes,
                       (hipStream_t)stream);
}

lmx_status lmx_attn_fwd_noalloc(const lmx_attn_params* p, const void* q, lmx_dtype q_dt,
                                const void* k_cache, const void* v_cache, lmx_dtype kv_dt,
                                const void* k_cur, const void* v_cur, float* out,
                                lmx_stream stream) {
    lmx_status s = check_attn_params(p);
    if (s != LMX_OK) return s;
    const size_t need = lmx_attn_workspace_bytes(p);
    if (need > kScratchBytes) return LMX_E_WORKSPACE;
    void* ws = nullptr;
    if (need > 0) {
        s = scratch_of_stream_device((hipStream_t)stream, &ws);
        if (s != LMX_OK) return s;
    }
    return lmx_attn_fwd_ext(p, nullptr, q, q_dt, k_cache, v_cache, kv_dt, k_cur, v_cur, out, ws,
                            need > 0 ? kScratchBytes : 0, stream);
}

size_t lmx_attn_decode_batched_workspace_bytes(const lmx_attn_params* p, int32_t n_seq,
                                               int32_t max_ctx) {
    if (!p || n_seq < 1 || max_ctx < 1) return 0;
    if (!p->n_kv_heads || !p->n_heads || p->n_heads % p->n_kv_heads) return 0;
    return decode_batched_workspace_bytes(p, n_seq, max_ctx);
}

lmx_status lmx_attn_decode_batched(const lmx_attn_params* p, int32_t n_seq, int32_t max_ctx,
                                   const int32_t* ctx_lens, const void* const* k_ptrs,
                                   const void* const* v_ptrs, const void* q, lmx_dtype q_dt,
                                   lmx_dtype kv_dt, float* out, void* ws, size_t ws_bytes,
                                   lmx_stream stream) {
    if (!p) return LMX_E_NULL;
    if (p->n_tokens != 1 || n_seq < 1 || max_ctx < 1) return LMX_E_SHAPE;
    lmx_attn_params pp = *p;
    pp.base_pos = 0;
    lmx_status s = check_attn_params(&pp);
    if (s != LMX_OK) return s;
    if (!native_head_dim(p->head_dim)) return LMX_E_UNSUPPORTED;  // no padded batched path
    if (p->bidi) return LMX_E_SHAPE;
    if (p->window == 0 && (uint32_t)max_ctx > p->n_slots) return LMX_E_CONTEXT;
    if (q_dt != LMX_F32 && q_dt != LMX_F16) return LMX_E_UNSUPPORTED;
    if (kv_dt != LMX_F16) return LMX_E_UNSUPPORTED;
    if (!ctx_lens || !k_ptrs || !v_ptrs || !q || !out) return LMX_E_NULL;
    if (!aligned(q, 16) || !aligned(out, 16) || !aligned(k_ptrs, 8) || !aligned(v_ptrs, 8) ||
        !aligned(ctx_lens, 4))
        return LMX_E_ALIGN;
    return decode_batched(p, n_seq, max_ctx, ctx_lens, k_ptrs, v_ptrs, q, q_dt, out, ws, ws_bytes,
                          (hipStream_t)stream);
}

static lmx_status check_dop(const lmx_dop* op) {
    if (!op) return LMX_E_NULL;
    if (!op->n_tok || !op->n_vh || !op->n_kh || !op->s_dim) return LMX_E_SHAPE;
    if (op->s_dim != 128 && op->s_dim != 64) return LMX_E_UNSUPPORTED;
    if (op->key_dim != op->n_kh * op->s_dim || op->d_inner != op->n_vh * op->s_dim) return LMX_E_SHAPE;
    if (op->conv_dim < 2 * op->key_dim + op->d_inner || op->conv_dim % 4) return LMX_E_SHAPE;
    if (!std::isfinite(op->scale)) return LMX_E_SHAPE;
    return LMX_OK;
}

lmx_status lmx_deltanet_recur(const lmx_dop* op, const float* ssm_a, const float* dt_bias,
                              const float* alpha, const float* beta, const float* conv,
                              float* state, float* out, lmx_stream stream) {
    lmx_status s = check_dop(op);
    if (s != LMX_OK) return s;
    if (!ssm_a || !dt_bias || !alpha || !beta || !conv || !state || !out) return LMX_E_NULL;
    if (!aligned(conv, 16) || !aligned(state, 16) || !aligned(out, 16)) return LMX_E_ALIGN;
    return deltanet_recur(op, ssm_a, dt_bias, alpha, beta, conv, state, out, (hipStream_t)stream);
}

size_t lmx_deltanet_chunked_workspace_bytes(const lmx_dop* op, int32_t chunk) {
    if (check_dop(op) != LMX_OK) return 0;
    if (chunk != 16 && chunk != 32 && chunk != 64) return 0;
    return deltanet_chunked_ws(op, chunk);
}

lmx_status lmx_deltanet_chunked(const lmx_dop* op, const float* ssm_a, const float* dt_bias,
                                const float* alpha, const float* beta, const float* conv,
                                float* state, float* out, int32_t chunk, void* ws,
                                size_t ws_bytes, lmx_stream stream) {
    lmx_status s = check_dop(op);
    if (s != LMX_OK) return s;
    if (chunk != 16 && chunk != 32 && chunk != 64) return LMX_E_SHAPE;
    if (!ssm_a || !dt_bias || !alpha || !beta || !conv || !state || !out) return LMX_E_NULL;
    if (!aligned(conv, 16) || !aligned(state, 16) || !aligned(out, 16)) return LMX_E_ALIGN;
    const size_t need = deltanet_chunked_ws(op, chunk);
    if (need > 0) {
        if (!ws || ws_bytes < need) return LMX_E_WORKSPACE;
        if (!aligned(ws, 256)) return LMX_E_ALIGN;
    }
    return deltanet_chunked(op, ssm_a, dt_bias, alpha, beta, conv, state, out, chunk, ws, ws_bytes,
                            (hipStream_t)stream);
}

lmx_status lmx_deltanet_front(const lmx_delta_front_desc* d, const float* x, const float* taps,
                              float* conv_state, float* conv_out, lmx_stream stream) {
    if (!d || !x || !taps || !conv_state || !conv_out) return LMX_E_NULL;
    if (d->n_tok == 0 || d->conv_dim == 0 || d->conv_dim % 128) return LMX_E_SHAPE;
    if (d->s_dim != 64 && d->s_dim != 128) return LMX_E_UNSUPPORTED;
    if (d->key_dim == 0 || d->key_dim % d->s_dim || 2ull * d->key_dim > d->conv_dim) return LMX_E_SHAPE;
    if (d->kernel < 2 || d->kernel > 8) return LMX_E_UNSUPPORTED;
    if (!(d->eps >= 0.f) || d->eps == INFINITY) return LMX_E_SHAPE;
    if ((uint64_t)d->n_tok * d->conv_dim >= (1ull << 31)) return LMX_E_SHAPE;
    for (const void* p : {(const void*)x, (const void*)taps, (const void*)conv_state,
                          (const void*)conv_out})
        if (!aligned(p, 4)) return LMX_E_ALIGN;
    // the batch rows are read by later tokens' taps: the output must not overlay them
    const size_t bytes = (size_t)d->n_tok * d->conv_dim * sizeof(float);
    if (overlaps(conv_out, bytes, x, bytes)) return LMX_E_SHAPE;
    return deltanet_front(d, x, taps, conv_state, conv_out, (hipStream_t)stream);
}

lmx_status lmx_deltanet_back(const lmx_delta_back_desc* d, float* o, const float* z,
                             const float* w, lmx_stream stream) {
    if (!d || !o || !z || !w) return LMX_E_NULL;
    if (d->n_tok == 0 || d->n_vh == 0) return LMX_E_SHAPE;
    if (d->s_dim != 64 && d->s_dim != 128 && d->s_dim != 256) return LMX_E_UNSUPPORTED;
    if (!(d->eps >= 0.f) || d->eps == INFINITY) return LMX_E_SHAPE;
    if ((uint64_t)d->n_tok * d->n_vh * d->s_dim >= (1ull << 31)) return LMX_E_SHAPE;
    for (const void* p : {(const void*)o, (const void*)z, (const void*)w})
        if (!aligned(p, 4)) return LMX_E_ALIGN;
    return deltanet_back(d, o, z, w, (hipStream_t)stream);
}

lmx_status lmx_matvec(const lmx_qmv_desc* d, const void* w, const float* x, float* y,
                      lmx_stream stream) {
    if (!d || !w || !x || !y) return LMX_E_NULL;
    if (d->rows == 0 || d->n_tok == 0 || d->in_dim == 0) return LMX_E_SHAPE;
    uint32_t mult = 0;
    size_t bb = 0, be = 1;
    switch (d->type) {
        case 12: mult = 256; bb = 144; be = 256; break;
        case 14: mult = 256; bb = 210; be = 256; break;
        case 8: mult = 64; bb = 34; be = 32; break;
        case 0: mult = 64; bb = 4; break;
        case 1: case 30: mult = 64; bb = 2; break;
        default: return LMX_E_UNSUPPORTED;
    }
    if (d->in_dim % mult || d->in_dim > 16384) return LMX_E_SHAPE;
    if (!aligned(w, 16) || !aligned(x, 16) || !aligned(y, 16)) return LMX_E_ALIGN;
    const size_t wb = (size_t)d->rows * (d->in_dim / be) * bb;
    const size_t xb = (size_t)d->n_tok * d->in_dim * 4, yb = (size_t)d->n_tok * d->rows * 4;
    if (overlaps(y, yb, x, xb) || overlaps(y, yb, w, wb)) return LMX_E_SHAPE;
    return qmatvec(d, w, x, y, (hipStream_t)stream);
}

}  // extern "C"
