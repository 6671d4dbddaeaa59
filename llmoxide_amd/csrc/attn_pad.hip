// Attention at head sizes outside the kernels' set (64, 128, 256, 512).
//
// The reference's attention takes any head_dim that is a multiple of 4 up to
// 512: its passes work on vec4 rows with room for 128 of them
// (attn.wgsl:36-46), and its vision tower calls them with head_dim =
// embedding_length / head_count (crates/model/src/vision.rs:77-86;
// crates/gpu/src/vision.rs:587-631, bidirectional, scale 1.0).  Here such a
// call runs the kernels of the next native size HP on zero-padded copies
// held in the caller's workspace:
//
//   Q    [t][H][HP]            the query dtype; dims >= head_dim are 0
//   K, V [rows][Hkv][HP] f16   the cache rows the call can read (the
//                              window's ring slots, or positions below
//                              base_pos + t); K's pad is 0
//   K, V [t][Hkv][HP] f16      the batch's own rows (k_cur / v_cur), if given
//   out  [t][H][HP] fp32
//
// With Q's padded dims zero every score is the unpadded one, so the softmax
// and the first head_dim dims of the output are those of the unpadded call.
// Those dims are copied to the caller's out, where the output gate, if any,
// is applied.  The copies are HBM-bound passes of their own (read + write of
// each padded buffer); the attention kernels run as at the native size.
#include "common.hpp"

namespace lmx {

lmx_status decode_fwd(const lmx_attn_params* p, const AttnIo& io, const void* q, lmx_dtype q_dt,
                      const void* k_cache, const void* v_cache, const void* k_cur, const void* v_cur,
                      float* out, void* ws, size_t ws_bytes, hipStream_t st);
lmx_status prefill_fwd(const lmx_attn_params* p, const AttnIo& io, const void* q, lmx_dtype q_dt,
                       const void* k_cache, const void* v_cache, const void* k_cur, const void* v_cur,
                       float* out, void* ws, size_t ws_bytes, hipStream_t st);
size_t decode_workspace_bytes(const lmx_attn_params* p);
size_t prefill_workspace_bytes(const lmx_attn_params* p);
bool use_split_k(const lmx_attn_params* p, lmx_dtype q_dt);

bool native_head_dim(uint32_t hd) { return hd == 64 || hd == 128 || hd == 256 || hd == 512; }
uint32_t padded_head_dim(uint32_t hd) { return hd <= 64 ? 64 : hd <= 128 ? 128 : hd <= 256 ? 256 : 512; }

// Rows the call reads from the cache: the ring's window slots, or every
// position below base_pos + t of a linear cache.
static uint32_t cache_rows(const lmx_attn_params* p) {
    if (p->window) return p->window;
    const uint64_t end = (uint64_t)p->base_pos + p->n_tokens;
    return (uint32_t)(end < p->n_slots ? end : p->n_slots);
}

static size_t up256(size_t x) { return (x + 255) / 256 * 256; }

// The native-size parameters of a padded call.
static lmx_attn_params padded_params(const lmx_attn_params* p) {
    lmx_attn_params pp = *p;
    pp.head_dim = padded_head_dim(p->head_dim);
    pp.kv_dim = p->n_kv_heads * pp.head_dim;
    pp.n_slots = cache_rows(p);
    return pp;
}

struct PadLayout {
    size_t inner, q, kv, cur, out, total;  // byte offsets of each buffer, and the total
};

static PadLayout pad_layout(const lmx_attn_params* p) {
    const lmx_attn_params pp = padded_params(p);
    const size_t hp = pp.head_dim;
    size_t inner = 0;
    for (lmx_dtype dt : {LMX_F32, LMX_F16}) {
        const size_t b = use_split_k(&pp, dt) ? decode_workspace_bytes(&pp) : prefill_workspace_bytes(&pp);
        if (b > inner) inner = b;
    }
    PadLayout L;
    L.inner = 0;
    L.q = up256(inner);
    L.kv = L.q + up256((size_t)p->n_tokens * p->n_heads * hp * 4);  // room for an fp32 query
    L.cur = L.kv + 2 * up256((size_t)pp.n_slots * pp.kv_dim * 2);
    L.out = L.cur + 2 * up256((size_t)p->n_tokens * pp.kv_dim * 2);
    L.total = L.out + up256((size_t)p->n_tokens * p->n_heads * hp * 4);
    return L;
}

size_t padded_workspace_bytes(const lmx_attn_params* p) { return pad_layout(p).total; }

// dst[r][h][0 .. hp) = src[r * row_stride + h * head_stride + 0 .. hd), zero
// beyond hd.  Four elements a thread (hd, hp, the strides multiples of 4).
template <typename T>
__global__ __launch_bounds__(256) void pad_rows_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                       long n_rows, int n_heads, long row_stride,
                                                       int head_stride, int hd, int hp) {
    typedef T T4 __attribute__((ext_vector_type(4)));
    const int c4n = hp / 4;
    const long n = n_rows * n_heads * c4n;
    for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
        const int c4 = (int)(i % c4n);
        const long rh = i / c4n;
        const int h = (int)(rh % n_heads);
        const long r = rh / n_heads;
        T4 v = {};
        if (4 * c4 < hd) v = *reinterpret_cast<const T4*>(src + r * row_stride + (long)h * head_stride + 4 * c4);
        *reinterpret_cast<T4*>(dst + i * 4) = v;
    }
}

// out[row][0 .. hd) = src[row][0 .. hd) of the padded rows, gated.
__global__ __launch_bounds__(256) void unpad_out_kernel(const float* __restrict__ src, float* __restrict__ out,
                                                        long n_rows, int hd, int hp, const float* gate,
                                                        int gate_stride) {
    const int c4n = hd / 4;
    const long n = n_rows * c4n;
    for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
        const int c4 = (int)(i % c4n);
        const long r = i / c4n;
        f32x4 y = *reinterpret_cast<const f32x4*>(src + r * hp + 4 * c4);
        if (gate) y = gate_sigmoid4(y, gate + r * gate_stride + 4 * c4);
        *reinterpret_cast<f32x4*>(out + r * hd + 4 * c4) = y;
    }
}

static unsigned grid_for(long items) {
    long b = (items + 255) / 256;
    return (unsigned)(b < 1 ? 1 : (b > 16384 ? 16384 : b));
}

lmx_status padded_attn(const lmx_attn_params* p, const AttnIo& io, const void* q, lmx_dtype q_dt,
                       const void* k_cache, const void* v_cache, const void* k_cur, const void* v_cur,
                       float* out, void* ws, size_t ws_bytes, hipStream_t st) {
    const PadLayout L = pad_layout(p);
    if (!ws || ws_bytes < L.total) return LMX_E_WORKSPACE;
    if (((uintptr_t)ws & 255) != 0) return LMX_E_ALIGN;
    const lmx_attn_params pp = padded_params(p);
    const int hd = (int)p->head_dim, hp = (int)pp.head_dim;
    const int H = (int)p->n_heads, Hkv = (int)p->n_kv_heads;
    const long t = p->n_tokens;
    char* w = static_cast<char*>(ws);
    void* qp = w + L.q;
    f16* kp = reinterpret_cast<f16*>(w + L.kv);
    f16* vp = reinterpret_cast<f16*>(w + L.kv + up256((size_t)pp.n_slots * pp.kv_dim * 2));
    f16* kcp = k_cur ? reinterpret_cast<f16*>(w + L.cur) : nullptr;
    f16* vcp = k_cur ? reinterpret_cast<f16*>(w + L.cur + up256((size_t)t * pp.kv_dim * 2)) : nullptr;
    float* op = reinterpret_cast<float*>(w + L.out);
    (void)hipGetLastError();
    if (q_dt == LMX_F32)
        hipLaunchKernelGGL(pad_rows_kernel<float>, dim3(grid_for(t * H * hp / 4)), dim3(256), 0, st,
                           static_cast<const float*>(q), static_cast<float*>(qp), t * H, 1, (long)io.q_stride, 0,
                           hd, hp);
    else
        hipLaunchKernelGGL(pad_rows_kernel<f16>, dim3(grid_for(t * H * hp / 4)), dim3(256), 0, st,
                           static_cast<const f16*>(q), static_cast<f16*>(qp), t * H, 1, (long)io.q_stride, 0, hd,
                           hp);
    const long rows = pp.n_slots;
    hipLaunchKernelGGL(pad_rows_kernel<f16>, dim3(grid_for(rows * Hkv * hp / 4)), dim3(256), 0, st,
                       static_cast<const f16*>(k_cache), kp, rows, Hkv, (long)p->kv_dim, hd, hd, hp);
    hipLaunchKernelGGL(pad_rows_kernel<f16>, dim3(grid_for(rows * Hkv * hp / 4)), dim3(256), 0, st,
                       static_cast<const f16*>(v_cache), vp, rows, Hkv, (long)p->kv_dim, hd, hd, hp);
    if (k_cur) {
        hipLaunchKernelGGL(pad_rows_kernel<f16>, dim3(grid_for(t * Hkv * hp / 4)), dim3(256), 0, st,
                           static_cast<const f16*>(k_cur), kcp, t, Hkv, (long)p->kv_dim, hd, hd, hp);
        hipLaunchKernelGGL(pad_rows_kernel<f16>, dim3(grid_for(t * Hkv * hp / 4)), dim3(256), 0, st,
                           static_cast<const f16*>(v_cur), vcp, t, Hkv, (long)p->kv_dim, hd, hd, hp);
    }
    if (hipGetLastError() != hipSuccess) return LMX_E_LAUNCH;
    const AttnIo pio{hp, hp, nullptr};
    const lmx_status s = use_split_k(&pp, q_dt)
                             ? decode_fwd(&pp, pio, qp, q_dt, kp, vp, kcp, vcp, op, w + L.inner, L.q, st)
                             : prefill_fwd(&pp, pio, qp, q_dt, kp, vp, kcp, vcp, op, w + L.inner, L.q, st);
    if (s != LMX_OK) return s;
    hipLaunchKernelGGL(unpad_out_kernel, dim3(grid_for(t * H * hd / 4)), dim3(256), 0, st, op, out, t * H, hd, hp,
                       io.gate, io.gate_stride);
    LMX_CHECK_LAUNCH();
    return LMX_OK;
}

}  // namespace lmx
