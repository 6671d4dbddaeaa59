// Gated delta rule on gfx950: token-sequential form.
//
// Replaces delta_recur (deltanet.wgsl:193-239), which runs one workgroup per
// v-head with each thread owning a state row in global memory and re-reading
// and re-writing it every token.  State rows are independent in this
// recurrence (row j only ever sees its own value v_j), so here the rows of
// every head are spread over many workgroups, and each row lives in the
// registers of one 16-lane DPP row for the whole batch: S is read from HBM
// once and written once per call.
//
// Per token and row j (qwen35/cpu.rs:228-244, term for term):
//   S_j <- g S_j;  pred = S_j . k;  d = b (v_j - pred);  S_j += d k;
//   o_j = scale * (S_j . q)
#include "common.hpp"

namespace lmx {

struct DeltaArgs {
    const float* ssm_a;
    const float* dt_bias;
    const float* alpha;
    const float* beta;
    const float* conv;
    float* state;
    float* out;
    int n_tok, conv_dim, key_dim, d_inner, n_vh, n_kh;
    float scale;
};

// ops.rs:187-193
__device__ __forceinline__ float softplus_f(float x) { return x > 20.f ? x : logf(1.f + expf(x)); }

// One 256-thread workgroup = 16 state rows of one v-head; lane (row r, col c)
// holds elements [c*SD/16, (c+1)*SD/16) of row 16*blk + 4*wave + r.
template <int SD>
__global__ __launch_bounds__(256) void delta_recur_kernel(DeltaArgs a) {
    constexpr int E = SD / 16;
    const int hv = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15;
    const int j = blockIdx.x * 16 + wave * 4 + (lane >> 4);
    const int hk = hv % a.n_kh;
    const float A = a.ssm_a[hv], dt = a.dt_bias[hv];

    float S[E];
    float* srow = a.state + ((size_t)hv * SD + j) * SD + col * E;
    load_f32<E>(srow, S);

    const float* qbase = a.conv + (size_t)hk * SD + col * E;
    const float* kbase = a.conv + a.key_dim + (size_t)hk * SD + col * E;
    const float* vbase = a.conv + 2 * (size_t)a.key_dim + (size_t)hv * SD + j;

    float kn[E], qn[E];
    load_f32<E>(kbase, kn);
    load_f32<E>(qbase, qn);
    float vn = vbase[0];
    float an = a.alpha[hv], bn = a.beta[hv];

    for (int i = 0; i < a.n_tok; ++i) {
        float k[E], q[E];
#pragma unroll
        for (int e = 0; e < E; ++e) {
            k[e] = kn[e];
            q[e] = qn[e];
        }
        const float v = vn, al = an, be = bn;
        if (i + 1 < a.n_tok) {  // prefetch the next token
            const size_t ro = (size_t)(i + 1) * a.conv_dim;
            load_f32<E>(kbase + ro, kn);
            load_f32<E>(qbase + ro, qn);
            vn = vbase[ro];
            an = a.alpha[(size_t)(i + 1) * a.n_vh + hv];
            bn = a.beta[(size_t)(i + 1) * a.n_vh + hv];
        }
        const float g = expf(A * softplus_f(al + dt));
        const float bmix = 1.f / (1.f + expf(-be));
        float pred = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            S[e] *= g;
            pred = fmaf(S[e], k[e], pred);
        }
        pred = row_sum16(pred);
        const float delta = (v - pred) * bmix;
        float o = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            S[e] = fmaf(delta, k[e], S[e]);
            o = fmaf(S[e], q[e], o);
        }
        o = row_sum16(o);
        if (col == 0) a.out[(size_t)i * a.d_inner + (size_t)hv * SD + j] = o * a.scale;
    }
#pragma unroll
    for (int e = 0; e < E; e += 4)
        *reinterpret_cast<f32x4*>(srow + e) = f32x4{S[e], S[e + 1], S[e + 2], S[e + 3]};
}

static DeltaArgs make_args(const lmx_dop* op, const float* ssm_a, const float* dt_bias,
                           const float* alpha, const float* beta, const float* conv, float* state,
                           float* out) {
    DeltaArgs a{};
    a.ssm_a = ssm_a;
    a.dt_bias = dt_bias;
    a.alpha = alpha;
    a.beta = beta;
    a.conv = conv;
    a.state = state;
    a.out = out;
    a.n_tok = (int)op->n_tok;
    a.conv_dim = (int)op->conv_dim;
    a.key_dim = (int)op->key_dim;
    a.d_inner = (int)op->d_inner;
    a.n_vh = (int)op->n_vh;
    a.n_kh = (int)op->n_kh;
    a.scale = op->scale;
    return a;
}

lmx_status deltanet_recur(const lmx_dop* op, const float* ssm_a, const float* dt_bias,
                          const float* alpha, const float* beta, const float* conv, float* state,
                          float* out, hipStream_t st) {
    const DeltaArgs a = make_args(op, ssm_a, dt_bias, alpha, beta, conv, state, out);
    const int sd = (int)op->s_dim;
    dim3 grid(sd / 16, op->n_vh);
    (void)hipGetLastError();
    if (sd == 128)
        hipLaunchKernelGGL(delta_recur_kernel<128>, grid, dim3(256), 0, st, a);
    else if (sd == 64)
        hipLaunchKernelGGL(delta_recur_kernel<64>, grid, dim3(256), 0, st, a);
    else
        return LMX_E_UNSUPPORTED;
    LMX_CHECK_LAUNCH();
    return LMX_OK;
}

// ------------------------------------------------------------ chunked form --
//
// For a chunk of C tokens with in-chunk log-decay cumsum lg_t = sum_{i<=t}
// log g_i (log g = ssm_a * softplus(alpha + dt), kept in log space so products
// of 64 decays never underflow before they are used), the recurrence above is
// exactly (rows of S are value dims, U/V/O are [C x rows]):
//
//   A[t,i] = b_t exp(lg_t - lg_i) k_t.k_i  (i < t),   Tb = (I + A)^-1 diag(b)
//   U      = Tb (V - diag(exp lg) K S0^T)
//   O      = diag(exp lg) Q S0^T + P U,   P[t,i] = exp(lg_t - lg_i) q_t.k_i (i <= t)
//   S_C    = exp(lg_C) S0 + U^T diag(exp(lg_C - lg)) K
//
// Kernel 1 (all (v-head, chunk) pairs in parallel) builds Tb, P and lg.
// Kernel 2 (one workgroup per (v-head, 16 state rows)) walks the chunks in
// order, with its 16 rows of S in LDS for the whole call.

template <int SD, int C>
__global__ __launch_bounds__(256) void delta_chunk_prep_kernel(DeltaArgs a, float* ws_T,
                                                               float* ws_P, float* ws_lg,
                                                               int n_chunks) {
    constexpr int LD = SD + 4;
    constexpr int PARTS = 256 / C;
    __shared__ __attribute__((aligned(16))) float Ks[C][LD];
    __shared__ __attribute__((aligned(16))) float Qs[C][LD];
    __shared__ float Am[C][C + 1];
    __shared__ float Tm[C][C + 1];
    __shared__ float red[PARTS][C];
    __shared__ float lg[C], bt[C];
    const int ch = blockIdx.x, hv = blockIdx.y, tid = threadIdx.x;
    const int c0 = ch * C, nv = min(C, a.n_tok - c0);
    const int hk = hv % a.n_kh;

    for (int i = tid; i < C * SD / 4; i += 256) {
        const int r = i / (SD / 4), c4 = i % (SD / 4);
        f32x4 kq = {0.f, 0.f, 0.f, 0.f}, qq = {0.f, 0.f, 0.f, 0.f};
        if (r < nv) {
            const float* row = a.conv + (size_t)(c0 + r) * a.conv_dim + (size_t)hk * SD + 4 * c4;
            qq = *reinterpret_cast<const f32x4*>(row);
            kq = *reinterpret_cast<const f32x4*>(row + a.key_dim);
        }
        *reinterpret_cast<f32x4*>(&Ks[r][4 * c4]) = kq;
        *reinterpret_cast<f32x4*>(&Qs[r][4 * c4]) = qq;
    }
    if (tid < C) {
        float l = 0.f, b = 0.f;  // padded tokens: g = 1, b = 0
        if (tid < nv) {
            const size_t gi = (size_t)(c0 + tid) * a.n_vh + hv;
            l = a.ssm_a[hv] * softplus_f(a.alpha[gi] + a.dt_bias[hv]);
            b = 1.f / (1.f + expf(-a.beta[gi]));
        }
        lg[tid] = l;
        bt[tid] = b;
    }
    __syncthreads();
    if (tid == 0) {
        float s = 0.f;
        for (int t = 0; t < C; ++t) {
            s += lg[t];
            lg[t] = s;
        }
    }
    __syncthreads();

    // Gram matrices: thread (bt_, bi) owns rows t = bt_ + 16u, cols i = bi + 16v.
    float* Pg = ws_P + ((size_t)hv * n_chunks + ch) * C * C;
    for (int blk = tid; blk < 16 * 16; blk += 256) {
        const int tr = blk / 16, ic = blk % 16;
        constexpr int NU = C / 16;
        float gkk[NU][NU], gqk[NU][NU];
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int v = 0; v < NU; ++v) gkk[u][v] = gqk[u][v] = 0.f;
#pragma unroll 2
        for (int d = 0; d < SD; d += 4) {
            f32x4 kt[NU], qt[NU], ki[NU];
#pragma unroll
            for (int u = 0; u < NU; ++u) {
                kt[u] = *reinterpret_cast<const f32x4*>(&Ks[tr + 16 * u][d]);
                qt[u] = *reinterpret_cast<const f32x4*>(&Qs[tr + 16 * u][d]);
                ki[u] = *reinterpret_cast<const f32x4*>(&Ks[ic + 16 * u][d]);
            }
#pragma unroll
            for (int u = 0; u < NU; ++u)
#pragma unroll
                for (int v = 0; v < NU; ++v)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        gkk[u][v] = fmaf(kt[u][e], ki[v][e], gkk[u][v]);
                        gqk[u][v] = fmaf(qt[u][e], ki[v][e], gqk[u][v]);
                    }
        }
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int v = 0; v < NU; ++v) {
                const int t = tr + 16 * u, i = ic + 16 * v;
                const float dec = i <= t ? expf(lg[t] - lg[i]) : 0.f;
                Am[t][i] = i < t ? bt[t] * dec * gkk[u][v] : 0.f;
                Pg[t * C + i] = gqk[u][v] * dec;
            }
    }
    __syncthreads();

    // T = (I + A)^-1, unit lower triangular, one row at a time:
    //   T[t][c] = [t == c] - sum_{c <= i < t} A[t][i] T[i][c]
    const int c = tid % C, part = tid / C;  // 256/C threads per column
    for (int t = 0; t < C; ++t) {
        float s = 0.f;
        if (c < t)
            for (int i = c + part; i < t; i += PARTS) s = fmaf(Am[t][i], Tm[i][c], s);
        red[part][c] = s;
        __syncthreads();
        if (part == 0) {
            float tot = 0.f;
            for (int pp = 0; pp < PARTS; ++pp) tot += red[pp][c];
            Tm[t][c] = c < t ? -tot : (c == t ? 1.f : 0.f);
        }
        __syncthreads();
    }
    float* Tg = ws_T + ((size_t)hv * n_chunks + ch) * C * C;
    for (int i = tid; i < C * C; i += 256) Tg[i] = Tm[i / C][i % C] * bt[i % C];
    if (tid < C) ws_lg[((size_t)hv * n_chunks + ch) * C + tid] = lg[tid];
}

template <int SD, int C, int R>
__global__ __launch_bounds__(256) void delta_chunk_scan_kernel(DeltaArgs a, const float* ws_T,
                                                               const float* ws_P,
                                                               const float* ws_lg, int n_chunks) {
    constexpr int LD = SD + 4;
    __shared__ __attribute__((aligned(16))) float KQ[2 * C][LD];  // K rows, then Q rows
    __shared__ __attribute__((aligned(16))) float Ss[R][LD];
    __shared__ float Tb[C][C + 1];
    __shared__ float Pm[C][C + 1];
    __shared__ float XY[2 * C][R + 1];
    __shared__ float Zs[C][R + 1];
    __shared__ float Us[C][R + 1];
    __shared__ float lgs[C];
    const int tid = threadIdx.x;
    // blockIdx % 8 == hv % 8: the row blocks of one head share an XCD's L2.
    const int hv = blockIdx.x % a.n_vh, rb = blockIdx.x / a.n_vh;
    const int row0 = rb * R, hk = hv % a.n_kh;
    float* S_g = a.state + ((size_t)hv * SD + row0) * SD;

    for (int i = tid; i < R * SD / 4; i += 256) {
        const int j = i / (SD / 4), c4 = i % (SD / 4);
        *reinterpret_cast<f32x4*>(&Ss[j][4 * c4]) = *reinterpret_cast<const f32x4*>(S_g + (size_t)j * SD + 4 * c4);
    }

    for (int ch = 0; ch < n_chunks; ++ch) {
        const int c0 = ch * C, nv = min(C, a.n_tok - c0);
        __syncthreads();
        for (int i = tid; i < C * SD / 4; i += 256) {
            const int r = i / (SD / 4), c4 = i % (SD / 4);
            f32x4 kq = {0.f, 0.f, 0.f, 0.f}, qq = {0.f, 0.f, 0.f, 0.f};
            if (r < nv) {
                const float* row = a.conv + (size_t)(c0 + r) * a.conv_dim + (size_t)hk * SD + 4 * c4;
                qq = *reinterpret_cast<const f32x4*>(row);
                kq = *reinterpret_cast<const f32x4*>(row + a.key_dim);
            }
            *reinterpret_cast<f32x4*>(&KQ[r][4 * c4]) = kq;
            *reinterpret_cast<f32x4*>(&KQ[C + r][4 * c4]) = qq;
        }
        const float* Tg = ws_T + ((size_t)hv * n_chunks + ch) * C * C;
        const float* Pg = ws_P + ((size_t)hv * n_chunks + ch) * C * C;
        for (int i = tid; i < C * C; i += 256) {
            Tb[i / C][i % C] = Tg[i];
            Pm[i / C][i % C] = Pg[i];
        }
        for (int i = tid; i < C * R; i += 256) {
            const int t = i / R, j = i % R;
            Zs[t][j] = t < nv ? a.conv[(size_t)(c0 + t) * a.conv_dim + 2 * (size_t)a.key_dim +
                                       (size_t)hv * SD + row0 + j]
                              : 0.f;
        }
        if (tid < C) lgs[tid] = ws_lg[((size_t)hv * n_chunks + ch) * C + tid];
        __syncthreads();

        // XY = [K; Q] S_rows^T
        for (int it = tid; it < 2 * C * (R / 8); it += 256) {
            const int r = it / (R / 8), j0 = 8 * (it % (R / 8));
            float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            for (int d = 0; d < SD; d += 4) {
                const f32x4 x = *reinterpret_cast<const f32x4*>(&KQ[r][d]);
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    const f32x4 s = *reinterpret_cast<const f32x4*>(&Ss[j0 + jj][d]);
                    acc[jj] = fmaf(x[0], s[0], fmaf(x[1], s[1], fmaf(x[2], s[2], fmaf(x[3], s[3], acc[jj]))));
                }
            }
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) XY[r][j0 + jj] = acc[jj];
        }
        __syncthreads();
        // Z = V - exp(lg) X
        for (int i = tid; i < C * R; i += 256) {
            const int t = i / R, j = i % R;
            Zs[t][j] -= expf(lgs[t]) * XY[t][j];
        }
        __syncthreads();
        // U = Tb Z  (Tb lower triangular)
        for (int i = tid; i < C * R; i += 256) {
            const int t = i / R, j = i % R;
            float u = 0.f;
            for (int k = 0; k <= t; ++k) u = fmaf(Tb[t][k], Zs[k][j], u);
            Us[t][j] = u;
        }
        __syncthreads();
        // O = exp(lg) Y + P U
        for (int i = tid; i < C * R; i += 256) {
            const int t = i / R, j = i % R;
            float o = expf(lgs[t]) * XY[C + t][j];
            for (int k = 0; k <= t; ++k) o = fmaf(Pm[t][k], Us[k][j], o);
            if (t < nv) a.out[(size_t)(c0 + t) * a.d_inner + (size_t)hv * SD + row0 + j] = o * a.scale;
        }
        // S_rows = exp(lg_C) S_rows + (U * exp(lg_C - lg))^T K
        {
            const float lgC = lgs[C - 1];
            const float decC = expf(lgC);
            for (int i = tid; i < R * SD / 4; i += 256) {
                const int j = i / (SD / 4), d = 4 * (i % (SD / 4));
                f32x4 s = *reinterpret_cast<const f32x4*>(&Ss[j][d]);
                s[0] *= decC;
                s[1] *= decC;
                s[2] *= decC;
                s[3] *= decC;
                for (int t = 0; t < C; ++t) {
                    const float w = Us[t][j] * expf(lgC - lgs[t]);
                    const f32x4 k = *reinterpret_cast<const f32x4*>(&KQ[t][d]);
                    s[0] = fmaf(w, k[0], s[0]);
                    s[1] = fmaf(w, k[1], s[1]);
                    s[2] = fmaf(w, k[2], s[2]);
                    s[3] = fmaf(w, k[3], s[3]);
                }
                *reinterpret_cast<f32x4*>(&Ss[j][d]) = s;
            }
        }
    }
    __syncthreads();
    for (int i = tid; i < R * SD / 4; i += 256) {
        const int j = i / (SD / 4), c4 = i % (SD / 4);
        *reinterpret_cast<f32x4*>(S_g + (size_t)j * SD + 4 * c4) = *reinterpret_cast<const f32x4*>(&Ss[j][4 * c4]);
    }
}

static size_t chunk_ws_floats(const lmx_dop* op, int chunk) {
    const size_t n_chunks = (op->n_tok + chunk - 1) / chunk;
    return (size_t)op->n_vh * n_chunks * ((size_t)2 * chunk * chunk + chunk);
}

size_t deltanet_chunked_ws(const lmx_dop* op, int chunk) {
    return (chunk_ws_floats(op, chunk) * 4 + 255) / 256 * 256;
}

template <int SD, int C>
static void launch_chunked(const DeltaArgs& a, int n_vh, int n_chunks, float* wsT, float* wsP,
                           float* wsL, hipStream_t st) {
    constexpr int R = 16;
    hipLaunchKernelGGL((delta_chunk_prep_kernel<SD, C>), dim3(n_chunks, n_vh), dim3(256), 0, st, a,
                       wsT, wsP, wsL, n_chunks);
    hipLaunchKernelGGL((delta_chunk_scan_kernel<SD, C, R>), dim3(n_vh * (SD / R)), dim3(256), 0, st,
                       a, wsT, wsP, wsL, n_chunks);
}

lmx_status deltanet_chunked(const lmx_dop* op, const float* ssm_a, const float* dt_bias,
                            const float* alpha, const float* beta, const float* conv,
                            float* state, float* out, int chunk, void* ws, size_t ws_bytes,
                            hipStream_t st) {
    (void)ws_bytes;
    const DeltaArgs a = make_args(op, ssm_a, dt_bias, alpha, beta, conv, state, out);
    const int n_chunks = (int)((op->n_tok + chunk - 1) / chunk);
    const size_t per = (size_t)op->n_vh * n_chunks;
    float* wsT = static_cast<float*>(ws);
    float* wsP = wsT + per * chunk * chunk;
    float* wsL = wsP + per * chunk * chunk;
    const int sd = (int)op->s_dim;
    (void)hipGetLastError();
#define LMX_CH(SDV, CV)                                                                   \
    if (sd == SDV && chunk == CV) {                                                       \
        launch_chunked<SDV, CV>(a, (int)op->n_vh, n_chunks, wsT, wsP, wsL, st);            \
        LMX_CHECK_LAUNCH();                                                               \
        return LMX_OK;                                                                    \
    }
    LMX_CH(128, 64) LMX_CH(128, 32) LMX_CH(128, 16)
    LMX_CH(64, 64) LMX_CH(64, 32) LMX_CH(64, 16)
#undef LMX_CH
    return LMX_E_UNSUPPORTED;
}

}  // namespace lmx
