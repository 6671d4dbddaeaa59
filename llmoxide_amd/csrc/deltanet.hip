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

// Placeholder until the chunked kernel lands: the sequential kernel computes
// the same recurrence.
size_t deltanet_chunked_ws(const lmx_dop*, int) { return 0; }

lmx_status deltanet_chunked(const lmx_dop* op, const float* ssm_a, const float* dt_bias,
                            const float* alpha, const float* beta, const float* conv,
                            float* state, float* out, int, void*, size_t, hipStream_t st) {
    return deltanet_recur(op, ssm_a, dt_bias, alpha, beta, conv, state, out, st);
}

}  // namespace lmx
