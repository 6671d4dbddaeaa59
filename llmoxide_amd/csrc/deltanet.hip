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
#include <atomic>

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
//   Z      = V - diag(exp lg) K S0^T,       U = Tb Z
//   O      = diag(exp lg) Q S0^T + M Z,     M = P Tb,
//            P[t,i] = exp(lg_t - lg_i) q_t.k_i (i <= t)
//   S_C    = exp(lg_C) S0 + U^T diag(exp(lg_C - lg)) K
//
// (M Z = P U; folding Tb into M lets O be formed from Z alongside U.)
//
// With chunks of 16 every product runs on the fp32 matrix cores
// (v_mfma_f32_16x16x4_f32); with chunks of 32 and 64 on the bf16 ones with
// split operands (see "split-bf16 operands" below: about 2^-16 relative per
// product, fp32 accumulation, the state kept in fp32).  Kernel 1 (one
// workgroup per (chunk, k-head), all in parallel) builds Tb, M and the decay
// vectors of every v-head that reads that k-head.  Kernel 2 (one workgroup
// per (v-head, 16 state rows)) walks the chunks in order with its rows of S
// in registers.
//
// Operand layouts of the 16x16x4 fp32 MFMA, lane l = 16 * lq + lr:
//   A[i][k]: lane (i = lr, k = lq);  B[k][j]: lane (j = lr, k = lq);
//   D[i][j]: lane (j = lr), register r holds row i = 4 * lq + r.
// A contraction may visit its index in any order as long as A and B agree.
// Over a feature dim d the order used is d = 16 tau + 4 lq + r (step 4 tau + r),
// so a lane's operands for 4 steps are one contiguous float4 of a row; over a
// token dim it is t = 16 m + 4 lq + r, which makes a D tile (rows 4 lq + r,
// column lr) usable as the B operand of the next product without a shuffle.

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 ld4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }

// ---- split-bf16 operands (chunks of 32 and 64 tokens)
//
// The 16x16x32 bf16 MFMA runs 16 times the fp32 MFMA's FLOPs per cycle.
// Each fp32 operand x is carried as hi = bf16(x) and lo = bf16(x - hi)
// (round to nearest even both times), and a product a b is accumulated in
// fp32 as lo_a hi_b + hi_a lo_b + hi_a hi_b: the dropped lo_a lo_b and the
// rounding of lo leave a relative error near 2^-16 per product, against
// 2^-8 for a single bf16 product (measured on the C5 shapes over 2048
// tokens: 1e-5 of max|S| and of max|o|, where one f16 pass gives 6e-4).
// The state and every accumulator stay fp32.
//
// Operand layout of v_mfma_f32_16x16x32_bf16, lane l = 16 lq + lr:
//   A[i][k]: lane (i = lr) holds k = 8 lq + e, e = 0..7;  B[k][j] likewise
//   with j = lr;  D as for the fp32 MFMA (rows 4 lq + r, column lr).
// Contraction slot 8 lq + e of step s is mapped to index
//   32 s + 16 (e / 4) + 4 lq + e % 4,
// so a lane's eight operands are its own four-element groups of two
// adjacent 16-wide tiles: D tiles feed the next product's B operand, and
// fp32 rows give the A operand as two float4, with no shuffle.
//
// A "piece" is one such operand for all 64 lanes: hi of lane l at byte
// 16 l, lo at 1024 + 16 l (2 KiB).
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
struct Bf8 {
    bf16x8 hi, lo;
};
constexpr int kPiece = 2048;

__device__ __forceinline__ void split4(f32x4 x, bf16x4& hi, bf16x4& lo) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const __bf16 h = (__bf16)x[e];
        hi[e] = h;
        lo[e] = (__bf16)(x[e] - (float)h);
    }
}
__device__ __forceinline__ Bf8 split8(f32x4 x0, f32x4 x1) {
    bf16x4 h0, l0, h1, l1;
    split4(x0, h0, l0);
    split4(x1, h1, l1);
    return Bf8{__builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7),
               __builtin_shufflevector(l0, l1, 0, 1, 2, 3, 4, 5, 6, 7)};
}
__device__ __forceinline__ Bf8 join8(bf16x4 h0, bf16x4 h1, bf16x4 l0, bf16x4 l1) {
    return Bf8{__builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7),
               __builtin_shufflevector(l0, l1, 0, 1, 2, 3, 4, 5, 6, 7)};
}
__device__ __forceinline__ Bf8 ld_piece(const uint8_t* p, int lane) {
    return Bf8{*reinterpret_cast<const bf16x8*>(p + 16 * lane),
               *reinterpret_cast<const bf16x8*>(p + 1024 + 16 * lane)};
}
__device__ __forceinline__ void st_piece(uint8_t* p, int lane, const Bf8& v) {
    *reinterpret_cast<bf16x8*>(p + 16 * lane) = v.hi;
    *reinterpret_cast<bf16x8*>(p + 1024 + 16 * lane) = v.lo;
}
// c + a b over one 32-wide contraction step, both operands split.
__device__ __forceinline__ f32x4 mfma3(const Bf8& a, const Bf8& b, f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.lo, b.hi, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.lo, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.hi, c, 0, 0, 0);
}

// Per-chunk inputs of a scan wave that are not K or Q (see the scan kernel).
template <int NM>
struct ChunkIn {
    f32x4 v, e;           // V and exp(lg) at tokens 16 m + 4 lq + r
    f32x4 tb[NM], mm[NM]; // Tb, M row 16 m + lr, columns 16 n + 4 lq + r (block (m, n))
    f32x4 w[NM];          // exp(lg_C - lg) at tokens 16 n + 4 lq + r
    float gam;            // exp(lg_C)
};

template <int C>
struct ChunkSmem {
    static constexpr int LD = C + 4;  // row stride in floats; keeps float4 rows aligned
};

// LDS of the prep: the K/Q staging rows or the A, T, P work matrices (the
// same space, in turn), then the decays and b, one copy per wave.
template <int SD, int C>
struct PrepLds {
    static constexpr int LD = ChunkSmem<C>::LD, KLD = SD + 4;
    static constexpr int STAGE = 2 * C * KLD, WORK = 3 * C * LD;
    static constexpr int MAIN = STAGE > WORK ? STAGE : WORK;
    static constexpr int FLOATS = MAIN + 2 * 4 * 64;
};

// Stores of what the scan reads, in the one-launch form.  Each XCD has its
// own L2: a plain store stays in the writer's L2 until the launch ends, so it
// is seen only by workgroups on the writer's XCD; an agent-scope store (sc1)
// writes through to memory, where a workgroup on another XCD that has not yet
// read the line finds it.  The 16-byte agent form is two 8-byte atomic stores
// that the compiler emits itself (an asm store is opaque to its hazard and
// wait tracking).
__device__ __forceinline__ void st16_agent(uint8_t* p, bf16x8 v) {
    uint64_t u[2];
    __builtin_memcpy(u, &v, 16);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p), u[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p) + 1, u[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_piece_m(uint8_t* p, int lane, const Bf8& v, bool agent) {
    if (agent) {
        st16_agent(p + 16 * lane, v.hi);
        st16_agent(p + 1024 + 16 * lane, v.lo);
    } else {
        st_piece(p, lane, v);
    }
}
__device__ __forceinline__ void st_f32_m(float* p, float v, bool agent) {
    if (agent)
        __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        *p = v;
}
// The XCD (accelerator complex die) this wave runs on.
__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return x & 15;
}

// One workgroup per (chunk, k-head).  K K^T and Q K^T are shared by the v-heads
// hv = hk + u * n_kh (hv % n_kh == hk, deltanet.wgsl:200), so they are formed
// once, into registers, from K and Q rows staged in LDS with whole-line loads;
// the decays, the solve and M are per v-head, in LDS that reuses the staging
// space.  Decays are handled in log2 units (exp2 is the native instruction).
//
// SPLIT (chunks of 32 and 64): Tb and M go out as split-bf16 pieces, and the
// chunk's K and Q rows are written once more, split, in the scan's operand
// order for X and Y to ws_K, so the 16 scan workgroups that read a k-head's
// chunk split nothing themselves (the scan forms K^T from its K tiles in LDS).
//
// The workgroup walks items first, first + stride, ...  FUSED (inside
// delta_chunk_fused_kernel): items are numbered chunk-major (chunk ch, k-head
// hk is item ch n_kh + hk) so that early chunks are done first, and once the
// factors of v-head hv are out, flags[ch n_vh + hv] is set to 1.  Items below
// n_split are shared: split_u 0 does v-head u = 0 of the k-head, split_u 1
// the others (both write the same K/Q pieces).  Scan workgroup j records its
// XCD as reg[j] = XCD + 1 (reg follows the flags and the error word): an
// item's stores stay plain only when every scan workgroup that reads them has
// registered on this workgroup's XCD, and are agent-scope otherwise, so the
// result never depends on where workgroups run.  Otherwise items are numbered
// k-head-major and the stores are plain.
template <int SD, int C, bool SPLIT, bool FUSED>
__device__ __forceinline__ void chunk_prep_body(const DeltaArgs& a, float* ws_T, float* ws_P,
                                                float* ws_e, uint8_t* ws_K, int n_chunks,
                                                int first, int stride, float* lds,
                                                uint32_t* flags, int n_split, int split_u) {
    constexpr int NM = C / 16, LD = ChunkSmem<C>::LD;
    constexpr int NTILE = NM * (NM + 1) / 2, TPW = (NTILE + 3) / 4;
    constexpr int KLD = PrepLds<SD, C>::KLD;  // staged K/Q row stride in floats
    float* const Ks = lds;
    float* const Qs = lds + C * KLD;
    float* const As = lds;               // strictly lower A, later M
    float* const Tm = lds + C * LD;      // (I + A)^-1
    float* const Ps = lds + 2 * C * LD;  // P
    float (*const lg_w)[64] = reinterpret_cast<float (*)[64]>(lds + PrepLds<SD, C>::MAIN);
    float (*const b_w)[64] = lg_w + 4;
    const int tid = threadIdx.x;
    const int lane = tid & 63, lr = lane & 15, lq = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};

    // Items first, first + stride, ... (two workgroups a CU in the prep
    // kernel): the next item's K and Q rows load into registers while this one is
    // worked, so only a workgroup's first staging waits on memory (staging
    // was a third of a workgroup's time, all of them loading at once).
    // Rows past the end of the batch are zero.
    constexpr int SJ = C * SD / 4 / 256;
    f32x4 rq[SJ], rk[SJ];
    const int n_items = n_chunks * a.n_kh;
    auto item_ch = [&](int item) { return FUSED ? item / a.n_kh : item % n_chunks; };
    auto item_hk = [&](int item) { return FUSED ? item % a.n_kh : item / n_chunks; };
    auto load_rows = [&](int item) {
        const int lc0 = item_ch(item) * C, lnv = min(C, a.n_tok - lc0), lhk = item_hk(item);
#pragma unroll
        for (int j = 0; j < SJ; ++j) {
            const int idx = tid + 256 * j, row = idx / (SD / 4), c4 = idx % (SD / 4);
            f32x4 q = z4, k = z4;
            if (row < lnv) {
                const float* src = a.conv + (size_t)(lc0 + row) * a.conv_dim + (size_t)lhk * SD + 4 * c4;
                q = ld4(src);
                k = ld4(src + a.key_dim);
            }
            rq[j] = q;
            rk[j] = k;
        }
    };
    if (first < n_items) load_rows(first);
    const uint32_t my_xcc = FUSED ? xcc_id() : 0;
    const uint32_t* const reg = FUSED ? flags + n_chunks * a.n_vh + 1 : nullptr;
    for (int item = first; item < n_items; item += stride) {
        const int ch = item_ch(item), hk = item_hk(item);
        const int c0 = ch * C, nv = min(C, a.n_tok - c0);
        // the v-heads hk + u n_kh (u = 0 .. u_last; n_vh need not be a multiple
        // of n_kh) this workgroup does: all, or its share of a shared item
        // (none, u_last = -1, for a k-head past the v-heads)
        const int u_last = hk < a.n_vh ? (a.n_vh - 1 - hk) / a.n_kh : -1;
        const bool shared = FUSED && item < n_split;
        const int u_lo = shared && split_u > 0 ? 1 : 0;
        const int u_hi = shared && split_u == 0 ? min(0, u_last) : u_last;

        // alpha and beta of the next v-head, in flight during the work before it
        // (and its ssm_a, dt_bias)
        float al_n = 0.f, be_n = 0.f, sa_n, dtb_n;
        auto ab_fetch = [&](int hv) {
            sa_n = a.ssm_a[hv];
            dtb_n = a.dt_bias[hv];
            if (lane < nv) {
                const size_t gi = (size_t)(c0 + lane) * a.n_vh + hv;
                al_n = a.alpha[gi];
                be_n = a.beta[gi];
            }
        };
        if (u_lo <= u_hi) ab_fetch(hk + u_lo * a.n_kh);

        // Stage the chunk's K and Q rows (the previous item's LDS reads are done).
        __syncthreads();
#pragma unroll
        for (int j = 0; j < SJ; ++j) {
            const int idx = tid + 256 * j, row = idx / (SD / 4), c4 = idx % (SD / 4);
            *reinterpret_cast<f32x4*>(Qs + row * KLD + 4 * c4) = rq[j];
            *reinterpret_cast<f32x4*>(Ks + row * KLD + 4 * c4) = rk[j];
        }
        __syncthreads();
        // FUSED: the registrations of this item's readers (v-heads hk + u n_kh,
        // every row block), combined after the Gram tiles, so their round trip
        // is hidden; issued before the row prefetch, so that wait does not
        // cover it.  A registration, once made, never changes, so a reader
        // seen on this XCD here is there for good.
        int here = 1;
        if constexpr (FUSED) {
            const int nu = u_hi - u_lo + 1, n_rd = nu * (SD / 16);
            for (int r = tid; r < n_rd; r += 256) {
                const int hv = hk + (u_lo + r % nu) * a.n_kh, rb = r / nu;
                here &= __hip_atomic_load(reg + rb * a.n_vh + hv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                        my_xcc + 1;
            }
        }
        // The next item's rows.  FUSED issues them once this item is
        // published: beside the scan, issuing them stalls the wave for
        // microseconds, and an item's latency matters most for the first
        // chunks, which the scan waits for; later rounds run ahead of it.
        const bool more = item + stride < n_items;
        if (!FUSED && more) load_rows(item + stride);

        // Gram tiles (m, n), n <= m, dealt round-robin to the 4 waves; a tile's
        // D layout is lane (column 16 n + lr), rows 16 m + 4 lq + r.  SPLIT:
        // split-bf16 triples over 32-wide dim steps (the operands of both
        // tiles are rows of K or Q, in the same slot order), a fifth of the
        // matrix-core time of the fp32 steps, which matters most beside the
        // scan's chains in the one-launch form.
        f32x4 gk[TPW], gq[TPW];
        int tile_m[TPW], tile_n[TPW];
#pragma unroll
        for (int k = 0; k < TPW; ++k) {
            int m = 0, n = w + 4 * k;
            while (n > m) {
                n -= m + 1;
                ++m;
            }
            tile_m[k] = m;
            tile_n[k] = n;
            gk[k] = z4;
            gq[k] = z4;
            if (w + 4 * k >= NTILE) continue;
            const float* km = Ks + (16 * m + lr) * KLD + 4 * lq;
            const float* qm = Qs + (16 * m + lr) * KLD + 4 * lq;
            const float* kn = Ks + (16 * n + lr) * KLD + 4 * lq;
            if constexpr (SPLIT) {
#pragma unroll
                for (int sg = 0; sg < SD / 32; ++sg) {
                    const Bf8 ka = split8(ld4(km + 32 * sg), ld4(km + 32 * sg + 16));
                    const Bf8 qa = split8(ld4(qm + 32 * sg), ld4(qm + 32 * sg + 16));
                    const Bf8 kb = split8(ld4(kn + 32 * sg), ld4(kn + 32 * sg + 16));
                    gk[k] = mfma3(ka, kb, gk[k]);
                    gq[k] = mfma3(qa, kb, gq[k]);
                }
            } else {
#pragma unroll
                for (int u = 0; u < SD / 16; ++u) {
                    const f32x4 a4 = ld4(km + 16 * u), q4 = ld4(qm + 16 * u), b4 = ld4(kn + 16 * u);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        gk[k] = mfma4(a4[r], b4[r], gk[k]);
                        gq[k] = mfma4(q4[r], b4[r], gq[k]);
                    }
                }
            }
        }

        bool agent = false;  // this item's stores write through (see above)
        if constexpr (FUSED) agent = __builtin_amdgcn_readfirstlane(__syncthreads_and(here)) == 0;

        if constexpr (SPLIT) {
            // K, Q pieces (token tile m, dim step sg): lane (lr, lq) row 16 m + lr,
            // dims 32 sg + 4 lq + {0..3} and + 16.  Staged rows past the chunk's
            // end are zero.
            constexpr int SX = SD / 32;
            uint8_t* kb = ws_K + ((size_t)ch * a.n_kh + hk) * (2 * C * SD * 4);
            for (int q = tid; q < NM * SX * 64; q += 256) {
                const int l = q & 63, pc = q >> 6, m = pc / SX, sg = pc % SX;
                const int t = 16 * m + (l & 15), c0 = 32 * sg + 4 * (l >> 4);
                st_piece_m(kb + pc * kPiece, l, split8(ld4(Ks + t * KLD + c0), ld4(Ks + t * KLD + c0 + 16)), agent);
                st_piece_m(kb + C * SD * 4 + pc * kPiece, l,
                           split8(ld4(Qs + t * KLD + c0), ld4(Qs + t * KLD + c0 + 16)), agent);
            }
        }

        for (int hv = hk + u_lo * a.n_kh; hv <= hk + u_hi * a.n_kh; hv += a.n_kh) {
            const size_t cb = (size_t)hv * n_chunks + ch;
            // the staging (first head) or the previous head's A, T, P are no longer read
            __syncthreads();
            // Every wave forms the log2-decay cumsum and b for lane = token itself.
            {
                float l = 0.f, b = 0.f;  // padded tokens: g = 1, b = 0
                if (lane < nv) {
                    l = kLog2e * sa_n * softplus_f(al_n + dtb_n);
                    b = 1.f / (1.f + expf(-be_n));
                }
                if (hv + a.n_kh <= hk + u_hi * a.n_kh) ab_fetch(hv + a.n_kh);
#pragma unroll
                for (int off = 1; off < 64; off <<= 1) {
                    const float y = __shfl_up(l, off);
                    if (lane >= off) l += y;
                }
                lg_w[w][lane] = l;
                b_w[w][lane] = b;
                if (w == 0 && lane < C) {
                    const float lgC = __shfl(l, C - 1);
                    st_f32_m(ws_e + cb * 2 * C + lane, fast_exp2(l), agent);
                    st_f32_m(ws_e + cb * 2 * C + C + lane, fast_exp2(lgC - l), agent);
                }
            }
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int k = 0; k < TPW; ++k) {
                if (w + 4 * k >= NTILE) continue;
                const int i = 16 * tile_n[k] + lr;
                const float li = lg_w[w][i];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = 16 * tile_m[k] + 4 * lq + r;
                    const float dec = i <= t ? fast_exp2(lg_w[w][t] - li) : 0.f;
                    As[t * LD + i] = i < t ? b_w[w][t] * dec * gk[k][r] : 0.f;
                    Ps[t * LD + i] = dec * gq[k][r];
                }
            }
            __syncthreads();  // A and P complete

            // (I + A)^-1 by 16x16 blocks.  Diagonal blocks by forward substitution,
            // lane lr owning column lr of block w:
            //   T[t][c] = [t == c] - sum_{i < t} A[t][i] T[i][c]
            if (w < NM) {
                const int base = 16 * w;
                float tv[16];
#pragma unroll
                for (int t = 0; t < 16; ++t) {
                    float s = t == lr ? 1.f : 0.f;
                    const float* arow = As + (base + t) * LD + base;
#pragma unroll
                    for (int i = 0; i < t; ++i) s = fmaf(-arow[i], tv[i], s);
                    tv[t] = s;
                }
                if (lq == 0)
#pragma unroll
                    for (int t = 0; t < 16; ++t) Tm[(base + t) * LD + base + lr] = tv[t];
            }
            // Off-diagonal blocks level by level:
            //   T[M][N] = -T[M][M] * sum_{N <= Q < M} A[M][Q] T[Q][N]
            for (int lev = 1; lev < NM; ++lev) {
                __syncthreads();
                if (w < NM - lev) {
                    const int N = w, M = w + lev;
                    f32x4 x = z4;
                    for (int Q = N; Q < M; ++Q) {
                        const f32x4 av = ld4(As + (16 * M + lr) * LD + 16 * Q + 4 * lq);
#pragma unroll
                        for (int s = 0; s < 4; ++s)
                            x = mfma4(av[s], Tm[(16 * Q + 4 * lq + s) * LD + 16 * N + lr], x);
                    }
                    const f32x4 tv = ld4(Tm + (16 * M + lr) * LD + 16 * M + 4 * lq);
                    f32x4 y = z4;
#pragma unroll
                    for (int s = 0; s < 4; ++s) y = mfma4(tv[s], x[s], y);
#pragma unroll
                    for (int r = 0; r < 4; ++r) Tm[(16 * M + 4 * lq + r) * LD + 16 * N + lr] = -y[r];
                }
            }
            __syncthreads();
            // M = P Tb on the blocks at or below the diagonal, into As (free now):
            //   M[m][n] = sum_{n <= k <= m} P[m][k] T[k][n] diag(b)
#pragma unroll
            for (int q = 0; q < TPW; ++q) {
                if (w + 4 * q >= NTILE) continue;
                const int m = tile_m[q], n = tile_n[q];
                const float bc = b_w[w][16 * n + lr];
                f32x4 acc = z4;
                for (int k = n; k <= m; ++k) {
                    const f32x4 pv = ld4(Ps + (16 * m + lr) * LD + 16 * k + 4 * lq);
#pragma unroll
                    for (int s = 0; s < 4; ++s)
                        acc = mfma4(pv[s], Tm[(16 * k + 4 * lq + s) * LD + 16 * n + lr] * bc, acc);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) As[(16 * m + 4 * lq + r) * LD + 16 * n + lr] = acc[r];
            }
            __syncthreads();
            if constexpr (SPLIT) {
                // Tb and M as split pieces (row tile bm, token step sg): lane
                // (lr, lq) row 16 bm + lr, columns 32 sg + 4 lq + {0..3} and + 16.
                // Entries above the diagonal (Tb) or in blocks above it (M) are 0.
                constexpr int SC = C / 32;
                uint8_t* Tg = reinterpret_cast<uint8_t*>(ws_T + cb * C * C);
                uint8_t* Mg = reinterpret_cast<uint8_t*>(ws_P + cb * C * C);
                for (int q = tid; q < NM * SC * 64; q += 256) {
                    const int l = q & 63, pc = q >> 6, bm = pc / SC, sg = pc % SC;
                    const int t = 16 * bm + (l & 15);
                    f32x4 to[2], mo[2];
#pragma unroll
                    for (int hf = 0; hf < 2; ++hf) {
                        const int i0 = 32 * sg + 16 * hf + 4 * (l >> 4), bn = 2 * sg + hf;
                        const f32x4 tv = ld4(Tm + t * LD + i0), bv = ld4(&b_w[w][i0]), mv = ld4(As + t * LD + i0);
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            to[hf][e] = i0 + e <= t ? tv[e] * bv[e] : 0.f;
                            mo[hf][e] = bn <= bm ? mv[e] : 0.f;
                        }
                    }
                    st_piece_m(Tg + pc * kPiece, l, split8(to[0], to[1]), agent);
                    st_piece_m(Mg + pc * kPiece, l, split8(mo[0], mo[1]), agent);
                }
                continue;
            }
            // Tb and M go out in MFMA A-operand order: block (m, n), lane
            // l = 16 lq + lr, element e holds row 16 m + lr, column 16 n + 4 lq + e,
            // so each lane of a scan wave reads its block with one float4 and the
            // wave reads 1 KB contiguous.  Blocks above the diagonal are zero.
            float* Tg = ws_T + cb * C * C;
            float* Mg = ws_P + cb * C * C;
            for (int q = tid; q < C * C / 4; q += 256) {
                const int l = q & 63, blk = q >> 6;
                const int bm = blk / NM, bn = blk % NM;
                const int t = 16 * bm + (l & 15), i0 = 16 * bn + 4 * (l >> 4);
                const f32x4 tv = ld4(Tm + t * LD + i0), bv = ld4(&b_w[w][i0]), mv = ld4(As + t * LD + i0);
                f32x4 to, mo;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    to[e] = i0 + e <= t ? tv[e] * bv[e] : 0.f;
                    mo[e] = bn <= bm ? mv[e] : 0.f;
                }
                *reinterpret_cast<f32x4*>(Tg + 4 * q) = to;
                *reinterpret_cast<f32x4*>(Mg + 4 * q) = mo;
            }
        }
        if constexpr (FUSED) {
            // Every thread's stores of the item acknowledged, then the flag.
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (tid <= u_hi - u_lo)
                __hip_atomic_store(flags + ch * a.n_vh + hk + (u_lo + tid) * a.n_kh, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            if (more) load_rows(item + stride);
        }
    }
}

template <int SD, int C, bool SPLIT>
__global__ __launch_bounds__(256, 2) void delta_chunk_prep_kernel(DeltaArgs a, float* ws_T,
                                                               float* ws_P, float* ws_e,
                                                               uint8_t* ws_K, int n_chunks) {
    __shared__ __attribute__((aligned(16))) float lds[PrepLds<SD, C>::FLOATS];
    chunk_prep_body<SD, C, SPLIT, false>(a, ws_T, ws_P, ws_e, ws_K, n_chunks, blockIdx.x, gridDim.x,
                                         lds, nullptr, 0, 0);
}

// One workgroup per (v-head, 16 state rows); blockIdx % n_vh == hv, so with
// n_vh a multiple of 8 the row blocks of a head land on one XCD and share
// its L2 for K, Q, Tb and P.  Wave w owns token tile w of each chunk (X, Y,
// U, O) and state columns [16 TPW w, 16 TPW (w + 1)) for the update; the
// updated columns are exchanged through LDS once per chunk.
template <int SD, int C>
__global__ __launch_bounds__(256) void delta_chunk_scan_kernel(DeltaArgs a, const float* ws_T,
                                                               const float* ws_P,
                                                               const float* ws_e, int n_chunks) {
    constexpr int NT = SD / 16, NM = C / 16, TPW = NT / 4, LD = ChunkSmem<C>::LD;
    __shared__ __attribute__((aligned(16))) float Kt[SD * LD];  // K^T of the chunk
    __shared__ f32x4 Zx[NM * 64];                                // Z tiles, D layout
    __shared__ f32x4 Ux[NM * 64];                                // U tiles, D layout
    __shared__ f32x4 Sx[NT * 64];                                // S columns, D layout
    const int lane = threadIdx.x & 63, lr = lane & 15, lq = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hv = blockIdx.x % a.n_vh, rb = blockIdx.x / a.n_vh;
    const int row0 = rb * 16, hk = hv % a.n_kh;
    // With C = 64 every wave owns a token tile; the constant keeps the loads
    // out of branches, so their waits count only what each use needs.
    const bool tok_wave = NM >= 4 || w < NM;
    const int m = tok_wave ? w : 0;
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};

    // Row j = row0 + lr of S; register u holds columns 16 u + 4 lq + [0, 4).
    float* srow = a.state + ((size_t)hv * SD + row0 + lr) * SD + 4 * lq;
    f32x4 S[NT];
#pragma unroll
    for (int u = 0; u < NT; ++u) S[u] = ld4(srow + 16 * u);
    f32x4 Sown[TPW];  // this wave's columns 16 (TPW w + j) + 4 lq + r, which it updates
#pragma unroll
    for (int j = 0; j < TPW; ++j) Sown[j] = ld4(srow + 16 * (TPW * w + j));

    // Inputs of one chunk.  The next chunk's are loaded during this chunk's
    // X/Y products: after the MFMAs of column block u, K and Q block u (dead
    // by then) are reloaded in place and a share of the other loads is issued,
    // so the vector-memory path is fed at the MFMA pace instead of in one
    // burst that stalls issue.  The non-K/Q inputs alternate between two
    // register sets (the loop is unrolled by two), so nothing is copied.
    f32x4 kr[NT], qr[NT];  // K, Q row 16 m + lr
    ChunkIn<NM> in0, in1;
    // A zero the compiler cannot see through: indexing with it keeps uniform
    // loads on the vector path, counted by vmcnt, instead of the scalar path,
    // whose counter is shared with LDS and drained at every barrier.
    int vzero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(vzero));

    // Tokens past the end of the last chunk read row 0 of the chunk instead:
    // their b is 0, so their rows and columns of Tb are exactly zero, their U
    // rows are exactly zero, and only finiteness of what they read matters.
    auto kq_row = [&](int ch) {
        const int t = 16 * m + lr;
        return a.conv + (size_t)(ch * C + (t < a.n_tok - ch * C ? t : 0)) * a.conv_dim +
               (size_t)hk * SD + 4 * lq;
    };
    constexpr int NITEM = 6 + 3 * NM;
    auto fetch_item = [&](int ch, ChunkIn<NM>& d, int k) {
        const size_t cb = (size_t)hv * n_chunks + ch;
        const float* eb = ws_e + cb * 2 * C;
        if (k == 0) {
            d.gam = eb[C - 1 + vzero];
        } else if (k == 1) {
            d.e = ld4(eb + 16 * m + 4 * lq);
        } else if (k < 6) {
            const int tv = 16 * m + 4 * lq + (k - 2);
            const float* vcol = a.conv + 2 * (size_t)a.key_dim + (size_t)hv * SD + row0 + lr;
            d.v[k - 2] = vcol[(size_t)(ch * C + (tv < a.n_tok - ch * C ? tv : 0)) * a.conv_dim];
        } else if (k < 6 + NM) {
            d.tb[k - 6] = ld4(ws_T + cb * C * C + ((m * NM + (k - 6)) * 64 + lane) * 4);
        } else if (k < 6 + 2 * NM) {
            d.mm[k - 6 - NM] = ld4(ws_P + cb * C * C + ((m * NM + (k - 6 - NM)) * 64 + lane) * 4);
        } else {
            d.w[k - 6 - 2 * NM] = ld4(eb + C + 16 * (k - 6 - 2 * NM) + 4 * lq);
        }
    };
    auto fetch_all = [&](int ch, ChunkIn<NM>& d) {
        if (tok_wave) {
            const float* row = kq_row(ch);
#pragma unroll
            for (int u = 0; u < NT; ++u) kr[u] = ld4(row + a.key_dim + 16 * u);
#pragma unroll
            for (int u = 0; u < NT; ++u) qr[u] = ld4(row + 16 * u);
        }
#pragma unroll
        for (int k = 0; k < NITEM; ++k)
            if (tok_wave || k == 0 || k >= 6 + 2 * NM) fetch_item(ch, d, k);
    };

    auto step = [&](int ch, const ChunkIn<NM>& cur, ChunkIn<NM>& nxt) {
        const int nv = a.n_tok - ch * C;
        const int cn = min(ch + 1, n_chunks - 1);
        f32x4 X = z4, Y = z4;
        if (tok_wave) {
            // X = K S^T, Y = Q S^T over d = 16 u + 4 lq + r
            const float* row = kq_row(cn);
#pragma unroll
            for (int u = 0; u < NT; ++u) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    X = mfma4(kr[u][r], S[u][r], X);
                    Y = mfma4(qr[u][r], S[u][r], Y);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) Kt[(16 * u + 4 * lq + r) * LD + 16 * m + lr] = kr[u][r];
                kr[u] = ld4(row + a.key_dim + 16 * u);
                qr[u] = ld4(row + 16 * u);
                if (u < 2) fetch_item(cn, nxt, u);  // gam, e
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            fetch_item(cn, nxt, 0);  // gam
        }
        if (tok_wave) {
            // Z = V - exp(lg) X
            f32x4 Z;
#pragma unroll
            for (int r = 0; r < 4; ++r) Z[r] = cur.v[r] - cur.e[r] * X[r];
            Zx[m * 64 + lane] = Z;
        }
        __syncthreads();

        if (tok_wave) {
            // U = Tb Z and O = exp(lg) Y + M Z over t = 16 n + 4 lq + r, as two
            // interleaved chains; blocks above the diagonal of Tb and M are zero.
            f32x4 U = z4, O;
#pragma unroll
            for (int r = 0; r < 4; ++r) O[r] = cur.e[r] * Y[r];
#pragma unroll
            for (int n = 0; n < NM; ++n) {
                const f32x4 zb = Zx[n * 64 + lane];
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    U = mfma4(cur.tb[n][s], zb[s], U);
                    O = mfma4(cur.mm[n][s], zb[s], O);
                }
                fetch_item(cn, nxt, 2 + n);  // V
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int k = 2 + NM; k < 6; ++k) fetch_item(cn, nxt, k);
            Ux[m * 64 + lane] = U;
            float* orow = a.out + (size_t)ch * C * a.d_inner + (size_t)hv * SD + row0 + lr;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * m + 4 * lq + r;
                if (t < nv) orow[(size_t)t * a.d_inner] = O[r] * a.scale;
            }
#pragma unroll
            for (int n = 0; n < NM; ++n) fetch_item(cn, nxt, 6 + n);  // Tb
        }
        __syncthreads();

        // S <- exp(lg_C) S + (U diag(exp(lg_C - lg)))^T K on this wave's
        // columns, one chain per column tile, interleaved.
        f32x4 W[NM];
#pragma unroll
        for (int n = 0; n < NM; ++n) {
            const f32x4 ub = Ux[n * 64 + lane];
#pragma unroll
            for (int s = 0; s < 4; ++s) W[n][s] = ub[s] * cur.w[n][s];
        }
        f32x4 acc[TPW];
#pragma unroll
        for (int j = 0; j < TPW; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[j][r] = cur.gam * Sown[j][r];
#pragma unroll
        for (int n = 0; n < NM; ++n) {
            f32x4 kt[TPW];
#pragma unroll
            for (int j = 0; j < TPW; ++j) kt[j] = ld4(Kt + (16 * (TPW * w + j) + lr) * LD + 16 * n + 4 * lq);
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int j = 0; j < TPW; ++j) acc[j] = mfma4(kt[j][s], W[n][s], acc[j]);
            // M and exp(lg_C - lg) of the next chunk, spread over the products
#pragma unroll
            for (int k = 6 + NM + n; k < NITEM; k += NM)
                if (tok_wave || k >= 6 + 2 * NM) fetch_item(cn, nxt, k);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
            Sx[(TPW * w + j) * 64 + lane] = acc[j];
            Sown[j] = acc[j];
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < NT; ++u) S[u] = Sx[u * 64 + lane];
    };

    fetch_all(0, in0);
    // Drain the first chunk's loads here: with nothing outstanding on entry,
    // the waits inside the loop follow the loop body's own issue order.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    int ch = 0;
    for (; ch + 1 < n_chunks; ch += 2) {
        step(ch, in0, in1);
        step(ch + 1, in1, in0);
    }
    if (ch < n_chunks) step(ch, in0, in1);
#pragma unroll
    for (int j = 0; j < TPW; ++j) *reinterpret_cast<f32x4*>(srow + 16 * (TPW * w + j)) = Sown[j];
}

// The scan on split-bf16 operands (chunks of 32 and 64 tokens): the same
// work split and chunk algebra as delta_chunk_scan_kernel, every product a
// 16x16x32 bf16 MFMA triple (mfma3).  K, Q, Tb and M arrive as pieces
// from the prep kernel; the three operands formed here (Z, W = U exp(lg_C -
// lg), and the updated state columns) are split once by the wave that
// produces them and pass through LDS as bf16 hi/lo tiles in the D layout.
// Each wave keeps its own state columns in fp32 (Sown) for the decay term
// and the final store.  A piece register is reloaded with the next chunk's
// piece right after its last use in this chunk.
//
// The K^T operand of the state update comes from LDS, not from pieces of its
// own: each token wave writes the K tile it already holds for X (rows = its
// 16 tokens) into Kth/Ktl [token][dim] (bf16 hi, lo), and after the Z
// barrier every wave reads its K^T operand with ds_read_b64_tr_b16: in a
// 16-lane group, lane a + 4 i addresses row t0 + i, dims 16 ct + 4 a .. + 3,
// and lane L receives tokens t0 .. t0 + 3 of dim 16 ct + L.  That saves a
// third of the K/Q piece bytes the prep writes and a quarter of the pieces
// each scan workgroup reads from L2 per chunk.
//
// LDS: the Z, W and state tiles (bf16 hi/lo, D layout), then Kth and Ktl.
template <int SD, int C>
struct ScanLds {
    static constexpr int NT = SD / 16, NM = C / 16, KTLD = SD + 4;  // Kth/Ktl row stride (bf16)
    static constexpr int TILES = (4 * NM + 2 * NT) * 64;           // bf16x4 entries
    static constexpr int BYTES = TILES * 8 + 2 * C * KTLD * 2;
};

// A wait for a ready flag gives up after this many polls (each a memory
// round trip of a microsecond or more and a short sleep: seconds in all, far
// beyond any delay a busy GPU imposes on the prep), records the failure in
// *err and lets the workgroup finish, so no launch can hang on a producer
// that never runs.  (A test launches with no prep and a bound of 64.)
constexpr uint32_t kFlagPolls = 1u << 21;

// blk: the workgroup's (v-head, row block) index.  FUSED: chunk ch's inputs
// of its v-head are ready once flags[ch n_vh + hv] is 1, and the flag of the
// chunk after next is polled a chunk ahead, so a producer that keeps ahead
// costs no round trip on the chain.
template <int SD, int C, bool FUSED>
__device__ __forceinline__ void chunk_scan_bf_body(const DeltaArgs& a, const uint8_t* ws_T,
                                                   const uint8_t* ws_P, const float* ws_e,
                                                   const uint8_t* ws_K, int n_chunks, int blk,
                                                   uint8_t* lds, const uint32_t* flags,
                                                   uint32_t* err, uint32_t max_polls) {
    constexpr int NT = SD / 16, NM = C / 16, TPW = NT / 4;
    constexpr int SX = SD / 32, SC = C / 32;  // 32-wide steps over dims, over tokens
    constexpr size_t KQB = (size_t)2 * C * SD * 4;  // ws_K bytes per (chunk, k-head)
    static_assert(NM % 2 == 0 && NT % 4 == 0, "whole 32-wide steps, whole column tiles per wave");
    bf16x4* const Zh = reinterpret_cast<bf16x4*>(lds);  // Z tiles, D layout
    bf16x4* const Zl = Zh + NM * 64;
    bf16x4* const Wh = Zl + NM * 64;  // W tiles, D layout
    bf16x4* const Wl = Wh + NM * 64;
    bf16x4* const Sh = Wl + NM * 64;  // state columns, D layout
    bf16x4* const Sl = Sh + NT * 64;
    constexpr int KTLD = ScanLds<SD, C>::KTLD;  // 8-byte rows
    __bf16 (*const Kth)[KTLD] = reinterpret_cast<__bf16 (*)[KTLD]>(Sl + NT * 64);
    __bf16 (*const Ktl)[KTLD] = Kth + C;
    const int lane = threadIdx.x & 63, lr = lane & 15, lq = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hv = blk % a.n_vh, rb = blk / a.n_vh;
    const int row0 = rb * 16, hk = hv % a.n_kh;
    const bool tok_wave = NM >= 4 || w < NM;
    const int m = tok_wave ? w : 0;
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
    int vzero;  // a zero the compiler cannot see through (keeps gam on the vector path)
    asm volatile("v_mov_b32 %0, 0" : "=v"(vzero));

    // Row j = row0 + lr of S; Sown[jj] holds columns 16 (TPW w + jj) + 4 lq + r.
    float* srow = a.state + ((size_t)hv * SD + row0 + lr) * SD + 4 * lq;
    f32x4 Sown[TPW];
#pragma unroll
    for (int jj = 0; jj < TPW; ++jj) Sown[jj] = ld4(srow + 16 * (TPW * w + jj));
    auto put_s = [&]() {
#pragma unroll
        for (int jj = 0; jj < TPW; ++jj) {
            bf16x4 h, l;
            split4(Sown[jj], h, l);
            Sh[(TPW * w + jj) * 64 + lane] = h;
            Sl[(TPW * w + jj) * 64 + lane] = l;
        }
    };
    Bf8 sb[SX];  // S^T as the B operand of X and Y
    auto get_s = [&]() {
#pragma unroll
        for (int sg = 0; sg < SX; ++sg)
            sb[sg] = join8(Sh[2 * sg * 64 + lane], Sh[(2 * sg + 1) * 64 + lane], Sl[2 * sg * 64 + lane],
                           Sl[(2 * sg + 1) * 64 + lane]);
    };

    auto kq_base = [&](int ch) { return ws_K + ((size_t)ch * a.n_kh + hk) * KQB; };
    auto mat_base = [&](const uint8_t* ws, int ch) { return ws + ((size_t)hv * n_chunks + ch) * (C * C * 4); };
    Bf8 kx[SX], qx[SX], kt[TPW][SC], tb[SC], mm[SC];
    auto ld_kx = [&](int ch, int sg) { kx[sg] = ld_piece(kq_base(ch) + (m * SX + sg) * kPiece, lane); };
    auto ld_qx = [&](int ch, int sg) { qx[sg] = ld_piece(kq_base(ch) + C * SD * 4 + (m * SX + sg) * kPiece, lane); };
    // This wave's K tile (tokens 16 m + lr, dims 32 sg + 4 lq + {0..3}, + 16) to LDS
    auto put_k = [&](int sg) {
        const int t = 16 * m + lr, d0 = 32 * sg + 4 * lq;
        *reinterpret_cast<bf16x4*>(&Kth[t][d0]) = __builtin_shufflevector(kx[sg].hi, kx[sg].hi, 0, 1, 2, 3);
        *reinterpret_cast<bf16x4*>(&Kth[t][d0 + 16]) = __builtin_shufflevector(kx[sg].hi, kx[sg].hi, 4, 5, 6, 7);
        *reinterpret_cast<bf16x4*>(&Ktl[t][d0]) = __builtin_shufflevector(kx[sg].lo, kx[sg].lo, 0, 1, 2, 3);
        *reinterpret_cast<bf16x4*>(&Ktl[t][d0 + 16]) = __builtin_shufflevector(kx[sg].lo, kx[sg].lo, 4, 5, 6, 7);
    };
    // K^T operands of this wave's column tiles (dim 16 ct + lr, tokens 32 sg +
    // 4 lq + {0..3}, + 16), transposed out of LDS
    auto get_kt = [&]() {
        typedef __attribute__((address_space(3))) bf16x4 lds_b4;
        const int row = 4 * lq + (lr >> 2), col = 4 * (lr & 3);
#pragma unroll
        for (int jj = 0; jj < TPW; ++jj)
#pragma unroll
            for (int sg = 0; sg < SC; ++sg) {
                const int r0 = 32 * sg + row, c0 = 16 * (TPW * w + jj) + col;
                const bf16x4 h0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_b4*)&Kth[r0][c0]);
                const bf16x4 h1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_b4*)&Kth[r0 + 16][c0]);
                const bf16x4 l0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_b4*)&Ktl[r0][c0]);
                const bf16x4 l1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_b4*)&Ktl[r0 + 16][c0]);
                kt[jj][sg] = join8(h0, h1, l0, l1);
            }
    };
    // Tb and M are lower triangular by 16 x 16 blocks: piece (m, sg) covers
    // blocks 2 sg and 2 sg + 1 of row tile m, all zero when 2 sg > m.  Those
    // are never loaded (their registers keep the zeros set below), which
    // spares waves 0 and 1 of chunks of 64 a sixth of their piece bytes.
    auto tb_live = [&](int sg) { return 2 * sg <= m; };
    auto ld_tb = [&](int ch, int sg) {
        if (tb_live(sg)) tb[sg] = ld_piece(mat_base(ws_T, ch) + (m * SC + sg) * kPiece, lane);
    };
    auto ld_mm = [&](int ch, int sg) {
        if (tb_live(sg)) mm[sg] = ld_piece(mat_base(ws_P, ch) + (m * SC + sg) * kPiece, lane);
    };
#pragma unroll
    for (int sg = 0; sg < SC; ++sg) {
        const bf16x8 zb = {};
        tb[sg] = mm[sg] = Bf8{zb, zb};
    }

    // Small per-chunk inputs, two register sets (the loop is unrolled by two).
    struct Small {
        f32x4 v, e, wo;  // V, exp(lg), exp(lg_C - lg) at tokens 16 m + 4 lq + r
        float gam;       // exp(lg_C)
        uint32_t rdy;    // FUSED: the flag of the chunk after this one, as polled
    };
    // FUSED: flag polls, and the bounded wait (after one failure the
    // workgroup waits no more).
    bool failed = false;
    auto poll = [&](int c) -> uint32_t {
        return __hip_atomic_load(flags + (size_t)c * a.n_vh + hv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    auto wait_ready = [&](int c) {
        for (uint32_t n = 0; !failed && __builtin_amdgcn_readfirstlane(poll(c)) == 0; ++n) {
            if (n == max_polls) {
                failed = true;
                if (lane == 0) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __builtin_amdgcn_s_sleep(8);
        }
    };
    // Tokens past the end of the last chunk read row 0 of the chunk instead:
    // their b is 0, so their rows and columns of Tb are exactly zero and so
    // are their U rows; only finiteness of what they read matters.
    auto fetch_small = [&](int ch, Small& d) {
        const float* eb = ws_e + ((size_t)hv * n_chunks + ch) * 2 * C;
        d.gam = eb[C - 1 + vzero];
        if (tok_wave) {
            d.e = ld4(eb + 16 * m + 4 * lq);
            d.wo = ld4(eb + C + 16 * m + 4 * lq);
            const float* vcol = a.conv + 2 * (size_t)a.key_dim + (size_t)hv * SD + row0 + lr;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tv = 16 * m + 4 * lq + r;
                d.v[r] = vcol[(size_t)(ch * C + (tv < a.n_tok - ch * C ? tv : 0)) * a.conv_dim];
            }
        }
    };

    auto step = [&](int ch, const Small& cur, Small& nxt) {
        const int nv = a.n_tok - ch * C;
        const int cn = min(ch + 1, n_chunks - 1);
        if constexpr (FUSED) {
            if (__builtin_amdgcn_readfirstlane(cur.rdy) == 0) wait_ready(cn);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);  // chunk cn's loads stay after the wait
            nxt.rdy = poll(min(cn + 1, n_chunks - 1));
        }
        fetch_small(cn, nxt);
        f32x4 X = z4, Y = z4;
        if (tok_wave) {
            // X = K S^T, Y = Q S^T over the dims
#pragma unroll
            for (int sg = 0; sg < SX; ++sg) {
                X = mfma3(kx[sg], sb[sg], X);
                Y = mfma3(qx[sg], sb[sg], Y);
                put_k(sg);
                ld_kx(cn, sg);
                ld_qx(cn, sg);
            }
            // Z = V - exp(lg) X
            f32x4 Z;
#pragma unroll
            for (int r = 0; r < 4; ++r) Z[r] = cur.v[r] - cur.e[r] * X[r];
            bf16x4 h, l;
            split4(Z, h, l);
            Zh[m * 64 + lane] = h;
            Zl[m * 64 + lane] = l;
        }
        __syncthreads();  // Z complete, and the chunk's K tile in LDS
        get_kt();

        if (tok_wave) {
            // U = Tb Z and O = exp(lg) Y + M Z over the chunk's tokens
            f32x4 U = z4, O;
#pragma unroll
            for (int r = 0; r < 4; ++r) O[r] = cur.e[r] * Y[r];
#pragma unroll
            for (int sg = 0; sg < SC; ++sg) {
                const Bf8 zb = join8(Zh[2 * sg * 64 + lane], Zh[(2 * sg + 1) * 64 + lane],
                                     Zl[2 * sg * 64 + lane], Zl[(2 * sg + 1) * 64 + lane]);
                U = mfma3(tb[sg], zb, U);
                O = mfma3(mm[sg], zb, O);
                ld_tb(cn, sg);
                ld_mm(cn, sg);
            }
            float* orow = a.out + (size_t)ch * C * a.d_inner + (size_t)hv * SD + row0 + lr;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * m + 4 * lq + r;
                if (t < nv) orow[(size_t)t * a.d_inner] = O[r] * a.scale;
            }
            f32x4 W;
#pragma unroll
            for (int r = 0; r < 4; ++r) W[r] = U[r] * cur.wo[r];
            bf16x4 h, l;
            split4(W, h, l);
            Wh[m * 64 + lane] = h;
            Wl[m * 64 + lane] = l;
        }
        __syncthreads();  // W complete

        // S <- exp(lg_C) S + W^T K on this wave's columns
        f32x4 acc[TPW];
#pragma unroll
        for (int jj = 0; jj < TPW; ++jj)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[jj][r] = cur.gam * Sown[jj][r];
#pragma unroll
        for (int sg = 0; sg < SC; ++sg) {
            const Bf8 wb = join8(Wh[2 * sg * 64 + lane], Wh[(2 * sg + 1) * 64 + lane],
                                 Wl[2 * sg * 64 + lane], Wl[(2 * sg + 1) * 64 + lane]);
#pragma unroll
            for (int jj = 0; jj < TPW; ++jj) acc[jj] = mfma3(kt[jj][sg], wb, acc[jj]);
        }
#pragma unroll
        for (int jj = 0; jj < TPW; ++jj) Sown[jj] = acc[jj];
        put_s();
        __syncthreads();  // state columns complete
        get_s();
    };

    // Chunk 0's inputs, drained before the loop so the waits inside it follow
    // the loop body's own issue order.
    Small in0, in1;
    if constexpr (FUSED) {
        // The chain first: when a scan wave and a prep wave on one SIMD are
        // both ready, the scan's instruction issues.
        __builtin_amdgcn_s_setprio(2);
        wait_ready(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
    fetch_small(0, in0);
    if (tok_wave) {
#pragma unroll
        for (int sg = 0; sg < SX; ++sg) {
            ld_kx(0, sg);
            ld_qx(0, sg);
        }
#pragma unroll
        for (int sg = 0; sg < SC; ++sg) {
            ld_tb(0, sg);
            ld_mm(0, sg);
        }
    }
    put_s();
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    // FUSED: the next chunk's flag, polled after the drain (an agent-scope
    // load is a long round trip, which the drain would otherwise wait out)
    if constexpr (FUSED) in0.rdy = poll(min(1, n_chunks - 1));
    __syncthreads();
    get_s();
    int ch = 0;
    for (; ch + 1 < n_chunks; ch += 2) {
        step(ch, in0, in1);
        step(ch + 1, in1, in0);
    }
    if (ch < n_chunks) step(ch, in0, in1);
#pragma unroll
    for (int jj = 0; jj < TPW; ++jj) *reinterpret_cast<f32x4*>(srow + 16 * (TPW * w + jj)) = Sown[jj];
}

template <int SD, int C>
__global__ __launch_bounds__(256) void delta_chunk_scan_bf_kernel(DeltaArgs a, const uint8_t* ws_T,
                                                                  const uint8_t* ws_P,
                                                                  const float* ws_e,
                                                                  const uint8_t* ws_K, int n_chunks) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[ScanLds<SD, C>::BYTES];
    chunk_scan_bf_body<SD, C, false>(a, ws_T, ws_P, ws_e, ws_K, n_chunks, blockIdx.x, lds, nullptr, nullptr, 0);
}

// Prep and scan in one launch (chunks of 32 and 64).  Workgroups [0, n_prep)
// run the prep over items b, b + n_prep, ... in chunk order and publish each
// v-head's flag; workgroups [n_prep, n_prep + n_vh SD / 16) run the scan, each
// waiting for a chunk's flag before it loads that chunk's inputs.  The first
// n_split items (the first round, which the scan waits for) are shared: prep
// workgroup j does v-head 0 of item j and scan workgroup j, idle until then,
// the other v-heads before its scan, which shortens the first chunk's wait by
// a v-head's solve and products.  Prep
// workgroups never wait and come first in dispatch order, and the host
// launches this form only when the GPU holds more workgroups than the scan
// has, so a prep workgroup can always run.  Two workgroups a CU (one prep,
// one scan when all are resident): the scan's chains leave most issue cycles
// idle, and the prep fills them.  The scan starts once the first chunk's
// items are done (one item's latency, about 20 us at T = 4096 and 32 v-heads)
// and slows by a quarter while prep rounds share its CUs; both together cost
// less than the prep as a launch of its own.  Results are bit-identical to
// the two-launch form.
template <int SD, int C>
__global__ __launch_bounds__(256, 2) void delta_chunk_fused_kernel(DeltaArgs a, float* ws_T, float* ws_P,
                                                                   float* ws_e, uint8_t* ws_K,
                                                                   int n_chunks, int n_prep, int n_split,
                                                                   uint32_t* flags, uint32_t* err,
                                                                   uint32_t max_polls) {
    constexpr int PB = PrepLds<SD, C>::FLOATS * 4, SB = ScanLds<SD, C>::BYTES;
    __shared__ __attribute__((aligned(16))) uint8_t lds[PB > SB ? PB : SB];
    const int b = blockIdx.x;
    if (b < n_prep) {
        chunk_prep_body<SD, C, true, true>(a, ws_T, ws_P, ws_e, ws_K, n_chunks, b, n_prep,
                                           reinterpret_cast<float*>(lds), flags, n_split, 0);
    } else {
        const int j = b - n_prep;
        if (threadIdx.x == 0) __hip_atomic_store(err + 1 + j, xcc_id() + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (j < n_split) {
            // Above the prep workgroup sharing this CU, whose waves are older
            // and would otherwise issue first: the first chunk needs both halves.
            __builtin_amdgcn_s_setprio(1);
            chunk_prep_body<SD, C, true, true>(a, ws_T, ws_P, ws_e, ws_K, n_chunks, j, n_chunks * a.n_kh,
                                               reinterpret_cast<float*>(lds), flags, n_split, 1);
            __syncthreads();  // the scan reuses the LDS
        }
        chunk_scan_bf_body<SD, C, true>(a, reinterpret_cast<const uint8_t*>(ws_T),
                                        reinterpret_cast<const uint8_t*>(ws_P), ws_e, ws_K, n_chunks, j, lds,
                                        flags, err, max_polls);
    }
}

// Clears the one-launch form's flags, error word and registrations (a kernel,
// not a memset, so the call may sit in a captured graph).
__global__ __launch_bounds__(256) void delta_flags_clear_kernel(uint32_t* p, int n) {
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0u;
}

// Workspace: Tb and M [n_vh][n_chunks][chunk^2] floats (fp32 fragments, or
// split-bf16 pieces of the same size), the decays [n_vh][n_chunks][2 chunk],
// and, for the split path (chunks of 32 and 64), K and Q pieces
// [n_chunks][n_kh][2 chunk s_dim] floats' worth, then the one-launch form's
// ready flags [n_chunks][n_vh], its error word and the scan workgroups' XCD
// registrations [n_vh s_dim / 16].
static bool chunk_split(int chunk) { return chunk >= 32; }

static size_t chunk_ws_floats(const lmx_dop* op, int chunk) {
    const size_t n_chunks = (op->n_tok + chunk - 1) / chunk;
    const bool split = chunk_split(chunk);
    const size_t kq = split ? (size_t)op->n_kh * n_chunks * 2 * chunk * op->s_dim : 0;
    const size_t fl = split ? (size_t)op->n_vh * n_chunks + 1 + (size_t)op->n_vh * (op->s_dim / 16) : 0;
    return (size_t)op->n_vh * n_chunks * ((size_t)2 * chunk * chunk + 2 * chunk) + kq + fl;
}

size_t deltanet_chunked_ws(const lmx_dop* op, int chunk) {
    return (chunk_ws_floats(op, chunk) * 4 + 255) / 256 * 256;
}

// Workgroups of delta_chunk_fused_kernel the current GPU holds at once
// (occupancy x CUs), 0 if unknown; cached per device.
template <int SD, int C>
static int fused_slots() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v != 0) return v > 0 ? v : 0;
    int per_cu = 0, n_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void*>(&delta_chunk_fused_kernel<SD, C>), 256, 0) != hipSuccess ||
        hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        per_cu = n_cu = 0;
    v = per_cu * n_cu;
    cache[dev].store(v > 0 ? v : -1, std::memory_order_relaxed);
    return v > 0 ? v : 0;
}

template <int SD, int C>
static void launch_chunked(const DeltaArgs& a, int n_vh, int n_kh, int n_chunks, float* wsT,
                           float* wsP, float* wsE, uint8_t* wsK, uint32_t* wsF, hipStream_t st) {
    constexpr bool SPLIT = C >= 32;
    const int n_items = n_chunks * n_kh;
    if constexpr (SPLIT) {
        // One launch when the GPU holds more workgroups than the scan has, so
        // that a prep workgroup can always run.  Prep workgroups: one per item,
        // at most what the GPU holds beside the scan, rounded up to a multiple
        // of 8 where that fits (the extra ones have no item and exit) so that
        // scan workgroup j still runs on XCD j % 8 with the other row blocks
        // of its v-head.  A
        // round of items (one per prep workgroup, about 25 us beside the scan)
        // yields n_prep / n_kh chunks while the scan takes about ten, so with
        // fewer than 12 n_kh prep workgroups the scan would wait on the prep
        // and two launches are faster.
        const int n_scan = n_vh * (SD / 16);
        const int mode = tuning().delta_fused;
        const int slots = mode == 0 ? 0 : fused_slots<SD, C>();
        int n_prep = std::min(n_items, slots - n_scan);
        n_prep = std::min((n_prep + 7) & ~7, slots - n_scan);
        const bool starve = mode == 2;  // tests only: no prep, so every wait gives up
        if (starve) n_prep = 0;
        if (starve || (slots > n_scan && n_prep >= std::min(n_items, 12 * n_kh))) {
            const int n_flags = n_chunks * n_vh;
            const int n_words = n_flags + 1 + n_scan;  // flags, error word, registrations
            // the first round's items are shared with the scan workgroups when
            // a k-head has several v-heads
            const int n_split = n_vh > n_kh ? std::min(n_prep, std::min(n_scan, n_items)) : 0;
            const uint32_t max_polls = starve ? 64u : kFlagPolls;
            hipLaunchKernelGGL(delta_flags_clear_kernel, dim3((n_words + 255) / 256), dim3(256), 0, st,
                               wsF, n_words);
            hipLaunchKernelGGL((delta_chunk_fused_kernel<SD, C>), dim3(n_prep + n_scan), dim3(256), 0, st, a,
                               wsT, wsP, wsE, wsK, n_chunks, n_prep, n_split, wsF, wsF + n_flags, max_polls);
            return;
        }
    }
    hipLaunchKernelGGL((delta_chunk_prep_kernel<SD, C, SPLIT>), dim3(std::min(n_items, 2 * 256)), dim3(256), 0, st,
                       a, wsT, wsP, wsE, wsK, n_chunks);
    if constexpr (SPLIT)
        hipLaunchKernelGGL((delta_chunk_scan_bf_kernel<SD, C>), dim3(n_vh * (SD / 16)), dim3(256), 0, st,
                           a, reinterpret_cast<const uint8_t*>(wsT), reinterpret_cast<const uint8_t*>(wsP),
                           wsE, wsK, n_chunks);
    else
        hipLaunchKernelGGL((delta_chunk_scan_kernel<SD, C>), dim3(n_vh * (SD / 16)), dim3(256), 0, st,
                           a, wsT, wsP, wsE, n_chunks);
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
    float* wsE = wsP + per * chunk * chunk;
    uint8_t* wsK = reinterpret_cast<uint8_t*>(wsE + per * 2 * chunk);
    const int sd = (int)op->s_dim;
    uint32_t* wsF = reinterpret_cast<uint32_t*>(
        wsK + (chunk_split(chunk) ? (size_t)op->n_kh * n_chunks * 2 * chunk * sd * 4 : 0));
    (void)hipGetLastError();
#define LMX_CH(SDV, CV)                                                                          \
    if (sd == SDV && chunk == CV) {                                                              \
        launch_chunked<SDV, CV>(a, (int)op->n_vh, (int)op->n_kh, n_chunks, wsT, wsP, wsE, wsK, wsF, st); \
        LMX_CHECK_LAUNCH();                                                                      \
        return LMX_OK;                                                                           \
    }
    LMX_CH(128, 64) LMX_CH(128, 32) LMX_CH(128, 16)
    LMX_CH(64, 64) LMX_CH(64, 32) LMX_CH(64, 16)
#undef LMX_CH
    return LMX_E_UNSUPPORTED;
}

}  // namespace lmx
