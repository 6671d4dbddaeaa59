/*
 * lmx/attn.h -- C ABI of the MI355X (gfx950) attention hot path for llmoxide.
 *
 * One shared library, libllmoxide_amd.so, exports exactly the functions below.
 * They replace the wgpu dispatches that llmoxide's crates/gpu records for
 * attention, KV append and the gated delta rule; each declaration cites the
 * reference code it stands in for (paths relative to the llmoxide tree).
 *
 * Conventions (all entry points):
 *  - Plain C types only.  Device pointers are caller-owned HIP allocations;
 *    no entry point allocates, frees or synchronizes the host.  Work is
 *    enqueued on `stream` (a hipStream_t; NULL = the null stream) and is
 *    complete when that stream is.
 *  - Parameters are validated on the host before anything is enqueued.  A
 *    rejected call returns an LMX_E_* code and enqueues nothing.  No C++
 *    exception crosses the ABI.
 *  - Reentrant and thread-compatible: concurrent calls need distinct
 *    workspaces; one stream per caller thread mirrors the reference's
 *    Send + !Sync backend (llmoxide/src/backend.rs:57-62).
 *  - Layouts follow the reference buffers:
 *      q    [n_tokens, n_heads, head_dim]          (f32 or f16)
 *      out  [n_tokens, n_heads, head_dim]          f32
 *      K/V cache rows [n_slots, kv_dim], row = slot(pos)  (f16)
 *    kv head of query head h is h / (n_heads / n_kv_heads)  (attn.wgsl:78-80).
 */
#ifndef LMX_ATTN_H
#define LMX_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Binary-compatible with hipStream_t (typedef struct ihipStream_t*). */
typedef struct ihipStream_t *lmx_stream;

typedef enum {
    LMX_OK = 0,
    LMX_E_NULL = 1,           /* a required pointer is NULL                     */
    LMX_E_SHAPE = 2,          /* inconsistent or out-of-range geometry          */
    LMX_E_UNSUPPORTED = 3,    /* valid but not implemented (dtype, head_dim)    */
    LMX_E_WORKSPACE = 4,      /* workspace missing or too small                 */
    LMX_E_CONTEXT = 5,        /* positions exceed the cache (ContextOverflow)   */
    LMX_E_RING_HAZARD = 6,    /* windowed batch would read overwritten slots   */
    LMX_E_ALIGN = 7,          /* pointer not aligned as the layout requires     */
    LMX_E_LAUNCH = 8,         /* the HIP runtime rejected a launch              */
    LMX_E_DEVICE = 9,         /* no usable gfx950 device                        */
    LMX_E_FULL = 10,          /* no free sequence slot in a KV manager          */
    LMX_E_HOST = 11           /* host memory for bookkeeping ran out            */
} lmx_status;

typedef enum { LMX_F32 = 0, LMX_F16 = 1 } lmx_dtype;

/* The attention uniform, attn.wgsl:22-34 / qwen35.rs:36-49 / forward.rs:29-44,
 * minus max_vis (a scores-scratch stride this path does not need) and plus
 * n_slots (rows allocated in each cache buffer, for bounds validation). */
typedef struct {
    uint32_t n_tokens;    /* t >= 1, queries at base_pos .. base_pos+t-1      */
    uint32_t n_heads;     /* H, a multiple of n_kv_heads                      */
    uint32_t n_kv_heads;  /* Hkv                                              */
    uint32_t head_dim;    /* a multiple of 4 up to 512 (see below)            */
    uint32_t kv_dim;      /* cache row stride in elements, >= Hkv*head_dim    */
    uint32_t base_pos;    /* position of the batch's first token              */
    uint32_t window;      /* 0 = global linear cache, else ring of `window`   */
    uint32_t n_slots;     /* rows in each K/V cache buffer                    */
    uint32_t bidi;        /* 1 = the batch also attends forward to itself     */
    float scale;          /* softmax scale, applied verbatim                  */
} lmx_attn_params;

/* write_cache's view of one append, ops.wgsl:323-346 (Op{n_rows, dim, u0, u1}). */
typedef struct {
    uint32_t n_tokens;    /* rows to append                                   */
    uint32_t kv_dim;      /* elements per row                                 */
    uint32_t base_pos;    /* position of row 0                                */
    uint32_t window;      /* 0 = linear, else ring: slot = pos % window       */
    uint32_t n_slots;     /* rows allocated in the cache                      */
} lmx_kv_desc;

/* The delta-net uniform, deltanet.wgsl:20-34 / qwen35.rs:51-68, restricted to
 * what the recurrence reads.  Conv taps and the conv window belong to the
 * delta-net front (lmx_deltanet_front, below). */
typedef struct {
    uint32_t n_tok;       /* tokens in the batch                              */
    uint32_t conv_dim;    /* row stride of the conv stream, 2*key_dim+d_inner */
    uint32_t key_dim;     /* n_kh * s_dim                                     */
    uint32_t d_inner;     /* n_vh * s_dim                                     */
    uint32_t s_dim;       /* state side; 128 (64 also accepted)               */
    uint32_t n_vh;        /* value heads                                      */
    uint32_t n_kh;        /* key heads; v-head hv reads k-head hv % n_kh      */
    float scale;          /* output scale, 1/sqrt(s_dim) in the reference     */
} lmx_dop;

/* Human-readable name of a status code (static storage). */
const char *lmx_status_str(lmx_status s);

/* Library version as 10000*major + 100*minor + patch. */
int lmx_version(void);

/* Kernel-choice overrides (LMX_PREFILL_KERNEL, LMX_PREFILL_GP, LMX_PREFILL_KH,
 * LMX_DECODE_KROWS, LMX_DECODE_MH, LMX_DELTA_FUSED) are read from the
 * environment once, at the first launch.
 * This reads them again, for tests and tuning sweeps.  No reference
 * counterpart.  Not to be called while another thread launches. */
void lmx_tuning_reload(void);

/* Zero a workspace (a fill kernel, not hipMemsetAsync, so the call may sit
 * inside a captured graph).  No entry point needs a zeroed workspace: each
 * one writes every workspace byte it later reads within the same call. */
lmx_status lmx_workspace_init(void *ws, size_t ws_bytes, lmx_stream stream);

/* ------------------------------------------------------------------------
 * KV append.  Replaces the two `write_cache` dispatches per attention layer:
 * ops.wgsl:323-346, dispatched at qwen35.rs:1062-1074 and forward.rs:964-985;
 * CPU semantics LayerCache::store/slot, cache.rs:21-28, 58-62.
 * Row i of k_new/v_new ([n_tokens, kv_dim] f32) is rounded to f16 (RNE) and
 * stored at slot(base_pos + i).  When one call maps several rows to the same
 * ring slot, the latest position wins, as the reference's in-order store does.
 * Either of k_new/v_new (with its cache) may be NULL to append only the other.
 */
lmx_status lmx_kv_append(const lmx_kv_desc *d, const float *k_new, const float *v_new,
                         void *k_cache, void *v_cache, lmx_dtype cache_dt, lmx_stream stream);

/* ------------------------------------------------------------------------
 * Attention prologue.  Replaces, in one launch, the per-head rms_norm calls
 * (ops.wgsl:49-91), rope / rope_partial (ops.wgsl:269-306, 186-218) and the
 * two write_cache dispatches (ops.wgsl:323-346) in front of attention,
 * computing the CPU reference (cpu.rs:286-327; qwen35/cpu.rs:294-304).
 * For token i at pos = base_pos + i:
 *   each query head h (q + (i*n_heads + h)*q_stride, its first head_dim
 *   floats; a qwen35 head's gate half after them is untouched), in place:
 *     x <- rms_norm(x) * q_gain            (ops.rs:40-59; skipped if q_gain NULL)
 *     x[0:n_rot] <- rope_neox(x[0:n_rot])  (ops.rs:142-159; skipped if n_rot 0)
 *   each K head of k_new row i: the same with k_gain;
 *   each V head of v_new row i: rms_norm(x) without gain when v_norm;
 *   then the K and V rows are stored as lmx_kv_append stores them (f16 RNE at
 *   slot(pos); the latest position wins a ring slot).
 * rope_neox pairs dims (j, j + n_rot/2) with angle
 *   pos * rope_base^(-2j/n_rot) / factor_j  (factor_j = rope_factors[j], or 1
 *   when rope_factors is NULL), in double; the reference multiplies j times
 *   by rope_base^(-2/n_rot), this library by the bits of j, which agree to a
 *   few double ulps before sin/cos are rounded to float.
 * head_dim: 64, 128, 256 or 512; n_rot even, <= head_dim; q_stride >= head_dim.
 * k_new/v_new are read only. */
typedef struct {
    uint32_t n_tokens;    /* tokens in the batch                              */
    uint32_t n_heads;     /* query heads                                      */
    uint32_t n_kv_heads;  /* K/V heads; kv_dim = n_kv_heads*head_dim           */
    uint32_t head_dim;
    uint32_t q_stride;    /* floats from one query head to the next           */
    uint32_t n_rot;       /* leading dims of each head that rotate (0: none)  */
    uint32_t base_pos;    /* position of token 0                              */
    uint32_t window;      /* 0: linear cache; else ring of `window` slots     */
    uint32_t n_slots;     /* rows allocated in each cache                     */
    uint32_t v_norm;      /* 1: RMS-normalize V per head (Gemma)              */
    float rms_eps;
    float rope_base;
} lmx_prologue_desc;

lmx_status lmx_attn_prologue(const lmx_prologue_desc *d, float *q, const float *k_new,
                             const float *v_new, const float *q_gain, const float *k_gain,
                             const float *rope_factors, void *k_cache, void *v_cache,
                             lmx_dtype cache_dt, lmx_stream stream);

/* ------------------------------------------------------------------------
 * Attention.  Replaces the scores_pass / softmax_pass / weighted_v dispatch
 * triple (attn.wgsl:84-232) recorded at qwen35.rs:1076-1094 and
 * forward.rs:988-1011 (and vision.rs:587-631 with bidi=1), computing the CPU
 * reference's result (cpu.rs:342-387; qwen35/cpu.rs:324-365):
 *   out[i,h,:] = softmax_p(scale * q[i,h,:] . K[p, h/G, :]) V[p, h/G, :]
 * over the visible positions p of query pos = base_pos+i:
 *   lo = window ? max(0, pos-window+1) : 0
 *   hi = bidi ? (window ? min(base_pos+t-1, pos+window-1) : base_pos+t-1) : pos
 * K/V for position p are read from cache row slot(p) = window ? p%window : p,
 * except that positions >= base_pos are read from k_cur/v_cur row p-base_pos
 * when those are given ([n_tokens, kv_dim] f16).  The reference stores the
 * batch before attending, so a windowed batch with base_pos+t > window reads
 * slots that later rows of the same batch overwrote; this call refuses that
 * case (LMX_E_RING_HAZARD) unless k_cur/v_cur are given.
 * q_dt: LMX_F32 or LMX_F16.  kv_dt: LMX_F16.  out may not overlap q
 * (LMX_E_SHAPE): workgroups write out while others still read queries.
 * Workspace: lmx_attn_workspace_bytes(p) bytes, zeroed once by
 * lmx_workspace_init; 0 bytes may be asked for (ws may then be NULL).  It
 * holds the split partials of decode, and of prefill when a short batch on a
 * long cache is cut into key splits to fill the GPU.
 * head_dim: the kernels run 64, 128, 256 and 512 natively (rows 16-byte
 * aligned: kv_dim and q_stride multiples of 8, buffers 16-byte aligned).  Any
 * other multiple of 4 up to 512 (the reference's vec4 domain, attn.wgsl:36-46;
 * a vision tower's embedding_length / head_count) runs at the next native
 * size on zero-padded copies of Q, of the cache rows the call reads and of
 * k_cur/v_cur, held in the workspace, whose first head_dim output dims are
 * copied to out (gated there): kv_dim and q_stride multiples of 4, the f16
 * buffers 8-byte aligned.  The copies cost extra passes over those rows.
 * lmx_attn_decode_batched takes native sizes only.
 */
size_t lmx_attn_workspace_bytes(const lmx_attn_params *p);

lmx_status lmx_attn_fwd(const lmx_attn_params *p, const void *q, lmx_dtype q_dt,
                        const void *k_cache, const void *v_cache, lmx_dtype kv_dt,
                        const void *k_cur, const void *v_cur, float *out,
                        void *ws, size_t ws_bytes, lmx_stream stream);

/* ------------------------------------------------------------------------
 * lmx_attn_fwd without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation).  No counterpart in the
 * reference: its attention passes share a scratch buffer the model allocates
 * at load (qwen35.rs:480).  Same parameters, semantics and results as
 * lmx_attn_fwd; the split partials go to a library-owned scratch array of
 * LMX_NOALLOC_SCRATCH_BYTES per GPU (resident from the library's first use
 * on that GPU until the process ends).  Returns LMX_E_WORKSPACE, enqueuing
 * nothing, when the call needs more (lmx_attn_workspace_bytes(p) is the
 * need): a 32k-token decode at Qwen3-8B shape needs about 2 MiB, a
 * 512-token chunk on a 4k cache about 34 MiB.  No entry point allocates,
 * and this one takes no workspace either.  The scratch used is that of the
 * device `stream` belongs to (the current device for the null stream).
 * Every call on one GPU shares that GPU's scratch, so calls that overlap on
 * one GPU (concurrent streams, or threads) race; serialize them on one
 * stream.  The array lives in the library's code object, so every process
 * that loads the library holds it on each GPU the library runs on, whether
 * or not it calls this entry point.  Its address is cached per device: after
 * hipDeviceReset on a device, do not call this entry point there again in
 * the same process. */
#define LMX_NOALLOC_SCRATCH_BYTES (64u << 20)

lmx_status lmx_attn_fwd_noalloc(const lmx_attn_params *p, const void *q, lmx_dtype q_dt,
                                const void *k_cache, const void *v_cache, lmx_dtype kv_dt,
                                const void *k_cur, const void *v_cur, float *out,
                                lmx_stream stream);

/* ------------------------------------------------------------------------
 * Attention with Qwen3.5's fused query heads and sigmoid output gate (the
 * epilogue of the attention block).  The CPU reference reads query head h of
 * token i in place at q + (i*n_heads + h)*q_stride (q_stride = 2*head_dim when
 * the projection interleaves [query | gate] per head) and multiplies the
 * head's output by sigmoid(gate), gate being the second half of the same pair
 * (qwen35/cpu.rs:333-337, 359-363; sigmoid ops.rs:181-183).  The GPU reference
 * deinterleaves with split_half and gates with mul_sigmoid (ops.wgsl:150-184,
 * recorded at qwen35.rs:1012-1028 and 1098-1107): three more dispatches and
 * two more passes over the activations.  Here q is read at its stride and the
 * gate is applied where the output is written; no extra pass.
 *   x == NULL is lmx_attn_fwd.  Else:
 *   q_stride     elements between consecutive query heads (0: head_dim);
 *                a multiple of 8, >= head_dim
 *   gate         NULL: no gate; else out[i,h,d] *= 1/(1+exp(-g)) with
 *                g = gate[(i*n_heads + h)*gate_stride + d], 16-byte aligned
 *   gate_stride  floats between consecutive gate heads (0: head_dim);
 *                a multiple of 4, >= head_dim
 * gate may point into q's buffer (q + head_dim for the fused layout); out may
 * not overlap q or gate.  Same workspace as lmx_attn_fwd. */
typedef struct {
    uint32_t q_stride;
    uint32_t gate_stride;
    const float *gate;
} lmx_attn_ext;

lmx_status lmx_attn_fwd_ext(const lmx_attn_params *p, const lmx_attn_ext *x, const void *q,
                            lmx_dtype q_dt, const void *k_cache, const void *v_cache,
                            lmx_dtype kv_dt, const void *k_cur, const void *v_cur, float *out,
                            void *ws, size_t ws_bytes, lmx_stream stream);

/* ------------------------------------------------------------------------
 * Ragged multi-sequence decode: one query token per sequence, each sequence
 * with its own contiguous cache.  The reference serves one sequence at a time
 * (docs/limitations.md:21); this is the batched form of lmx_attn_fwd with
 * n_tokens = 1 and, for sequence b, base_pos = ctx_lens[b]-1.  With n_seq = 1
 * it computes exactly what lmx_attn_fwd does.
 *   p          geometry; n_tokens must be 1 and base_pos is ignored
 *   ctx_lens   device int32 [n_seq], each in [1, max_ctx], max_ctx <= n_slots
 *   k_ptrs     device array [n_seq] of f16 cache pointers (likewise v_ptrs)
 *   q          [n_seq, n_heads, head_dim];  out [n_seq, n_heads, head_dim] f32
 */
size_t lmx_attn_decode_batched_workspace_bytes(const lmx_attn_params *p, int32_t n_seq,
                                               int32_t max_ctx);

lmx_status lmx_attn_decode_batched(const lmx_attn_params *p, int32_t n_seq, int32_t max_ctx,
                                   const int32_t *ctx_lens, const void *const *k_ptrs,
                                   const void *const *v_ptrs, const void *q, lmx_dtype q_dt,
                                   lmx_dtype kv_dt, float *out, void *ws, size_t ws_bytes,
                                   lmx_stream stream);

/* ------------------------------------------------------------------------
 * Gated delta rule, token-sequential.  Replaces `delta_recur`
 * (deltanet.wgsl:193-239, dispatched at qwen35.rs:960-965); CPU semantics
 * qwen35/cpu.rs:218-245.  Per token i and v-head hv (k-head hk = hv % n_kh):
 *   g = exp(ssm_a[hv] * softplus(alpha[i,hv] + dt_bias[hv])), b = sigmoid(beta[i,hv])
 *   S <- g S;  for each row j: d = b (v_j - S_j . k);  S_j += d k;  o_j = scale S_j . q
 *   conv   [n_tok, conv_dim] f32, channels q | k | v, q and k L2-normalized
 *   alpha, beta [n_tok, n_vh] f32;  ssm_a, dt_bias [n_vh] f32
 *   state  [n_vh, s_dim (row j), s_dim] f32, updated in place
 *   out    [n_tok, d_inner] f32
 */
lmx_status lmx_deltanet_recur(const lmx_dop *op, const float *ssm_a, const float *dt_bias,
                              const float *alpha, const float *beta, const float *conv,
                              float *state, float *out, lmx_stream stream);

/* ------------------------------------------------------------------------
 * Gated delta rule, chunked (chunk tokens at a time, WY/UT form).  Same
 * contract and results as lmx_deltanet_recur within the stated tolerance; the
 * reference has no chunked form (it runs the token loop in one workgroup per
 * head, deltanet.wgsl:175-239), so this is the prefill counterpart of the same
 * dispatch.  chunk: 64 (or 32, 16).  Chunks of 32 and 64 form their products
 * on bf16 matrix cores from split (hi + lo) operands with fp32 accumulation
 * (about 1e-5 relative to fp32 products); the state stays fp32.  They run as
 * a small flag-clearing kernel and one kernel in which the per-chunk factors
 * are built beside the chunk chain (as two kernels when the GPU would not hold
 * enough workgroups for both); the results are bit-identical either way.
 */
size_t lmx_deltanet_chunked_workspace_bytes(const lmx_dop *op, int32_t chunk);

lmx_status lmx_deltanet_chunked(const lmx_dop *op, const float *ssm_a, const float *dt_bias,
                                const float *alpha, const float *beta, const float *conv,
                                float *state, float *out, int32_t chunk, void *ws,
                                size_t ws_bytes, lmx_stream stream);

/* ------------------------------------------------------------------------
 * Delta-net front.  Replaces the conv_silu, conv_shift, conv_commit and
 * l2norm_qk dispatches (deltanet.wgsl:54-173, recorded at qwen35.rs:928-958)
 * with one launch, computing the CPU reference (qwen35/cpu.rs:193-216):
 *   conv_out[i][c] = silu(x[i][c]*taps[c][K-1] + sum_{j<K-1} w_j[c]*taps[c][j])
 * where w_j is row j of the window [conv_state | x] as seen by token i (the
 * K-1 rows before it, oldest first), silu(a) = a/(1+exp(-a)) (ops.rs:175-178);
 * then each q and k head (channels [0, 2*key_dim) in heads of s_dim) is
 * L2-normalized, x / max(||x||, eps) (ops.rs:197-203).  conv_state ([K-1,
 * conv_dim], oldest first) becomes the last K-1 rows of [conv_state | x].
 * conv_out [n_tok, conv_dim] is what lmx_deltanet_recur/_chunked read.
 * conv_dim a multiple of 128; s_dim 64 or 128; 2 <= kernel <= 8. */
typedef struct {
    uint32_t n_tok;       /* tokens in the batch                              */
    uint32_t conv_dim;    /* channels: q (key_dim) | k (key_dim) | v          */
    uint32_t key_dim;     /* n_kh * s_dim                                     */
    uint32_t s_dim;       /* head size of the q/k L2 norm                     */
    uint32_t kernel;      /* conv taps per channel (4 in qwen35)              */
    float eps;            /* floor of the L2 norm                             */
} lmx_delta_front_desc;

lmx_status lmx_deltanet_front(const lmx_delta_front_desc *d, const float *x, const float *taps,
                              float *conv_state, float *conv_out, lmx_stream stream);

/* Delta-net back.  Replaces the rms_norm + mul_silu pair after the
 * recurrence (qwen35.rs:968-986), computing qwen35/cpu.rs:250-259 in place:
 * per token and v-head, o <- rms_norm(o) * w * silu(z), with rms_norm as
 * ops.rs:40-47 (eps inside the root).  o, z [n_tok, n_vh*s_dim]; w [s_dim];
 * s_dim 64, 128 or 256. */
typedef struct {
    uint32_t n_tok;
    uint32_t n_vh;
    uint32_t s_dim;
    float eps;
} lmx_delta_back_desc;

lmx_status lmx_deltanet_back(const lmx_delta_back_desc *d, float *o, const float *z,
                             const float *w, lmx_stream stream);

/* ------------------------------------------------------------------------
 * Quantized matrix-vector product: y[t] = W x[t], the attention epilogue's
 * attn_output projection (qwen35.rs:1098-1109; forward.rs after attention) and
 * any projection of the same form.  Replaces the reference's matvec_*
 * dispatches (quant.wgsl:76-826) and computes what its CPU reference
 * `dot_row` computes (crates/gguf/src/quant.rs:187-271).
 *   W  rows x in_dim in ggml's on-disk row-major block layout: type 12 Q4_K
 *      (144-byte blocks of 256), 14 Q6_K (210-byte blocks of 256, read in
 *      place, no repacking), 8 Q8_0 (34-byte blocks of 32), 0 F32, 1 F16,
 *      30 BF16; 16-byte aligned
 *   x  [n_tok, in_dim] f32, y [n_tok, rows] f32, 16-byte aligned, disjoint
 * in_dim: a multiple of 256 (Q4_K, Q6_K) or 64 (the others), at most 16384.
 * Below 16 tokens (and for the dense types) tokens go four per launch, each
 * launch reading W once.  From 16 tokens (the reference's GEMM_MIN_TOKENS,
 * crates/gpu/src/lib.rs:1083; its GEMM is gemm_q6k, gemm.wgsl:93-95) a Q4_K,
 * Q6_K or Q8_0 matrix with in_dim a multiple of 128 goes through one
 * matrix-core GEMM launch that reads W once; it computes each block's
 * integer dot products exactly and applies the block scales in fp32, and
 * needs |x| < 65504 (the f16 range; attention outputs over an f16 V cache
 * always are). */
typedef struct {
    uint32_t type;
    uint32_t rows;
    uint32_t in_dim;
    uint32_t n_tok;
} lmx_qmv_desc;

lmx_status lmx_matvec(const lmx_qmv_desc *d, const void *w, const float *x, float *y,
                      lmx_stream stream);

/* ------------------------------------------------------------------------
 * Multi-sequence KV manager.  The reference serves one sequence at a time
 * (docs/limitations.md:21): one KvCache per session (cache.rs:65-154), sized
 * per layer as kv_slots (config.rs:279-284: min(window, n_ctx) ring slots for
 * a windowed layer, n_ctx for a global one), with layers that share an
 * earlier layer's cache allocating nothing (cache.rs:86-104), and the
 * session's prefix reuse (session.rs:497-513, 546-570).  This keeps that
 * bookkeeping for up to max_seqs sequences whose f16 caches live in one
 * caller-allocated device arena, and hands out what the attention entry
 * points take: a sequence's per-layer cache pointers for appends, prologues
 * and prefill, and the pointer / length tables of lmx_attn_decode_batched for
 * a ragged batch.
 *
 * HBM layout: sequence s owns bytes [s*slab, (s+1)*slab) of the arena; inside
 * it every cache-owning layer has a K block then a V block of
 * [slots, kv_dim] f16 rows (the reference's row-major-by-slot layout,
 * cache.rs:10-18), each block 256-byte aligned.  Host bookkeeping only: no
 * call but lmx_kvm_wipe/lmx_kvm_begin enqueues device work, none allocates
 * device memory, none synchronizes.  A manager is not thread-safe; calls on
 * one manager must be serialized by the caller. */
typedef struct lmx_kvm lmx_kvm;

typedef struct {
    uint32_t window;     /* 0: global (linear, n_ctx slots); else ring of min(window, n_ctx) */
    uint32_t kv_dim;     /* elements per cache row (a multiple of 8)                          */
    int32_t kv_source;   /* -1: owns its cache; else an earlier layer whose cache it reads    */
} lmx_kvm_layer;

typedef struct {
    uint32_t n_layers;
    uint32_t n_ctx;              /* positions per sequence                 */
    uint32_t max_seqs;           /* sequence slots in the arena            */
    const lmx_kvm_layer *layers; /* [n_layers]                             */
} lmx_kvm_desc;

/* Device bytes the arena needs (0 for an invalid description). */
size_t lmx_kvm_arena_bytes(const lmx_kvm_desc *d);

lmx_status lmx_kvm_create(const lmx_kvm_desc *d, void *arena, size_t arena_bytes, lmx_kvm **out);
void lmx_kvm_destroy(lmx_kvm *m);

/* Claim an empty sequence slot (LMX_E_FULL when none is free) / release one. */
lmx_status lmx_kvm_open(lmx_kvm *m, int32_t *seq);
lmx_status lmx_kvm_close(lmx_kvm *m, int32_t seq);

/* Positions written so far: the next token lands at this position. */
lmx_status lmx_kvm_len(const lmx_kvm *m, int32_t seq, uint32_t *len);

/* session.rs:497-513: how much of the prompt tokens[0, n) the resident cache
 * serves.  Only a strict prefix of what is resident counts (ring layers have
 * already overwritten anything before a rewind point), and nothing once an
 * embedding span made the resident ids incomplete. */
lmx_status lmx_kvm_reusable_prefix(const lmx_kvm *m, int32_t seq, const int32_t *tokens,
                                   uint32_t n, uint32_t *reuse);

/* A new turn with prompt tokens[0, n) (session.rs:546-553): *reuse is the
 * reusable prefix; when it is 0 the sequence's caches are overwritten with
 * zeros on `stream` and its bookkeeping reset, as the reference wipes before
 * an unrelated conversation.  The caller then runs positions [*reuse, n) and
 * commits them.  LMX_E_CONTEXT when n > n_ctx. */
lmx_status lmx_kvm_begin(lmx_kvm *m, int32_t seq, const int32_t *tokens, uint32_t n,
                         uint32_t *reuse, lmx_stream stream);

/* Record that the caller appended n rows at positions [len, len + n):
 * len += n and the ids join the resident list (session.rs:568, 607-609).
 * tokens == NULL marks rows from an embedding span: the sequence stops being
 * comparable for prefix reuse (session.rs:569-571).  LMX_E_CONTEXT when
 * len + n > n_ctx; LMX_E_RING_HAZARD on a sequence a truncate left stale. */
lmx_status lmx_kvm_commit(lmx_kvm *m, int32_t seq, const int32_t *tokens, uint32_t n);

/* cache.rs:146-149: drop everything from pos onward (len = min(len, pos)).
 * A ring layer stores position p in slot p % ring, so once positions past
 * the new end have been written, the slots of some positions the next query
 * at len must see hold later ones (a ring of w >= 2 slots, positions [0, hw)
 * written since the last wipe: stale when hw >= len + 2 and hw >= w + 1).
 * Such a truncate leaves the sequence stale: it is no longer comparable for
 * prefix reuse (so the next lmx_kvm_begin wipes it), and lmx_kvm_commit and
 * lmx_kvm_batch return LMX_E_RING_HAZARD for it until it is wiped. */
lmx_status lmx_kvm_truncate(lmx_kvm *m, int32_t seq, uint32_t pos);

/* cache.rs:138-143: zero the sequence's caches on `stream`, len = 0. */
lmx_status lmx_kvm_wipe(lmx_kvm *m, int32_t seq, lmx_stream stream);

/* The caches layer `layer` of sequence `seq` reads and writes (a sharing
 * layer's are its source's): f16 [n_slots, kv_dim]; *window is what
 * lmx_kv_desc / lmx_attn_params take (0 linear, else the ring size). */
lmx_status lmx_kvm_layer_cache(const lmx_kvm *m, int32_t seq, uint32_t layer, void **k,
                               void **v, uint32_t *n_slots, uint32_t *window);

/* Host tables of lmx_attn_decode_batched for layer `layer` over seqs[0, n):
 * k_ptrs/v_ptrs[b] = the sequence's caches, ctx_lens[b] = its len + extra
 * (extra: rows appended for this step but not yet committed, 1 for a decode
 * step), *max_ctx = the largest.  The caller copies the tables to the device.
 * LMX_E_RING_HAZARD when a sequence was left stale by lmx_kvm_truncate. */
lmx_status lmx_kvm_batch(const lmx_kvm *m, uint32_t layer, const int32_t *seqs, uint32_t n,
                         uint32_t extra, const void **k_ptrs, const void **v_ptrs,
                         int32_t *ctx_lens, int32_t *max_ctx);

#ifdef __cplusplus
}
#endif

#endif /* LMX_ATTN_H */
