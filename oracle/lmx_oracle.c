/*
 * lmx_oracle.c -- CPU restatement of llmoxide's attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (llmoxide_amd/, include/)
 * links, loads or calls this file.  It is the parity checker for the HIP
 * kernels and the CPU baseline that bench.py reports next to the GPU figure.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.
 *
 * Every function follows a named piece of the reference (paths relative to the
 * llmoxide source tree) and keeps its loop and summation order: plain f32,
 * products rounded before the add (built with -ffp-contract=off, no fast-math),
 * libm expf / logf as Rust's f32::exp / ln call them on Linux.
 *
 * Parity pins (checked in tests/test_oracle_*.py):
 *   orc_rng_*            crates/model/src/sample.rs:73-92, pinned by
 *                        a hand-computed xorshift64* trace.
 *   orc_f32_to_f16 /     IEEE binary16 round-to-nearest-even, pinned against
 *   orc_f16_to_f32       numpy's float16 over all 65536 codes and 1e6 floats.
 *   orc_slot/visible     crates/model/src/cache.rs:21-38 + attn.wgsl:52-80,
 *                        pinned by the ported known-answer tests
 *                        (cache.rs:169-204) and brute-force enumeration.
 *   orc_softmax          crates/model/src/ops.rs:119-135, pinned by the ported
 *                        KATs (ops.rs:259-273) and float64 closed form.
 *   orc_write_cache      ops.wgsl:323-346 / cache.rs:58-62, pinned by a
 *                        brute-force last-writer-wins simulation.
 *   orc_attention        crates/model/src/cpu.rs:342-387 and
 *                        crates/model/src/qwen35/cpu.rs:324-365, pinned by an
 *                        independent float64 matrix-form implementation, by
 *                        torch scaled_dot_product_attention with an explicit
 *                        mask, and by invariants (one visible key -> out = v,
 *                        GQA == head-expanded MHA, constant V -> out = V).
 *   orc_rope_neox        crates/model/src/ops.rs:142-159, pinned by the ported
 *                        KATs (ops.rs:225-257) and a float64 closed form.
 *   orc_attn_prologue    the per-head norm / rotate / store sequence of
 *                        crates/model/src/cpu.rs:286-327 and
 *                        crates/model/src/qwen35/cpu.rs:294-304, pinned by a
 *                        float64 restatement and by invariants (unit RMS,
 *                        norm-preserving pairs, pos 0 and 1e30 factors leave
 *                        the head as normalized).
 *   orc_delta_front      crates/model/src/qwen35/cpu.rs:193-216 (conv + SiLU,
 *                        window shift, q/k L2 norm), pinned by a float64
 *                        restatement and by invariants (identity taps give
 *                        silu(x); two calls chained equal one call; unit-norm
 *                        q/k heads).
 *   orc_delta_back       crates/model/src/qwen35/cpu.rs:250-259 (gated RMS
 *                        norm), pinned by a float64 restatement.
 *   orc_dequant / orc_dot_row / orc_matvec
 *                        crates/gguf/src/quant.rs:33-260: ggml's Q4_K, Q6_K
 *                        and Q8_0 blocks (on-disk layouts) and F32/F16/BF16
 *                        rows, decoded and dotted in the reference's order;
 *                        pinned by the reference's tests (quant.rs:301-415)
 *                        and by a float64 decoder written from the layout.
 *   orc_attn_gate        crates/model/src/qwen35/cpu.rs:359-363 with
 *                        ops::sigmoid (ops.rs:181-183): the attention output
 *                        times sigmoid(gate); pinned by its special values
 *                        (gate 0 halves, large gates pass or zero) and a
 *                        float64 restatement.
 *   orc_delta_recur      crates/model/src/qwen35/cpu.rs:218-245 (and the GPU
 *                        form deltanet.wgsl:193-239), pinned by a float64
 *                        matrix restatement and by invariants (exact write at
 *                        g=1,beta=1 with unit k; beta=0 pure decay; linearity
 *                        in v; orthonormal keys write independently).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ rng -- */
/* xorshift64*, crates/model/src/sample.rs:73-92. */
typedef struct { uint64_t s; } orc_rng;

void orc_rng_init(orc_rng *r, uint64_t seed) {
    r->s = (seed * 0x9E3779B97F4A7C15ull) | 1ull;
}

float orc_rng_next_f32(orc_rng *r) {
    uint64_t x = r->s;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    r->s = x;
    return (float)((x * 0x2545F4914F6CDD1Dull) >> 40) / (float)(1u << 24);
}

/* n uniforms in [0,1) from one seed. */
void orc_fill_uniform(uint64_t seed, float *out, size_t n) {
    orc_rng r;
    orc_rng_init(&r, seed);
    for (size_t i = 0; i < n; ++i) out[i] = orc_rng_next_f32(&r);
}

/* n N(0,1) draws: Box-Muller, one normal per pair of uniforms, u1 -> 1-u1 so
 * the log argument is in (0,1].  Computed in double, rounded to f32 once. */
void orc_fill_normal(uint64_t seed, float *out, size_t n) {
    orc_rng r;
    orc_rng_init(&r, seed);
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; ++i) {
        double u1 = 1.0 - (double)orc_rng_next_f32(&r);
        double u2 = (double)orc_rng_next_f32(&r);
        out[i] = (float)(sqrt(-2.0 * log(u1)) * cos(two_pi * u2));
    }
}

/* ------------------------------------------------------------------ f16 -- */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ex = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (ex == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
    int e = (int)ex - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        int shift = 14 - e;
        uint32_t h = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t ex = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t man = (uint32_t)h & 0x3ffu;
    uint32_t x;
    if (ex == 0) {
        if (man == 0) {
            x = sign;
        } else {
            int e = -1;
            do { man <<= 1; ++e; } while (!(man & 0x400u));
            man &= 0x3ffu;
            x = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (ex == 31) {
        x = sign | 0x7f800000u | (man << 13);
    } else {
        x = sign | ((ex - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void orc_to_f16(const float *in, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16(in[i]);
}

void orc_from_f16(const uint16_t *in, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32(in[i]);
}

/* --------------------------------------------------------- bookkeeping -- */
/* cache.rs:21-28 (LayerCache::slot), attn.wgsl:68-71 (cache_slot). */
int64_t orc_slot(int64_t pos, int64_t window) {
    return window ? pos % window : pos;
}

/* Visible key positions [*lo, *hi] of the query at `pos`.
 * Causal: cache.rs:30-38 (visible), attn.wgsl:52-56 (first_visible).
 * Bidirectional end: cpu.rs:351-360, attn.wgsl:58-66 (last_visible). */
void orc_visible(int64_t pos, int64_t window, int64_t base_pos, int64_t n_tokens,
                 int bidi, int64_t *lo, int64_t *hi) {
    *lo = window ? (pos + 1 <= window ? 0 : pos + 1 - window) : 0;
    if (!bidi) {
        *hi = pos;
    } else {
        int64_t end = base_pos + n_tokens - 1;
        if (!window) {
            *hi = end;
        } else {
            int64_t h = pos + window - 1;
            *hi = end < h ? end : h;
        }
    }
}

/* ------------------------------------------------------------- softmax -- */
/* ops.rs:119-135: max-subtracted, an all -inf row becomes zeros. */
void orc_softmax(float *x, size_t n) {
    float mx = -INFINITY;
    for (size_t i = 0; i < n; ++i) mx = fmaxf(mx, x[i]);
    if (!isfinite(mx)) {
        for (size_t i = 0; i < n; ++i) x[i] = 0.0f;
        return;
    }
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; ++i) x[i] *= inv;
}

/* --------------------------------------------------------- write_cache -- */
/* ops.wgsl:323-346 and cache.rs:58-62: row i of the batch lands in slot
 * slot(base_pos + i); rows are stored in order, so within one call a later
 * position that maps to the same ring slot wins.  The cache holds f16. */
void orc_write_cache(int64_t n_tokens, int64_t kv_dim, int64_t base_pos,
                     int64_t window, const float *src, uint16_t *cache) {
    for (int64_t i = 0; i < n_tokens; ++i) {
        int64_t s = orc_slot(base_pos + i, window);
        for (int64_t d = 0; d < kv_dim; ++d)
            cache[s * kv_dim + d] = orc_f32_to_f16(src[i * kv_dim + d]);
    }
}

/* ----------------------------------------------------------- attention -- */
typedef struct {
    uint32_t n_tokens, n_heads, n_kv_heads, head_dim, kv_dim;
    uint32_t base_pos, window, bidi;
    float scale;
} orc_attn;

typedef struct {
    const orc_attn *p;
    const float *q, *k, *v;
    float *out;
    int linear;           /* 1: k/v indexed by position; 0: by ring slot */
    int64_t begin, end;   /* (token, head) work items [begin, end) */
} orc_attn_job;

static void *orc_attn_run(void *arg) {
    const orc_attn_job *j = (const orc_attn_job *)arg;
    const orc_attn *p = j->p;
    const int64_t hd = p->head_dim, kvd = p->kv_dim, H = p->n_heads;
    const int64_t group = p->n_heads / p->n_kv_heads;
    const int64_t win = p->window;
    int64_t cap = (int64_t)p->base_pos + p->n_tokens + 1;
    float *scores = (float *)malloc(sizeof(float) * (size_t)cap);
    for (int64_t item = j->begin; item < j->end; ++item) {
        const int64_t i = item / H, hq = item % H;
        const int64_t pos = (int64_t)p->base_pos + i;
        int64_t lo, hi;
        orc_visible(pos, win, p->base_pos, p->n_tokens, (int)p->bidi, &lo, &hi);
        const int64_t n_vis = hi - lo + 1;
        const int64_t kv_head = hq / group;
        const float *qh = j->q + (i * H + hq) * hd;
        /* cpu.rs:362-368: scores over the window, sequential f32 sum. */
        for (int64_t s = 0; s < n_vis; ++s) {
            const int64_t pp = lo + s;
            const int64_t row = j->linear ? pp : orc_slot(pp, win);
            const float *kh = j->k + row * kvd + kv_head * hd;
            float acc = 0.0f;
            for (int64_t d = 0; d < hd; ++d) acc += qh[d] * kh[d];
            scores[s] = acc * p->scale;
        }
        orc_softmax(scores, (size_t)n_vis);
        /* cpu.rs:371-385: weighted sum, zero weights skipped. */
        float *out = j->out + (i * H + hq) * hd;
        for (int64_t d = 0; d < hd; ++d) out[d] = 0.0f;
        for (int64_t s = 0; s < n_vis; ++s) {
            const float w = scores[s];
            if (w == 0.0f) continue;
            const int64_t pp = lo + s;
            const int64_t row = j->linear ? pp : orc_slot(pp, win);
            const float *vh = j->v + row * kvd + kv_head * hd;
            for (int64_t d = 0; d < hd; ++d) out[d] += w * vh[d];
        }
    }
    free(scores);
    return NULL;
}

/* Attention over K/V rows.  linear = 0 reads the reference's cache layout:
 * rows are ring slots, the batch has already been stored (cpu.rs:332-339 then
 * 343-387).  linear = 1 reads rows by absolute position (the documented window
 * semantics over keys that hold every visible position).  n_threads > 1 splits
 * the (token, head) items over pthreads; each item's arithmetic is unchanged.
 * Returns 0, or -1 on an invalid shape. */
int orc_attention(const orc_attn *p, const float *q, const float *k,
                  const float *v, float *out, int linear, int n_threads) {
    if (!p->n_tokens || !p->n_heads || !p->n_kv_heads || !p->head_dim) return -1;
    if (p->n_heads % p->n_kv_heads) return -1;
    if (p->kv_dim < p->n_kv_heads * p->head_dim) return -1;
    const int64_t items = (int64_t)p->n_tokens * p->n_heads;
    if (n_threads < 1) n_threads = 1;
    if (n_threads > items) n_threads = (int)items;
    orc_attn_job jobs[256];
    pthread_t th[256];
    if (n_threads > 256) n_threads = 256;
    for (int t = 0; t < n_threads; ++t) {
        jobs[t].p = p;
        jobs[t].q = q;
        jobs[t].k = k;
        jobs[t].v = v;
        jobs[t].out = out;
        jobs[t].linear = linear;
        jobs[t].begin = items * t / n_threads;
        jobs[t].end = items * (t + 1) / n_threads;
    }
    if (n_threads == 1) {
        orc_attn_run(&jobs[0]);
        return 0;
    }
    /* a thread that fails to start has its slice run here instead */
    int started[256];
    for (int t = 0; t < n_threads; ++t) {
        started[t] = pthread_create(&th[t], NULL, orc_attn_run, &jobs[t]) == 0;
        if (!started[t]) orc_attn_run(&jobs[t]);
    }
    for (int t = 0; t < n_threads; ++t)
        if (started[t]) pthread_join(th[t], NULL);
    return 0;
}

/* --------------------------------------------------------- delta rule -- */
typedef struct {
    uint32_t n_tok, conv_dim, key_dim, d_inner, s_dim, n_vh, n_kh;
    float scale; /* 1/sqrt(s_dim), qwen35.rs:923 / qwen35/cpu.rs:166 */
} orc_dop;

/* ops.rs:187-193 */
static float orc_softplus(float x) { return x > 20.0f ? x : logf(1.0f + expf(x)); }
/* ops.rs:181-183 */
static float orc_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* qwen35/cpu.rs:218-245: the gated delta rule over n_tok tokens.
 *   conv   [n_tok, conv_dim]  channels q(key_dim) | k(key_dim) | v(d_inner),
 *                             q and k already L2-normalized per head
 *   alpha  [n_tok, n_vh]      raw decay projection
 *   beta   [n_tok, n_vh]      raw mixing projection
 *   ssm_a, dt_bias [n_vh]
 *   S      [n_vh, s_dim (value row j), s_dim (key col)]  updated in place
 *   out    [n_tok, d_inner]
 * The v-head -> k-head map tiles: hk = hv % n_kh (cpu.rs:220). */
static void orc_delta_heads(const orc_dop *op, const float *ssm_a, const float *dt_bias,
                            const float *alpha, const float *beta, const float *conv,
                            float *S, float *out, int64_t hv_begin, int64_t hv_end) {
    const int64_t sd = op->s_dim;
    for (int64_t i = 0; i < op->n_tok; ++i) {
        const float *row_c = conv + i * op->conv_dim;
        const float *qn = row_c;
        const float *kn = row_c + op->key_dim;
        const float *vals = row_c + 2 * op->key_dim;
        float *o = out + i * op->d_inner;
        for (int64_t hv = hv_begin; hv < hv_end; ++hv) {
            const int64_t hk = (hv % op->n_kh) * sd;
            const float *qh = qn + hk, *kh = kn + hk, *vh = vals + hv * sd;
            const float g = expf(ssm_a[hv] * orc_softplus(alpha[i * op->n_vh + hv] + dt_bias[hv]));
            const float bmix = orc_sigmoid(beta[i * op->n_vh + hv]);
            float *sh = S + hv * sd * sd;
            for (int64_t x = 0; x < sd * sd; ++x) sh[x] *= g;
            float *oh = o + hv * sd;
            for (int64_t jr = 0; jr < sd; ++jr) {
                float *r = sh + jr * sd;
                float pred = 0.0f;
                for (int64_t d = 0; d < sd; ++d) pred += r[d] * kh[d];
                const float delta = (vh[jr] - pred) * bmix;
                for (int64_t d = 0; d < sd; ++d) r[d] += delta * kh[d];
                float acc = 0.0f;
                for (int64_t d = 0; d < sd; ++d) acc += r[d] * qh[d];
                oh[jr] = acc * op->scale;
            }
        }
    }
}

void orc_delta_recur(const orc_dop *op, const float *ssm_a, const float *dt_bias,
                     const float *alpha, const float *beta, const float *conv,
                     float *S, float *out) {
    orc_delta_heads(op, ssm_a, dt_bias, alpha, beta, conv, S, out, 0, op->n_vh);
}

typedef struct {
    const orc_dop *op;
    const float *ssm_a, *dt_bias, *alpha, *beta, *conv;
    float *S, *out;
    int64_t begin, end;
} orc_delta_job;

static void *orc_delta_run(void *arg) {
    const orc_delta_job *j = (const orc_delta_job *)arg;
    orc_delta_heads(j->op, j->ssm_a, j->dt_bias, j->alpha, j->beta, j->conv, j->S, j->out,
                    j->begin, j->end);
    return NULL;
}

/* The same recurrence with the v-heads split over n_threads pthreads.  The
 * heads are independent (each owns its S and its output columns), so every
 * value is computed by the same operations in the same order as above. */
void orc_delta_recur_mt(const orc_dop *op, const float *ssm_a, const float *dt_bias,
                        const float *alpha, const float *beta, const float *conv,
                        float *S, float *out, int n_threads) {
    if (n_threads < 1) n_threads = 1;
    if (n_threads > (int)op->n_vh) n_threads = (int)op->n_vh;
    if (n_threads > 256) n_threads = 256;
    if (n_threads == 1) {
        orc_delta_heads(op, ssm_a, dt_bias, alpha, beta, conv, S, out, 0, op->n_vh);
        return;
    }
    orc_delta_job jobs[256];
    pthread_t th[256];
    for (int t = 0; t < n_threads; ++t) {
        orc_delta_job j = {op, ssm_a, dt_bias, alpha, beta, conv, S, out,
                           (int64_t)op->n_vh * t / n_threads, (int64_t)op->n_vh * (t + 1) / n_threads};
        jobs[t] = j;
    }
    /* a thread that fails to start has its slice run here instead */
    int started[256];
    for (int t = 0; t < n_threads; ++t) {
        started[t] = pthread_create(&th[t], NULL, orc_delta_run, &jobs[t]) == 0;
        if (!started[t]) orc_delta_run(&jobs[t]);
    }
    for (int t = 0; t < n_threads; ++t)
        if (started[t]) pthread_join(th[t], NULL);
}

/* ops.rs:197-203: x / max(||x||, eps), per head of `dim` elements. */
void orc_l2_norm_rows(float *x, int64_t rows, int64_t dim, float eps) {
    for (int64_t r = 0; r < rows; ++r) {
        float *v = x + r * dim;
        float acc = 0.0f;
        for (int64_t d = 0; d < dim; ++d) acc += v[d] * v[d];
        float nrm = sqrtf(acc);
        float sc = 1.0f / (nrm > eps ? nrm : eps);
        for (int64_t d = 0; d < dim; ++d) v[d] *= sc;
    }
}

/* ops.rs:40-47: x / sqrt(mean(x^2) + eps), per head of `dim` elements. */
void orc_rms_norm_rows(float *x, int64_t rows, int64_t dim, float eps) {
    for (int64_t r = 0; r < rows; ++r) {
        float *v = x + r * dim;
        float acc = 0.0f;
        for (int64_t d = 0; d < dim; ++d) acc += v[d] * v[d];
        float mean_sq = acc / (float)dim;
        float sc = 1.0f / sqrtf(mean_sq + eps);
        for (int64_t d = 0; d < dim; ++d) v[d] *= sc;
    }
}

/* ------------------------------------------------------ rope / prologue -- */
/* ops.rs:142-159: NeoX pairs (i, i + d/2) of the d leading dims of a head.
 * The angle runs in double exactly as the reference: theta starts at pos and
 * is multiplied by base^(-2/d) once per pair; factor i (1 when absent)
 * divides the angle; sin and cos are rounded to float. */
void orc_rope_neox(float *head, int64_t d, int64_t pos, float base, const float *factors,
                   int64_t n_factors) {
    const int64_t half = d / 2;
    const double theta_scale = pow((double)base, -2.0 / (double)d);
    double theta = (double)pos;
    for (int64_t i = 0; i < half; ++i) {
        const double factor = (factors && i < n_factors) ? (double)factors[i] : 1.0;
        const double angle = theta / factor;
        const float sn = (float)sin(angle), cs = (float)cos(angle);
        const float x0 = head[i], x1 = head[i + half];
        head[i] = x0 * cs - x1 * sn;
        head[i + half] = x0 * sn + x1 * cs;
        theta *= theta_scale;
    }
}

typedef struct {
    uint32_t n_tokens, n_heads, n_kv_heads, head_dim;
    uint32_t q_stride;   /* floats from one query head to the next (>= head_dim) */
    uint32_t n_rot;      /* leading dims of each head that rotate (even)       */
    uint32_t base_pos, window;
    uint32_t v_norm;     /* 1: RMS-normalize V per head, no gain               */
    float rms_eps, rope_base;
} orc_prologue;

/* ops.rs:40-47 then the gain multiply of ops.rs:53-59 (gain may be NULL). */
static void orc_rms_norm_mul(float *x, int64_t n, const float *gain, float eps) {
    float acc = 0.0f;
    for (int64_t d = 0; d < n; ++d) acc += x[d] * x[d];
    const float mean_sq = acc / (float)n;
    const float sc = 1.0f / sqrtf(mean_sq + eps);
    for (int64_t d = 0; d < n; ++d) x[d] *= sc;
    if (gain)
        for (int64_t d = 0; d < n; ++d) x[d] *= gain[d];
}

/* cpu.rs:286-327 / qwen35/cpu.rs:294-304: per query head (stride q_stride,
 * first head_dim floats) RMS norm times q_gain then NeoX rope over n_rot dims
 * at pos = base_pos + token; per K head the same with k_gain; per V head an
 * RMS norm without gain when v_norm; then K and V rows go to the f16 caches
 * at slot(pos) (orc_write_cache).  A NULL gain skips that tensor's norm.
 * q is updated in place; k and v are scratch copies the caller owns. */
void orc_attn_prologue(const orc_prologue *p, float *q, float *k, float *v, const float *q_gain,
                       const float *k_gain, const float *rope_factors, uint16_t *k_cache,
                       uint16_t *v_cache) {
    const int64_t hd = p->head_dim, kv_dim = (int64_t)p->n_kv_heads * hd;
    for (int64_t i = 0; i < p->n_tokens; ++i) {
        const int64_t pos = (int64_t)p->base_pos + i;
        for (int64_t h = 0; h < p->n_heads; ++h) {
            float *head = q + (i * p->n_heads + h) * (int64_t)p->q_stride;
            if (q_gain) orc_rms_norm_mul(head, hd, q_gain, p->rms_eps);
            if (p->n_rot) orc_rope_neox(head, p->n_rot, pos, p->rope_base, rope_factors, p->n_rot / 2);
        }
        for (int64_t h = 0; h < p->n_kv_heads; ++h) {
            float *head = k + i * kv_dim + h * hd;
            if (k_gain) orc_rms_norm_mul(head, hd, k_gain, p->rms_eps);
            if (p->n_rot) orc_rope_neox(head, p->n_rot, pos, p->rope_base, rope_factors, p->n_rot / 2);
            if (p->v_norm) orc_rms_norm_mul(v + i * kv_dim + h * hd, hd, NULL, p->rms_eps);
        }
    }
    orc_write_cache(p->n_tokens, kv_dim, p->base_pos, p->window, k, k_cache);
    orc_write_cache(p->n_tokens, kv_dim, p->base_pos, p->window, v, v_cache);
}

/* ------------------------------------------------- delta front and back -- */
/* ops.rs:175-178 */
static float orc_silu(float x) { return x / (1.0f + expf(-x)); }

/* qwen35/cpu.rs:193-216, per token i in order: channel c of conv_out is
 * silu(x[i][c]*taps[c][K-1] + sum_{j<K-1} state[j][c]*taps[c][j]), the state
 * window (K-1 rows, oldest first) then drops its oldest row and appends x[i];
 * finally each of the 2*key_dim/s_dim q and k heads of conv_out is
 * L2-normalized (ops.rs:197-203; eps floors the norm). */
void orc_delta_front(int64_t n_tok, int64_t conv_dim, int64_t key_dim, int64_t s_dim,
                     int64_t kernel, float eps, const float *x, const float *taps,
                     float *state, float *conv_out) {
    for (int64_t i = 0; i < n_tok; ++i) {
        const float *row = x + i * conv_dim;
        float *out = conv_out + i * conv_dim;
        for (int64_t c = 0; c < conv_dim; ++c) {
            const float *tp = taps + c * kernel;
            float acc = row[c] * tp[kernel - 1];
            for (int64_t j = 0; j < kernel - 1; ++j) acc += state[j * conv_dim + c] * tp[j];
            out[c] = orc_silu(acc);
        }
        if (kernel > 1) {
            memmove(state, state + conv_dim, (size_t)((kernel - 2) * conv_dim) * sizeof(float));
            memcpy(state + (kernel - 2) * conv_dim, row, (size_t)conv_dim * sizeof(float));
        }
        orc_l2_norm_rows(out, 2 * key_dim / s_dim, s_dim, eps);
    }
}

/* out[r][d] *= sigmoid(gate[r*gate_stride + d]) for r < n_rows, d < dim, in
 * the reference's order: sigmoid(x) = 1 / (1 + exp(-x)) in f32, then the
 * product (qwen35/cpu.rs:359-363, ops.rs:181-183). */
void orc_attn_gate(int64_t n_rows, int64_t dim, int64_t gate_stride, float *out,
                   const float *gate) {
    for (int64_t r = 0; r < n_rows; ++r)
        for (int64_t d = 0; d < dim; ++d) {
            const float g = gate[r * gate_stride + d];
            const float s = 1.0f / (1.0f + expf(-g));
            out[r * dim + d] *= s;
        }
}

/* qwen35/cpu.rs:250-259: per token and v-head, rms_norm_mul(o, w) then
 * o *= silu(z), in place. */
void orc_delta_back(int64_t n_tok, int64_t n_vh, int64_t s_dim, float eps, float *o,
                    const float *z, const float *w) {
    for (int64_t r = 0; r < n_tok * n_vh; ++r) {
        float *oh = o + r * s_dim;
        const float *zh = z + r * s_dim;
        orc_rms_norm_mul(oh, s_dim, w, eps);
        for (int64_t j = 0; j < s_dim; ++j) oh[j] *= orc_silu(zh[j]);
    }
}

/* ------------------------------------------------------------ k-quants -- */
/* Type codes (ggml's GgmlType numbering): F32 0, F16 1, Q8_0 8, Q4_K 12,
 * Q6_K 14, BF16 30. */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q8_0 = 8, ORC_Q4K = 12, ORC_Q6K = 14, ORC_BF16 = 30 };

static float orc_le_f16(const uint8_t *b) { return orc_f16_to_f32((uint16_t)(b[0] | (b[1] << 8))); }

static float orc_le_bf16(const uint8_t *b) {
    uint32_t u = (uint32_t)(b[0] | (b[1] << 8)) << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* quant.rs:33-47 */
static void orc_q4k_scale_min(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* Bytes per block and elements per block of a type (0 for an unknown type). */
int64_t orc_block_bytes(int ty) {
    switch (ty) {
        case ORC_F32: return 4;
        case ORC_F16: case ORC_BF16: return 2;
        case ORC_Q8_0: return 34;
        case ORC_Q4K: return 144;
        case ORC_Q6K: return 210;
        default: return 0;
    }
}
int64_t orc_block_elems(int ty) {
    switch (ty) {
        case ORC_F32: case ORC_F16: case ORC_BF16: return 1;
        case ORC_Q8_0: return 32;
        case ORC_Q4K: case ORC_Q6K: return 256;
        default: return 0;
    }
}

/* quant.rs:54-128, 130-182: n elements (a multiple of the block size). */
void orc_dequant(int ty, const uint8_t *data, int64_t n, float *out) {
    if (ty == ORC_F32) { memcpy(out, data, (size_t)n * 4); return; }
    if (ty == ORC_F16) { for (int64_t i = 0; i < n; ++i) out[i] = orc_le_f16(data + 2 * i); return; }
    if (ty == ORC_BF16) { for (int64_t i = 0; i < n; ++i) out[i] = orc_le_bf16(data + 2 * i); return; }
    if (ty == ORC_Q8_0) {
        for (int64_t b = 0; b < n / 32; ++b) {
            const uint8_t *blk = data + b * 34;
            const float d = orc_le_f16(blk);
            for (int i = 0; i < 32; ++i) out[b * 32 + i] = d * (float)(int8_t)blk[2 + i];
        }
        return;
    }
    if (ty == ORC_Q4K) {
        for (int64_t b = 0; b < n / 256; ++b) {
            const uint8_t *blk = data + b * 144;
            const float d = orc_le_f16(blk), dmin = orc_le_f16(blk + 2);
            const uint8_t *sc = blk + 4, *qs = blk + 16;
            float *o = out + b * 256;
            for (int pair = 0; pair < 4; ++pair) {
                uint8_t sc1, m1, sc2, m2;
                orc_q4k_scale_min(pair * 2, sc, &sc1, &m1);
                orc_q4k_scale_min(pair * 2 + 1, sc, &sc2, &m2);
                const float d1 = d * (float)sc1, min1 = dmin * (float)m1;
                const float d2 = d * (float)sc2, min2 = dmin * (float)m2;
                const uint8_t *q = qs + pair * 32;
                for (int l = 0; l < 32; ++l) {
                    o[pair * 64 + l] = d1 * (float)(q[l] & 0xF) - min1;
                    o[pair * 64 + l + 32] = d2 * (float)(q[l] >> 4) - min2;
                }
            }
        }
        return;
    }
    if (ty == ORC_Q6K) {
        for (int64_t b = 0; b < n / 256; ++b) {
            const uint8_t *blk = data + b * 210;
            const float d = orc_le_f16(blk + 208);
            for (int h = 0; h < 2; ++h) {
                const uint8_t *ql = blk + h * 64, *qh = blk + 128 + h * 32;
                const int8_t *sc = (const int8_t *)(blk + 192 + h * 8);
                float *y = out + b * 256 + h * 128;
                for (int l = 0; l < 32; ++l) {
                    const int is = l / 16;
                    const uint8_t hb = qh[l];
                    const int q1 = ((ql[l] & 0xF) | ((hb & 3) << 4)) - 32;
                    const int q2 = ((ql[l + 32] & 0xF) | (((hb >> 2) & 3) << 4)) - 32;
                    const int q3 = ((ql[l] >> 4) | (((hb >> 4) & 3) << 4)) - 32;
                    const int q4 = ((ql[l + 32] >> 4) | (((hb >> 6) & 3) << 4)) - 32;
                    y[l] = d * (float)sc[is] * (float)q1;
                    y[l + 32] = d * (float)sc[is + 2] * (float)q2;
                    y[l + 64] = d * (float)sc[is + 4] * (float)q3;
                    y[l + 96] = d * (float)sc[is + 6] * (float)q4;
                }
            }
        }
    }
}

/* quant.rs:187-271: the fused decode-and-dot of one row with x[n]. */
float orc_dot_row(int ty, const uint8_t *row, const float *x, int64_t n) {
    float acc = 0.f;
    if (ty == ORC_Q4K) {
        for (int64_t b = 0; b < n / 256; ++b) {
            const uint8_t *blk = row + b * 144;
            const float d = orc_le_f16(blk), dmin = orc_le_f16(blk + 2);
            const uint8_t *sc = blk + 4, *qs = blk + 16;
            const float *xb = x + b * 256;
            for (int pair = 0; pair < 4; ++pair) {
                uint8_t sc1, m1, sc2, m2;
                orc_q4k_scale_min(pair * 2, sc, &sc1, &m1);
                orc_q4k_scale_min(pair * 2 + 1, sc, &sc2, &m2);
                const uint8_t *q = qs + pair * 32;
                const float *xl = xb + pair * 64;
                float s1 = 0.f, x1 = 0.f, s2 = 0.f, x2 = 0.f;
                for (int l = 0; l < 32; ++l) {
                    const float a = xl[l], c = xl[l + 32];
                    s1 += (float)(q[l] & 0xF) * a;
                    x1 += a;
                    s2 += (float)(q[l] >> 4) * c;
                    x2 += c;
                }
                acc += d * (float)sc1 * s1 - dmin * (float)m1 * x1;
                acc += d * (float)sc2 * s2 - dmin * (float)m2 * x2;
            }
        }
        return acc;
    }
    if (ty == ORC_Q6K) {
        for (int64_t b = 0; b < n / 256; ++b) {
            const uint8_t *blk = row + b * 210;
            const float d = orc_le_f16(blk + 208);
            const float *xb = x + b * 256;
            float sub = 0.f;
            for (int h = 0; h < 2; ++h) {
                const uint8_t *ql = blk + h * 64, *qh = blk + 128 + h * 32;
                const int8_t *sc = (const int8_t *)(blk + 192 + h * 8);
                const float *y = xb + h * 128;
                for (int l = 0; l < 32; ++l) {
                    const int is = l / 16;
                    const uint8_t hb = qh[l];
                    const int q1 = ((ql[l] & 0xF) | ((hb & 3) << 4)) - 32;
                    const int q2 = ((ql[l + 32] & 0xF) | (((hb >> 2) & 3) << 4)) - 32;
                    const int q3 = ((ql[l] >> 4) | (((hb >> 4) & 3) << 4)) - 32;
                    const int q4 = ((ql[l + 32] >> 4) | (((hb >> 6) & 3) << 4)) - 32;
                    sub += (float)sc[is] * (float)q1 * y[l] + (float)sc[is + 2] * (float)q2 * y[l + 32] +
                           (float)sc[is + 4] * (float)q3 * y[l + 64] + (float)sc[is + 6] * (float)q4 * y[l + 96];
                }
            }
            acc += d * sub;
        }
        return acc;
    }
    if (ty == ORC_Q8_0) {
        for (int64_t b = 0; b < n / 32; ++b) {
            const uint8_t *blk = row + b * 34;
            const float d = orc_le_f16(blk);
            float sub = 0.f;
            for (int i = 0; i < 32; ++i) sub += (float)(int8_t)blk[2 + i] * x[b * 32 + i];
            acc += d * sub;
        }
        return acc;
    }
    for (int64_t i = 0; i < n; ++i) {
        const float w = ty == ORC_F32 ? ((const float *)row)[i]
                      : ty == ORC_F16 ? orc_le_f16(row + 2 * i) : orc_le_bf16(row + 2 * i);
        acc += w * x[i];
    }
    return acc;
}

/* y[t][r] = dot_row(row r of w, x[t]) for t < n_tok, r < rows: what the
 * reference's matvec kernels compute and are checked against. */
int orc_matvec(int ty, const uint8_t *w, int64_t rows, int64_t in_dim, const float *x,
               int64_t n_tok, float *y) {
    const int64_t bb = orc_block_bytes(ty), be = orc_block_elems(ty);
    if (!bb || in_dim % be) return 1;
    const int64_t row_bytes = in_dim / be * bb;
    for (int64_t t = 0; t < n_tok; ++t)
        for (int64_t r = 0; r < rows; ++r)
            y[t * rows + r] = orc_dot_row(ty, w + r * row_bytes, x + t * in_dim, in_dim);
    return 0;
}

