// Multi-sequence KV manager: host bookkeeping for many sequences' f16 caches
// inside one caller-allocated device arena.
//
// The reference keeps one KvCache per session: per owning layer a
// [slots, kv_dim] cache, slots = min(window, n_ctx) for a windowed layer
// (config.rs:279-284), sharing layers pointing at their source's cache
// (cache.rs:86-104), a write position `len` (cache.rs:71-76), and in the
// session the ids that are resident plus whether they still describe the
// cache (session.rs:317, 497-513, 546-570, 607-609).  Here that state is kept
// per sequence slot, and each slot's caches are one contiguous slab of the
// arena, so wiping a sequence is one fill and the slab of sequence s starts at
// s * slab_bytes.
#include <algorithm>
#include <new>
#include <vector>

#include "common.hpp"

namespace {

constexpr size_t kBlockAlign = 256;

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

struct LayerMap {
    uint32_t owner;    // index of the cache-owning layer whose cache this layer reads
    uint32_t slots;
    uint32_t window;   // 0: linear; else the ring size min(window, n_ctx)
    uint32_t kv_dim;
    size_t k_off;      // byte offsets of the owner's blocks within a slab
    size_t v_off;
};

struct Seq {
    bool open = false;
    bool comparable = true;  // the resident ids describe the whole cache
    bool stale = false;      // a ring slot holds a position past len (after a truncate)
    uint32_t len = 0;
    uint32_t hw = 0;         // positions [0, hw) were written since the last wipe
    std::vector<int32_t> cached;
};

// After positions [0, hw) were stored in order into a ring of w slots, does
// continuing at position pos read a slot that a later position overwrote?
// The query at pos sees [max(0, pos - w + 1), pos]; slot x % w of a visible
// x < pos holds x only if no y in (x, hw) with y = x (mod w) was stored, and
// the first such y is x + w.  Some visible x has x + w < hw exactly when
// max(pos + 1, w) <= min(hw - 1, pos + w - 1).
bool ring_stale(uint32_t w, uint32_t hw, uint32_t pos) {
    if (w < 2 || hw == 0) return false;
    const uint64_t lo = std::max<uint64_t>((uint64_t)pos + 1, w);
    const uint64_t hi = std::min<uint64_t>((uint64_t)hw - 1, (uint64_t)pos + w - 1);
    return lo <= hi;
}

// Validates d and lays out one sequence slab; false for an invalid description.
bool plan(const lmx_kvm_desc* d, std::vector<LayerMap>& map, size_t& slab) {
    if (!d || !d->layers || d->n_layers == 0 || d->n_ctx == 0 || d->max_seqs == 0) return false;
    map.assign(d->n_layers, LayerMap{});
    slab = 0;
    for (uint32_t i = 0; i < d->n_layers; ++i) {
        const lmx_kvm_layer& L = d->layers[i];
        if (L.kv_source >= 0) {
            // cache.rs:97-103: a sharing layer reads an earlier layer's cache
            if ((uint32_t)L.kv_source >= i) return false;
            map[i] = map[(uint32_t)L.kv_source];
            continue;
        }
        if (L.kv_source != -1 || L.kv_dim == 0 || L.kv_dim % 8) return false;
        LayerMap m{};
        m.owner = i;
        m.kv_dim = L.kv_dim;
        m.slots = L.window ? std::min(L.window, d->n_ctx) : d->n_ctx;  // config.rs:279-284
        m.window = L.window ? m.slots : 0;
        const size_t block = round_up((size_t)m.slots * m.kv_dim * sizeof(uint16_t), kBlockAlign);
        m.k_off = slab;
        m.v_off = slab + block;
        slab += 2 * block;
        map[i] = m;
    }
    return true;
}

}  // namespace

struct lmx_kvm {
    std::vector<LayerMap> map;
    std::vector<Seq> seqs;
    size_t slab = 0;
    char* arena = nullptr;
    uint32_t n_ctx = 0;
    std::vector<uint32_t> rings;  // ring sizes of the cache-owning windowed layers

    Seq* seq(int32_t s) {
        if (s < 0 || (size_t)s >= seqs.size() || !seqs[s].open) return nullptr;
        return &seqs[s];
    }
    const Seq* seq(int32_t s) const { return const_cast<lmx_kvm*>(this)->seq(s); }
    char* slab_of(int32_t s) const { return arena + (size_t)s * slab; }

    // session.rs:497-513
    uint32_t reusable(const Seq& q, const int32_t* tokens, uint32_t n) const {
        if (!q.comparable) return 0;
        const size_t lim = std::min(q.cached.size(), (size_t)n);
        size_t k = 0;
        while (k < lim && q.cached[k] == tokens[k]) ++k;
        return (k == q.cached.size() && k < n) ? (uint32_t)k : 0;
    }

    lmx_status wipe(int32_t s, lmx_stream st) {
        Seq& q = seqs[s];
        q.len = 0;
        q.hw = 0;
        q.cached.clear();
        q.comparable = true;
        q.stale = false;
        return lmx_workspace_init(slab_of(s), slab, st);
    }
};

extern "C" {

size_t lmx_kvm_arena_bytes(const lmx_kvm_desc* d) {
    std::vector<LayerMap> map;
    size_t slab = 0;
    try {
        if (!plan(d, map, slab)) return 0;
    } catch (...) {
        return 0;
    }
    return slab * d->max_seqs;
}

lmx_status lmx_kvm_create(const lmx_kvm_desc* d, void* arena, size_t arena_bytes, lmx_kvm** out) {
    if (!d || !out || !arena) return LMX_E_NULL;
    *out = nullptr;
    if (((uintptr_t)arena % kBlockAlign) != 0) return LMX_E_ALIGN;
    try {
        lmx_kvm* m = new lmx_kvm();
        if (!plan(d, m->map, m->slab)) {
            delete m;
            return LMX_E_SHAPE;
        }
        if (arena_bytes < m->slab * d->max_seqs) {
            delete m;
            return LMX_E_WORKSPACE;
        }
        m->seqs.resize(d->max_seqs);
        for (uint32_t i = 0; i < d->n_layers; ++i)
            if (m->map[i].owner == i && m->map[i].window) m->rings.push_back(m->map[i].window);
        m->arena = static_cast<char*>(arena);
        m->n_ctx = d->n_ctx;
        *out = m;
        return LMX_OK;
    } catch (const std::bad_alloc&) {
        return LMX_E_HOST;
    }
}

void lmx_kvm_destroy(lmx_kvm* m) { delete m; }

lmx_status lmx_kvm_open(lmx_kvm* m, int32_t* seq) {
    if (!m || !seq) return LMX_E_NULL;
    for (size_t s = 0; s < m->seqs.size(); ++s) {
        Seq& q = m->seqs[s];
        if (!q.open) {
            q = Seq{};
            q.open = true;
            *seq = (int32_t)s;
            return LMX_OK;
        }
    }
    return LMX_E_FULL;
}

lmx_status lmx_kvm_close(lmx_kvm* m, int32_t seq) {
    if (!m) return LMX_E_NULL;
    Seq* q = m->seq(seq);
    if (!q) return LMX_E_SHAPE;
    *q = Seq{};
    return LMX_OK;
}

lmx_status lmx_kvm_len(const lmx_kvm* m, int32_t seq, uint32_t* len) {
    if (!m || !len) return LMX_E_NULL;
    const Seq* q = m->seq(seq);
    if (!q) return LMX_E_SHAPE;
    *len = q->len;
    return LMX_OK;
}

lmx_status lmx_kvm_reusable_prefix(const lmx_kvm* m, int32_t seq, const int32_t* tokens, uint32_t n,
                                   uint32_t* reuse) {
    if (!m || !reuse || (!tokens && n)) return LMX_E_NULL;
    const Seq* q = m->seq(seq);
    if (!q) return LMX_E_SHAPE;
    *reuse = m->reusable(*q, tokens, n);
    return LMX_OK;
}

lmx_status lmx_kvm_begin(lmx_kvm* m, int32_t seq, const int32_t* tokens, uint32_t n, uint32_t* reuse,
                         lmx_stream stream) {
    if (!m || !reuse || (!tokens && n)) return LMX_E_NULL;
    Seq* q = m->seq(seq);
    if (!q) return LMX_E_SHAPE;
    if (n > m->n_ctx) return LMX_E_CONTEXT;  // session.rs:539-544
    *reuse = m->reusable(*q, tokens, n);
    if (*reuse == 0) return m->wipe(seq, stream);
    // A strict prefix of what is resident: len already equals *reuse.
    return LMX_OK;
}

lmx_status lmx_kvm_commit(lmx_kvm* m, int32_t seq, const int32_t* tokens, uint32_t n) {
    if (!m) return LMX_E_NULL;
    Seq* q = m->seq(seq);
    if (!q) return LMX_E_SHAPE;
    if (q->stale) return LMX_E_RING_HAZARD;
    if ((uint64_t)q->len + n > m->n_ctx) return LMX_E_CONTEXT;
    try {
        if (!tokens) {
            q->comparable = false;  // session.rs:569-571
            q->cached.clear();
        } else if (q->comparable) {
            q->cached.insert(q->cached.end(), tokens, tokens + n);
        }
    } catch (const std::bad_alloc&) {
        return LMX_E_HOST;
    }
    q->len += n;
    q->hw = std::max(q->hw, q->len);
    return LMX_OK;
}

lmx_status lmx_kvm_truncate(lmx_kvm* m, int32_t seq, uint32_t pos) {
    if (!m) return LMX_E_NULL;
    Seq* q = m->seq(seq);
    if (!q) return LMX_E_SHAPE;
    q->len = std::min(q->len, pos);  // cache.rs:146-149
    if (q->cached.size() > q->len) q->cached.resize(q->len);
    // Ring layers have already overwritten slots of positions before the new
    // end with positions past it: the sequence can only restart from a wipe.
    for (uint32_t w : m->rings)
        if (ring_stale(w, q->hw, q->len)) q->stale = true;
    if (q->stale) {
        q->comparable = false;
        q->cached.clear();
    }
    return LMX_OK;
}

lmx_status lmx_kvm_wipe(lmx_kvm* m, int32_t seq, lmx_stream stream) {
    if (!m) return LMX_E_NULL;
    if (!m->seq(seq)) return LMX_E_SHAPE;
    return m->wipe(seq, stream);
}

lmx_status lmx_kvm_layer_cache(const lmx_kvm* m, int32_t seq, uint32_t layer, void** k, void** v,
                               uint32_t* n_slots, uint32_t* window) {
    if (!m || !k || !v || !n_slots || !window) return LMX_E_NULL;
    if (!m->seq(seq) || layer >= m->map.size()) return LMX_E_SHAPE;
    const LayerMap& L = m->map[layer];
    *k = m->slab_of(seq) + L.k_off;
    *v = m->slab_of(seq) + L.v_off;
    *n_slots = L.slots;
    *window = L.window;
    return LMX_OK;
}

lmx_status lmx_kvm_batch(const lmx_kvm* m, uint32_t layer, const int32_t* seqs, uint32_t n,
                         uint32_t extra, const void** k_ptrs, const void** v_ptrs, int32_t* ctx_lens,
                         int32_t* max_ctx) {
    if (!m || !seqs || !k_ptrs || !v_ptrs || !ctx_lens || !max_ctx) return LMX_E_NULL;
    if (n == 0 || layer >= m->map.size()) return LMX_E_SHAPE;
    const LayerMap& L = m->map[layer];
    int32_t mx = 0;
    for (uint32_t b = 0; b < n; ++b) {
        const Seq* q = m->seq(seqs[b]);
        if (!q) return LMX_E_SHAPE;
        if (q->stale) return LMX_E_RING_HAZARD;
        const uint64_t ctx = (uint64_t)q->len + extra;
        if (ctx == 0) return LMX_E_SHAPE;
        if (ctx > m->n_ctx) return LMX_E_CONTEXT;
        k_ptrs[b] = m->slab_of(seqs[b]) + L.k_off;
        v_ptrs[b] = m->slab_of(seqs[b]) + L.v_off;
        ctx_lens[b] = (int32_t)ctx;
        mx = std::max(mx, (int32_t)ctx);
    }
    *max_ctx = mx;
    return LMX_OK;
}

}  // extern "C"
