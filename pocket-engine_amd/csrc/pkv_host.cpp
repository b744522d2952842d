// Host half of the paged KV cache: the block allocator.
//
// Restates the reference scheduler's KV block bookkeeping
// (src/sched.rs:461-465 fields, :515 initial free list, :801-807
// take_blocks, :809-817 unref_blocks): a LIFO free list kept as a vector,
// initialised to [n-1, ..., 1, 0]; taking n blocks splits off the last n
// entries in vector order (a fresh pool's first request of 2 gets [1, 0]) and
// sets each reference count to 1; releasing a reference pushes a block whose
// count reaches 0 back on the end. Reference counts are 16-bit like the
// reference's Vec<u16>.
#include "../../include/pkv.h"

#include <algorithm>
#include <cstdint>
#include <map>
#include <new>
#include <unordered_map>
#include <vector>

struct pkv_pool {
    std::vector<uint32_t> free_blocks;
    std::vector<uint16_t> refs;
};

extern "C" {

pkv_pool* pkv_pool_create(int64_t n_blocks) {
    if (n_blocks <= 0 || n_blocks > (int64_t)UINT32_MAX) return nullptr;
    pkv_pool* p = new (std::nothrow) pkv_pool;
    if (!p) return nullptr;
    p->free_blocks.resize((size_t)n_blocks);
    for (int64_t i = 0; i < n_blocks; i++) p->free_blocks[(size_t)i] = (uint32_t)(n_blocks - 1 - i);
    p->refs.assign((size_t)n_blocks, 0);
    return p;
}

void pkv_pool_destroy(pkv_pool* pool) { delete pool; }

int pkv_pool_take(pkv_pool* pool, int n, uint32_t* ids) {
    if (!pool || n < 0 || (n > 0 && !ids)) return PKV_ERR_INVALID;
    if ((size_t)n > pool->free_blocks.size()) return PKV_ERR_NO_BLOCKS;
    const size_t at = pool->free_blocks.size() - (size_t)n;
    for (int i = 0; i < n; i++) {
        const uint32_t b = pool->free_blocks[at + (size_t)i];
        ids[i] = b;
        pool->refs[b] = 1;
    }
    pool->free_blocks.resize(at);
    return PKV_OK;
}

int pkv_pool_unref(pkv_pool* pool, const uint32_t* ids, int n) {
    if (!pool || n < 0 || (n > 0 && !ids)) return PKV_ERR_INVALID;
    // Validate first so a bad call changes nothing (the reference's u16
    // subtraction would panic on underflow).
    std::unordered_map<uint32_t, uint32_t> uses;
    for (int i = 0; i < n; i++) {
        if (ids[i] >= pool->refs.size()) return PKV_ERR_INVALID;
        if (++uses[ids[i]] > pool->refs[ids[i]]) return PKV_ERR_INVALID;
    }
    for (int i = 0; i < n; i++) {
        uint16_t& r = pool->refs[ids[i]];
        r--;
        if (r == 0) pool->free_blocks.push_back(ids[i]);
    }
    return PKV_OK;
}

int pkv_pool_ref(pkv_pool* pool, const uint32_t* ids, int n) {
    if (!pool || n < 0 || (n > 0 && !ids)) return PKV_ERR_INVALID;
    std::unordered_map<uint32_t, uint32_t> uses;
    for (int i = 0; i < n; i++) {
        if (ids[i] >= pool->refs.size() || pool->refs[ids[i]] == 0) return PKV_ERR_INVALID;
        if ((uint32_t)pool->refs[ids[i]] + ++uses[ids[i]] > 0xffffu) return PKV_ERR_INVALID;
    }
    for (int i = 0; i < n; i++) pool->refs[ids[i]]++;
    return PKV_OK;
}

int64_t pkv_pool_free_count(const pkv_pool* pool) { return pool ? (int64_t)pool->free_blocks.size() : -1; }

int64_t pkv_pool_total(const pkv_pool* pool) { return pool ? (int64_t)pool->refs.size() : -1; }

int pkv_pool_refs(const pkv_pool* pool, uint32_t id) {
    if (!pool || id >= pool->refs.size()) return -PKV_ERR_INVALID;
    return pool->refs[id];
}

int64_t pkv_pool_free_list(const pkv_pool* pool, uint32_t* out, int64_t cap) {
    if (!pool || cap < 0 || (cap > 0 && !out)) return -PKV_ERR_INVALID;
    const int64_t n = (int64_t)pool->free_blocks.size();
    for (int64_t i = 0; i < n && i < cap; i++) out[i] = pool->free_blocks[(size_t)i];
    return n;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// KV manager: per-sequence block tables over a pool, the prefix cache, the
// step metadata, copy-on-write and truncation. Restates the KV bookkeeping of
// the reference Scheduler (src/sched.rs): admission reserves blocks for
// prompt + max_new (:669-799, total blocks :681), reusing the longest cached
// whole-unit prefix (:687-765, lookup :832-842) and evicting least recently
// used entries while blocks are short (:697-714, evict_one :820-828); cache
// entries cover whole 64-token units (CACHE_UNIT :322) and hold a reference
// on each of their blocks (add_entry :1044-1067); fill writes pos, slot_map,
// tok_seq, cu, limits and block_table rows (:1071-1191); pad writes padding
// rows (:1219-1261); release drops a sequence's references (:844-854).
// Copy-on-write and truncation with page freeing are this build's own
// (the reference never writes into a shared page and keeps reserved pages
// on rollback, :1297-1327).

namespace {

constexpr int CACHE_UNIT = 64;

struct KvSeq {
    std::vector<uint32_t> blocks;
    int64_t len = 0;  // tokens whose K/V are written ("fed")
};

struct KvEntry {
    uint32_t adapter;
    std::vector<uint32_t> tokens;
    std::vector<uint32_t> blocks;
    uint64_t used;
};

// Chained hashes of whole units: element k covers tokens [0, (k + 1) * 64)
// (the reference chains Rust's DefaultHasher the same way, sched.rs:346-358;
// only equality of chains matters, and lookups compare tokens as well).
std::vector<uint64_t> unit_hashes(uint32_t adapter, const uint32_t* tokens, int64_t n) {
    std::vector<uint64_t> out;
    uint64_t h = 1469598103934665603ull ^ adapter;
    for (int64_t u = 0; u + CACHE_UNIT <= n; u += CACHE_UNIT) {
        for (int i = 0; i < CACHE_UNIT; i++) {
            uint32_t t = tokens[u + i];
            for (int b = 0; b < 4; b++) {
                h ^= (t >> (8 * b)) & 0xffu;
                h *= 1099511628211ull;
            }
        }
        h ^= h >> 29;
        h *= 0xbf58476d1ce4e5b9ull;
        h ^= h >> 32;
        out.push_back(h);
    }
    return out;
}

}  // namespace

struct pkv_kv {
    pkv_pool pool;
    int bs;
    int64_t max_entries;  // 0: unlimited (the reference bounds entries by snapshot slots)
    std::map<int, KvSeq> seqs;
    int next_id = 0;
    std::unordered_map<uint64_t, KvEntry> entries;
    uint64_t clock = 0;

    int take(int n, std::vector<uint32_t>& out) {
        const size_t at = out.size();
        out.resize(at + (size_t)n);
        return pkv_pool_take(&pool, n, out.data() + at);
    }
    void unref(const std::vector<uint32_t>& b) {
        if (!b.empty()) pkv_pool_unref(&pool, b.data(), (int)b.size());
    }
    void ref(const std::vector<uint32_t>& b) {
        if (!b.empty()) pkv_pool_ref(&pool, b.data(), (int)b.size());
    }
    bool evict_one(const uint64_t* keep) {
        auto best = entries.end();
        for (auto it = entries.begin(); it != entries.end(); ++it) {
            if (keep && it->first == *keep) continue;
            if (best == entries.end() || it->second.used < best->second.used) best = it;
        }
        if (best == entries.end()) return false;
        unref(best->second.blocks);
        entries.erase(best);
        return true;
    }
    // Longest cached whole-unit prefix leaving at least one token to compute.
    bool lookup(uint32_t adapter, const uint32_t* prompt, int64_t n, uint64_t* h, int64_t* len) {
        if (n < 1) return false;
        const auto hs = unit_hashes(adapter, prompt, n - 1);
        for (int64_t k = (int64_t)hs.size() - 1; k >= 0; k--) {
            const auto it = entries.find(hs[(size_t)k]);
            const int64_t l = (k + 1) * CACHE_UNIT;
            if (it != entries.end() && it->second.adapter == adapter &&
                std::equal(prompt, prompt + l, it->second.tokens.begin())) {
                *h = hs[(size_t)k];
                *len = l;
                return true;
            }
        }
        return false;
    }
    KvSeq* seq(int id) {
        const auto it = seqs.find(id);
        return it == seqs.end() ? nullptr : &it->second;
    }
};

extern "C" {

pkv_kv* pkv_kv_create(int64_t n_blocks, int block_size, int64_t max_entries) {
    if (n_blocks <= 0 || n_blocks > (int64_t)UINT32_MAX || block_size <= 0 || max_entries < 0) return nullptr;
    pkv_kv* kv = new (std::nothrow) pkv_kv;
    if (!kv) return nullptr;
    kv->pool.free_blocks.resize((size_t)n_blocks);
    for (int64_t i = 0; i < n_blocks; i++) kv->pool.free_blocks[(size_t)i] = (uint32_t)(n_blocks - 1 - i);
    kv->pool.refs.assign((size_t)n_blocks, 0);
    kv->bs = block_size;
    kv->max_entries = max_entries;
    return kv;
}

void pkv_kv_destroy(pkv_kv* kv) { delete kv; }

pkv_pool* pkv_kv_pool(pkv_kv* kv) { return kv ? &kv->pool : nullptr; }

int pkv_kv_admit(pkv_kv* kv, uint32_t adapter, const uint32_t* prompt, int64_t prompt_len, int64_t max_new,
                 int use_cache, int* seq_id, int64_t* cached) {
    if (!kv || !prompt || prompt_len < 1 || max_new < 0 || !seq_id) return PKV_ERR_INVALID;
    const int64_t total = (prompt_len + max_new + kv->bs - 1) / kv->bs;
    uint64_t h = 0;
    int64_t hit_len = 0;
    const bool hit = use_cache && kv->lookup(adapter, prompt, prompt_len, &h, &hit_len);
    const int64_t reused = hit_len / kv->bs;
    const int64_t need = total - reused;
    // Cache entries give way to new requests, oldest first, but not the one
    // this request is about to use (sched.rs:697-714).
    while ((int64_t)kv->pool.free_blocks.size() < need && (int64_t)kv->entries.size() > (hit ? 1 : 0))
        if (!kv->evict_one(hit ? &h : nullptr)) break;
    if ((int64_t)kv->pool.free_blocks.size() < need) return PKV_ERR_NO_BLOCKS;
    KvSeq s;
    if (hit) {
        KvEntry& e = kv->entries[h];
        e.used = ++kv->clock;
        kv->ref(e.blocks);
        s.blocks = e.blocks;
        s.len = hit_len;
    }
    const int st = kv->take((int)need, s.blocks);
    if (st != PKV_OK) return st;
    *seq_id = kv->next_id++;
    kv->seqs[*seq_id] = std::move(s);
    if (cached) *cached = hit_len;
    return PKV_OK;
}

int pkv_kv_lookup(pkv_kv* kv, uint32_t adapter, const uint32_t* prompt, int64_t prompt_len, int64_t* hit_len) {
    if (!kv || !prompt || !hit_len) return PKV_ERR_INVALID;
    uint64_t h;
    *hit_len = 0;
    kv->lookup(adapter, prompt, prompt_len, &h, hit_len);
    return PKV_OK;
}

int pkv_kv_cache_add(pkv_kv* kv, int seq_id, uint32_t adapter, const uint32_t* tokens, int64_t len) {
    KvSeq* s = kv ? kv->seq(seq_id) : nullptr;
    if (!s || !tokens || len < 0) return PKV_ERR_INVALID;
    const auto hs = unit_hashes(adapter, tokens, len);
    if (hs.empty() || (int64_t)hs.size() * CACHE_UNIT != len) return PKV_ERR_INVALID;  // whole units only
    if ((int64_t)(len / kv->bs) > (int64_t)s->blocks.size()) return PKV_ERR_INVALID;
    const uint64_t h = hs.back();
    if (kv->entries.count(h)) return PKV_OK;  // already cached (sched.rs:1032-1034)
    // A bounded cache makes room first (reserve_snap, sched.rs:1029-1041).
    if (kv->max_entries > 0 && (int64_t)kv->entries.size() >= kv->max_entries && !kv->evict_one(nullptr))
        return PKV_ERR_NO_BLOCKS;
    KvEntry e;
    e.adapter = adapter;
    e.tokens.assign(tokens, tokens + len);
    e.blocks.assign(s->blocks.begin(), s->blocks.begin() + (ptrdiff_t)(len / kv->bs));
    kv->ref(e.blocks);
    e.used = ++kv->clock;
    kv->entries[h] = std::move(e);
    return PKV_OK;
}

int pkv_kv_evict_one(pkv_kv* kv) { return kv && kv->evict_one(nullptr) ? 1 : 0; }

int64_t pkv_kv_cache_entries(const pkv_kv* kv) { return kv ? (int64_t)kv->entries.size() : -1; }

int pkv_kv_release(pkv_kv* kv, int seq_id) {
    KvSeq* s = kv ? kv->seq(seq_id) : nullptr;
    if (!s) return PKV_ERR_INVALID;
    kv->unref(s->blocks);
    kv->seqs.erase(seq_id);
    return PKV_OK;
}

int pkv_kv_new_seq(pkv_kv* kv, int* seq_id) {
    if (!kv || !seq_id) return PKV_ERR_INVALID;
    *seq_id = kv->next_id++;
    kv->seqs[*seq_id] = KvSeq{};
    return PKV_OK;
}

int pkv_kv_reserve(pkv_kv* kv, int seq_id, int64_t n_tokens) {
    KvSeq* s = kv ? kv->seq(seq_id) : nullptr;
    if (!s || n_tokens < 0) return PKV_ERR_INVALID;
    const int64_t need = (n_tokens + kv->bs - 1) / kv->bs - (int64_t)s->blocks.size();
    if (need <= 0) return PKV_OK;
    if ((int64_t)kv->pool.free_blocks.size() < need) return PKV_ERR_NO_BLOCKS;
    return kv->take((int)need, s->blocks);
}

int pkv_kv_share(pkv_kv* kv, int dst_id, int src_id, int64_t n_tokens) {
    KvSeq* d = kv ? kv->seq(dst_id) : nullptr;
    KvSeq* src = kv ? kv->seq(src_id) : nullptr;
    if (!d || !src || dst_id == src_id || n_tokens < 0 || !d->blocks.empty() || n_tokens > src->len)
        return PKV_ERR_INVALID;
    const size_t n = (size_t)((n_tokens + kv->bs - 1) / kv->bs);
    d->blocks.assign(src->blocks.begin(), src->blocks.begin() + (ptrdiff_t)n);
    kv->ref(d->blocks);
    d->len = n_tokens;
    return PKV_OK;
}

int pkv_kv_prepare_write(pkv_kv* kv, int seq_id, int64_t pos, int n, int32_t* cow_src, int32_t* cow_dst, int cap,
                         int* n_copies) {
    KvSeq* s = kv ? kv->seq(seq_id) : nullptr;
    if (!s || pos < 0 || n < 0 || !n_copies || (cap > 0 && (!cow_src || !cow_dst))) return PKV_ERR_INVALID;
    *n_copies = 0;
    if (n == 0) return PKV_OK;
    const int64_t first = pos / kv->bs, last = (pos + n - 1) / kv->bs;
    // Pages that need copies and new pages, counted before anything changes.
    int64_t grow = last + 1 - (int64_t)s->blocks.size(), shared = 0;
    for (int64_t i = first; i <= last && i < (int64_t)s->blocks.size(); i++) shared += kv->pool.refs[s->blocks[(size_t)i]] > 1;
    if (grow < 0) grow = 0;
    if (shared > cap) return PKV_ERR_INVALID;
    if ((int64_t)kv->pool.free_blocks.size() < grow + shared) return PKV_ERR_NO_BLOCKS;
    for (int64_t i = first; i <= last && i < (int64_t)s->blocks.size(); i++) {
        uint32_t& b = s->blocks[(size_t)i];
        if (kv->pool.refs[b] <= 1) continue;
        uint32_t fresh;
        pkv_pool_take(&kv->pool, 1, &fresh);
        cow_src[*n_copies] = (int32_t)b;
        cow_dst[*n_copies] = (int32_t)fresh;
        ++*n_copies;
        pkv_pool_unref(&kv->pool, &b, 1);
        b = fresh;
    }
    if (grow > 0) kv->take((int)grow, s->blocks);
    return PKV_OK;
}

int pkv_kv_set_len(pkv_kv* kv, int seq_id, int64_t len) {
    KvSeq* s = kv ? kv->seq(seq_id) : nullptr;
    if (!s || len < 0 || len > (int64_t)s->blocks.size() * kv->bs) return PKV_ERR_INVALID;
    s->len = len;
    return PKV_OK;
}

int pkv_kv_truncate(pkv_kv* kv, int seq_id, int64_t new_len, int free_pages) {
    KvSeq* s = kv ? kv->seq(seq_id) : nullptr;
    if (!s || new_len < 0 || new_len > s->len) return PKV_ERR_INVALID;
    s->len = new_len;
    if (free_pages) {
        const size_t keep = (size_t)((new_len + kv->bs - 1) / kv->bs);
        if (keep < s->blocks.size()) {
            std::vector<uint32_t> gone(s->blocks.begin() + (ptrdiff_t)keep, s->blocks.end());
            kv->unref(gone);
            s->blocks.resize(keep);
        }
    }
    return PKV_OK;
}

int64_t pkv_kv_len(pkv_kv* kv, int seq_id) {
    KvSeq* s = kv ? kv->seq(seq_id) : nullptr;
    return s ? s->len : -PKV_ERR_INVALID;
}

int64_t pkv_kv_blocks(pkv_kv* kv, int seq_id, uint32_t* out, int64_t cap) {
    KvSeq* s = kv ? kv->seq(seq_id) : nullptr;
    if (!s || cap < 0 || (cap > 0 && !out)) return -PKV_ERR_INVALID;
    for (int64_t i = 0; i < (int64_t)s->blocks.size() && i < cap; i++) out[i] = s->blocks[(size_t)i];
    return (int64_t)s->blocks.size();
}

int pkv_kv_fill(pkv_kv* kv, const int* seq_ids, const int* ntok, int nrows, int max_tokens, int max_blocks,
                int32_t* pos, int32_t* slot_map, int32_t* tok_seq, int32_t* cu, int32_t* limits, int32_t* block_table) {
    if (!kv || nrows < 0 || (nrows > 0 && (!seq_ids || !ntok)) || max_tokens < 0 || max_blocks <= 0 || !pos ||
        !slot_map || !tok_seq || !cu || !limits || !block_table)
        return PKV_ERR_INVALID;
    int64_t t = 0;
    for (int si = 0; si < nrows; si++) {
        KvSeq* s = kv->seq(seq_ids[si]);
        if (!s || ntok[si] < 0 || (int64_t)s->blocks.size() > max_blocks) return PKV_ERR_INVALID;
        if (s->len + ntok[si] > (int64_t)s->blocks.size() * kv->bs || t + ntok[si] > max_tokens)
            return PKV_ERR_INVALID;
        t += ntok[si];
    }
    t = 0;
    cu[0] = 0;
    for (int si = 0; si < nrows; si++) {
        const KvSeq& s = *kv->seq(seq_ids[si]);
        for (int k = 0; k < ntok[si]; k++) {
            const int64_t p = s.len + k;
            pos[t] = (int32_t)p;
            slot_map[t] = (int32_t)((int64_t)s.blocks[(size_t)(p / kv->bs)] * kv->bs + p % kv->bs);
            tok_seq[t] = si;
            t++;
        }
        cu[si + 1] = (int32_t)t;
        limits[si] = (int32_t)((int64_t)s.blocks.size() * kv->bs - 1);
        int32_t* row = block_table + (size_t)si * max_blocks;
        for (int b = 0; b < max_blocks; b++) row[b] = b < (int)s.blocks.size() ? (int32_t)s.blocks[(size_t)b] : 0;
    }
    return PKV_OK;
}

int pkv_meta_layout(int64_t max_tokens, int64_t max_seqs, int64_t max_blocks, int64_t spec, pkv_meta* out) {
    if (max_tokens <= 0 || max_seqs <= 0 || max_blocks <= 0 || spec <= 0 || !out) return PKV_ERR_INVALID;
    const int64_t T = max_tokens, S = max_seqs, outs = max_seqs * spec;
    const int64_t lora_tiles = max_tokens / 16 + max_seqs;  // adapter tiles of 16 tokens (lora.rs:18)
    pkv_meta m;
    // per token: ids, pos, slot_map, tok_seq, emb_src, rope (3 rows), mtp_ids, mtp_src
    m.ids = 0;
    m.pos = T;
    m.slot_map = 2 * T;
    m.tok_seq = 3 * T;
    m.emb_src = 4 * T;
    m.rope = 5 * T;
    m.mtp_ids = 8 * T;
    m.mtp_src = 9 * T;
    // per sequence: cu (S + 1), slots, fresh; per output row: outs
    m.cu = 10 * T;
    m.slots = m.cu + S + 1;
    m.fresh = m.slots + S;
    m.outs = m.fresh + S;
    m.ocu = m.outs + outs;  // S + 1
    m.last = m.ocu + S + 1;
    m.temps = m.last + outs;
    m.seeds = m.temps + outs;
    m.top_ks = m.seeds + outs;
    m.top_ps = m.top_ks + outs;
    m.min_ps = m.top_ps + outs;
    m.pen_cu = m.min_ps + outs;  // outs + 1
    m.limits = m.pen_cu + outs + 1;
    m.snaps = m.limits + S;  // 4 per sequence
    m.block_table = m.snaps + 4 * S;
    m.lora = m.block_table + S * max_blocks;  // 1 + 3 per tile
    m.masks = m.lora + 1 + 3 * lora_tiles;
    m.words = m.masks + outs;
    *out = m;
    return PKV_OK;
}

int pkv_kv_pad(int from, int to, int n, int max_rows, int max_tokens, int max_blocks, int32_t* pos,
               int32_t* slot_map, int32_t* tok_seq, int32_t* cu, int32_t* limits, int32_t* block_table) {
    if (from < 0 || to < from || n < 1 || max_blocks <= 0 || to > max_rows || (int64_t)to * n > max_tokens || !pos ||
        !slot_map || !tok_seq || !cu || !limits || !block_table)
        return PKV_ERR_INVALID;
    if (from == 0) cu[0] = 0;
    for (int i = from; i < to; i++) {
        for (int k = 0; k < n; k++) {
            const int t = i * n + k;
            pos[t] = k;
            slot_map[t] = -1;
            tok_seq[t] = i;
        }
        cu[i + 1] = (i + 1) * n;
        limits[i] = -1;
        for (int b = 0; b < max_blocks; b++) block_table[(size_t)i * max_blocks + b] = 0;
    }
    return PKV_OK;
}

}  // extern "C"
