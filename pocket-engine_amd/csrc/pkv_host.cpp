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

#include <cstdint>
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
