// C ABI over BlockAllocator (handle-based) for non-C++ callers.
#include <cstring>
#include <new>
#include <stdexcept>
#include <vector>

#include "common.h"
#include "lightllm/kv_cache/block_allocator.h"
#include "lightllm_kv.h"

using lightllm::DType;
using lightllm::kv_cache::BlockAllocator;
using lightllm::kv_cache::PoolStorage;
using lightllm::kv_cache::PrefixCachePolicy;

struct llkv_allocator {
    BlockAllocator impl;
    template <typename... A>
    explicit llkv_allocator(A&&... a) : impl(std::forward<A>(a)...) {}
};

extern "C" int llkv_allocator_create(int num_blocks, int block_size, int num_kv_heads, int head_dim,
                                     int policy, int dtype, int storage, llkv_allocator** out) {
    if (!out) return llkv::set_error(LLKV_ERR_INVALID, "llkv_allocator_create: null out");
    *out = nullptr;
    if (num_blocks < 0 || block_size <= 0 || num_kv_heads <= 0 || head_dim <= 0 || policy < 0 ||
        policy > 1 || dtype < 0 || dtype > 2 || storage < 0 || storage > 2)
        return llkv::set_error(LLKV_ERR_INVALID, "llkv_allocator_create: bad arguments");
    try {
        *out = new llkv_allocator(num_blocks, block_size, num_kv_heads, head_dim,
                                  policy == 1 ? PrefixCachePolicy::Radix : PrefixCachePolicy::Hash,
                                  static_cast<DType>(dtype), static_cast<PoolStorage>(storage));
    } catch (const std::exception& e) {
        return llkv::set_error(LLKV_ERR_HIP, "llkv_allocator_create: %s", e.what());
    }
    return LLKV_OK;
}

extern "C" void llkv_allocator_destroy(llkv_allocator* a) { delete a; }

extern "C" int llkv_allocator_allocate(llkv_allocator* a, uint64_t token_hash) {
    return a ? a->impl.allocate(token_hash) : -1;
}

extern "C" int llkv_allocator_allocate_tokens(llkv_allocator* a, const int* tokens, int n_tokens,
                                              int start_pos, int* out_blocks, int out_capacity,
                                              int* out_count) {
    if (!a || (n_tokens > 0 && !tokens)) return -1;
    std::vector<int> blocks;
    const int n_new = a->impl.allocate_tokens(tokens, n_tokens, start_pos, blocks);
    const int n = static_cast<int>(blocks.size());
    if (out_count) *out_count = n;
    for (int i = 0; i < n && i < out_capacity; ++i) out_blocks[i] = blocks[i];
    return n_new;
}

extern "C" void llkv_allocator_release(llkv_allocator* a, int block_id) {
    if (a) a->impl.release(block_id);
}

extern "C" int llkv_allocator_find_by_hash(llkv_allocator* a, uint64_t token_hash) {
    return a ? a->impl.find_by_hash(token_hash) : -1;
}

extern "C" int llkv_allocator_find_cached_prefix(llkv_allocator* a, const int* tokens, int n_tokens,
                                                 int start_pos, int* block_ids, int capacity,
                                                 int* n_ids) {
    if (!a) return 0;
    std::vector<int> seq(tokens, tokens + (n_tokens > 0 ? n_tokens : 0));
    auto r = a->impl.find_cached_prefix(seq, start_pos);
    const int n = static_cast<int>(r.matched_block_ids.size());
    if (n_ids) *n_ids = n;
    for (int i = 0; i < n && i < capacity; ++i) block_ids[i] = r.matched_block_ids[i];
    return r.matched_tokens;
}

extern "C" void llkv_allocator_insert_cached_blocks(llkv_allocator* a, const int* tokens,
                                                    int n_tokens, int start_pos,
                                                    const int* block_ids, int n_ids) {
    if (!a) return;
    std::vector<int> seq(tokens, tokens + (n_tokens > 0 ? n_tokens : 0));
    std::vector<int> ids(block_ids, block_ids + (n_ids > 0 ? n_ids : 0));
    a->impl.insert_cached_blocks(seq, start_pos, ids);
}

extern "C" int llkv_allocator_evict_lru(llkv_allocator* a) { return a ? a->impl.evict_lru() : -1; }

extern "C" void llkv_allocator_increment_ref(llkv_allocator* a, int block_id) {
    if (a) a->impl.increment_ref(block_id);
}

extern "C" int llkv_allocator_reset(llkv_allocator* a) {
    if (!a) return llkv::set_error(LLKV_ERR_INVALID, "llkv_allocator_reset: null handle");
    try {
        a->impl.reset();
    } catch (const std::exception& e) {
        return llkv::set_error(LLKV_ERR_HIP, "llkv_allocator_reset: %s", e.what());
    }
    return LLKV_OK;
}

extern "C" int llkv_allocator_num_free(const llkv_allocator* a) { return a ? a->impl.num_free() : 0; }
extern "C" int llkv_allocator_num_blocks(const llkv_allocator* a) { return a ? a->impl.num_blocks() : 0; }

extern "C" int llkv_allocator_ref_count(const llkv_allocator* a, int block_id) {
    if (!a || block_id < 0 || block_id >= a->impl.num_blocks()) return -1;
    return a->impl.block(block_id).ref_count;
}

extern "C" uint64_t llkv_allocator_token_hash(const llkv_allocator* a, int block_id) {
    if (!a || block_id < 0 || block_id >= a->impl.num_blocks()) return 0;
    return a->impl.block(block_id).token_hash;
}

extern "C" size_t llkv_allocator_prefix_cache_size(const llkv_allocator* a) {
    return a ? a->impl.prefix_cache()->size() : 0;
}

extern "C" void* llkv_allocator_k_storage(llkv_allocator* a) {
    return a ? const_cast<void*>(a->impl.k_storage_raw()) : nullptr;
}
extern "C" void* llkv_allocator_v_storage(llkv_allocator* a) {
    return a ? const_cast<void*>(a->impl.v_storage_raw()) : nullptr;
}
extern "C" size_t llkv_allocator_storage_bytes(const llkv_allocator* a) {
    return a ? a->impl.k_storage_bytes() : 0;
}

extern "C" uint64_t llkv_hash_tokens(const int* tokens, int n) {
    return lightllm::kv_cache::HashPrefixCache::hash_tokens(tokens, n);
}

extern "C" int llkv_blocks_for_budget(uint64_t budget_bytes, int block_size, int num_kv_heads,
                                      int head_dim, int dtype) {
    if (block_size <= 0 || num_kv_heads <= 0 || head_dim <= 0 || dtype < 0 || dtype > 2) return -1;
    return BlockAllocator::blocks_for_budget(budget_bytes, block_size, num_kv_heads, head_dim,
                                             static_cast<DType>(dtype));
}
