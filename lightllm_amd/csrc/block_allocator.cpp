// BlockAllocator / BlockTable for the MI355X build.
//
// Semantics of the reference's src/kv_cache/block_allocator.cpp:16-248:
//  allocate(hash):  Hash policy + non-zero hash probes the cache first (hit ->
//                   ref+1, same id); otherwise pop the FIFO free list, and on
//                   exhaustion evict one LRU cache entry and retry once; the
//                   block's token_hash is set to `hash`.
//  allocate_tokens: cache lookup from start_pos, adopt the matched blocks
//                   (ref+1), allocate fresh blocks while the covered position
//                   is below n_tokens (returning early on exhaustion), insert
//                   the fresh blocks into the cache and, under Hash, record the
//                   hashes of the full ones.
//  release:         ref-1 (ignored at 0); reaching 0 removes the block from
//                   the cache and pushes it to the back of the free list.
//  reset:           all metadata, a fresh cache, zeroed pools.
#include "lightllm/kv_cache/block_allocator.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <stdexcept>

namespace lightllm {
namespace kv_cache {

namespace {
Device pool_device(PoolStorage s) { return s == PoolStorage::Host ? Device::CPU : Device::CUDA; }
std::vector<int> pool_shape(PoolStorage s, int nb, int bs, int h, int d) {
    if (s == PoolStorage::None) return {0};
    return {nb, bs, h, d};
}
}  // namespace

BlockAllocator::BlockAllocator(int num_blocks, int block_size, int num_kv_heads, int head_dim,
                               PrefixCachePolicy policy, DType kv_dtype, PoolStorage storage)
    : num_blocks_(num_blocks), block_size_(block_size), num_kv_heads_(num_kv_heads),
      head_dim_(head_dim), kv_dtype_(kv_dtype), policy_(policy), storage_(storage),
      prefix_cache_(create_prefix_cache(policy, block_size)),
      k_storage_(pool_shape(storage, num_blocks, block_size, num_kv_heads, head_dim), kv_dtype,
                 pool_device(storage)),
      v_storage_(pool_shape(storage, num_blocks, block_size, num_kv_heads, head_dim), kv_dtype,
                 pool_device(storage)) {
    if (num_blocks < 0 || block_size <= 0 || num_kv_heads <= 0 || head_dim <= 0)
        throw std::runtime_error("BlockAllocator: bad geometry");
    blocks_.resize(static_cast<size_t>(num_blocks));
    for (int i = 0; i < num_blocks; ++i) {
        blocks_[i].block_id = i;
        free_list_.push_back(i);
    }
}

size_t BlockAllocator::block_bytes() const {
    return static_cast<size_t>(block_size_) * num_kv_heads_ * head_dim_ * dtype_size(kv_dtype_);
}

int BlockAllocator::allocate_free_block() {
    if (free_list_.empty()) return -1;
    const int id = free_list_.front();
    free_list_.pop_front();
    blocks_[id].ref_count = 1;
    blocks_[id].token_hash = 0;
    return id;
}

int BlockAllocator::allocate_with_eviction() {
    int id = allocate_free_block();
    if (id < 0 && evict_lru() >= 0) id = allocate_free_block();
    return id;
}

void BlockAllocator::free_block_physical(int block_id) {
    if (block_id < 0 || block_id >= num_blocks_) return;
    blocks_[block_id].token_hash = 0;
    blocks_[block_id].ref_count = 0;
    free_list_.push_back(block_id);
}

int BlockAllocator::allocate(uint64_t token_hash) {
    if (token_hash != 0 && policy_ == PrefixCachePolicy::Hash) {
        const int cached = find_by_hash(token_hash);
        if (cached >= 0) {
            ++blocks_[cached].ref_count;
            return cached;
        }
    }
    const int id = allocate_with_eviction();
    if (id < 0) return -1;
    blocks_[id].token_hash = token_hash;
    return id;
}

int BlockAllocator::allocate_tokens(const int* tokens, int n_tokens, int start_pos,
                                    std::vector<int>& out_blocks) {
    std::vector<int> seq(tokens, tokens + (n_tokens > 0 ? n_tokens : 0));
    PrefixCacheResult hit = prefix_cache_->lookup(seq, start_pos);
    for (int id : hit.matched_block_ids) {
        ++blocks_[id].ref_count;
        out_blocks.push_back(id);
    }
    const int first_new = start_pos + hit.matched_tokens;
    int n_new = 0;
    for (int covered = first_new; covered < n_tokens; covered += block_size_) {
        const int id = allocate_with_eviction();
        if (id < 0) return n_new;   // exhausted: out_blocks is short
        out_blocks.push_back(id);
        ++n_new;
    }
    if (n_new > 0) {
        std::vector<int> fresh(out_blocks.end() - n_new, out_blocks.end());
        prefix_cache_->insert(seq, first_new, fresh);
        if (policy_ == PrefixCachePolicy::Hash) {
            for (int i = 0; i < n_new; ++i) {
                const int off = first_new + i * block_size_;
                if (off + block_size_ <= n_tokens)
                    blocks_[fresh[i]].token_hash = HashPrefixCache::hash_tokens(tokens + off, block_size_);
            }
        }
    }
    return n_new;
}

void BlockAllocator::release(int block_id) {
    if (block_id < 0 || block_id >= num_blocks_) return;
    Block& b = blocks_[block_id];
    if (b.ref_count <= 0) return;
    if (--b.ref_count == 0) {
        prefix_cache_->remove(block_id);
        free_block_physical(block_id);
    }
}

int BlockAllocator::find_by_hash(uint64_t token_hash) const {
    if (policy_ != PrefixCachePolicy::Hash) return -1;
    return static_cast<const HashPrefixCache*>(prefix_cache_.get())->find_by_hash(token_hash);
}

PrefixCacheResult BlockAllocator::find_cached_prefix(const std::vector<int>& tokens,
                                                     int start_pos) const {
    return prefix_cache_->lookup(tokens, start_pos);
}

void BlockAllocator::insert_cached_blocks(const std::vector<int>& tokens, int start_pos,
                                          const std::vector<int>& block_ids) {
    prefix_cache_->insert(tokens, start_pos, block_ids);
    if (policy_ != PrefixCachePolicy::Hash) return;
    for (size_t i = 0; i < block_ids.size(); ++i) {
        const int off = start_pos + static_cast<int>(i) * block_size_;
        const int id = block_ids[i];
        if (id < 0 || id >= num_blocks_) continue;
        if (off + block_size_ <= static_cast<int>(tokens.size()))
            blocks_[id].token_hash = HashPrefixCache::hash_tokens(tokens.data() + off, block_size_);
    }
}

int BlockAllocator::evict_lru() {
    const int victim = prefix_cache_->evict_lru();
    if (victim >= 0) free_block_physical(victim);
    return victim;
}

void BlockAllocator::increment_ref(int block_id) {
    if (block_id < 0 || block_id >= num_blocks_) return;
    ++blocks_[block_id].ref_count;
    prefix_cache_->increment_ref(block_id);
}

int BlockAllocator::blocks_for_budget(size_t budget_bytes, int block_size, int num_kv_heads,
                                      int head_dim, DType kv_dtype) {
    const size_t esize = kv_dtype == DType::F32 ? 4 : 2;
    const size_t per_block = (size_t)block_size * num_kv_heads * head_dim * esize * 2;
    if (per_block == 0) return 0;
    const size_t n = budget_bytes / per_block;
    return n > (size_t)INT32_MAX ? INT32_MAX : (int)n;
}

void BlockAllocator::zero_pools() {
    if (!k_storage_.defined()) return;
    k_storage_.fill_zeros();
    v_storage_.fill_zeros();
}

void BlockAllocator::reset() {
    for (Block& b : blocks_) {
        b.ref_count = 0;
        b.token_hash = 0;
    }
    free_list_.clear();
    for (int i = 0; i < num_blocks_; ++i) free_list_.push_back(i);
    prefix_cache_ = create_prefix_cache(policy_, block_size_);
    zero_pools();
}

void* BlockAllocator::k_data(int block_id) {
    return static_cast<char*>(k_storage_.raw()) + static_cast<size_t>(block_id) * block_bytes();
}

void* BlockAllocator::v_data(int block_id) {
    return static_cast<char*>(v_storage_.raw()) + static_cast<size_t>(block_id) * block_bytes();
}

BlockTable::BlockTable(int max_blocks) : max_blocks_(max_blocks) { blocks_.reserve(max_blocks); }

void BlockTable::append(int physical_id) {
    if (static_cast<int>(blocks_.size()) >= max_blocks_)
        throw std::runtime_error("BlockTable: exceeded max_blocks");
    blocks_.push_back(physical_id);
}

int BlockTable::operator[](int pos) const { return blocks_[static_cast<size_t>(pos)]; }

}  // namespace kv_cache
}  // namespace lightllm
