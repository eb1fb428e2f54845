#pragma once
/// Block pool + per-sequence block table for the MI355X build.
///
/// Interface of the reference's include/lightllm/kv_cache/block_allocator.h:
/// 31-186 (wjb554/lightllm), semantics of src/kv_cache/block_allocator.cpp:
/// 16-248: FIFO free list (pop front, push back), ref counts, hash-probe in
/// allocate(), one LRU eviction + retry on exhaustion, release-to-zero frees
/// and removes from the prefix cache, reset() rebuilds everything.
///
/// Pools: K and V, each [num_blocks, block_size, num_kv_heads, head_dim] of
/// kv_dtype, allocated once.  Sizes are size_t throughout, so pools sized for
/// the 288 GB of an MI355X (e.g. 262144 Llama-3-8B blocks = 2 x 8.6 GB) index
/// correctly.  One optional constructor argument (storage) selects device
/// pools (default, as the reference), host pools, or no pools (metadata only).

#include <cstdint>
#include <deque>
#include <memory>
#include <string>
#include <vector>

#include "lightllm/kv_cache/prefix_cache.h"
#include "lightllm/tensor.h"

namespace lightllm {
namespace kv_cache {

struct Block {
    int block_id;
    int ref_count = 0;
    uint64_t token_hash = 0;
};

enum class PoolStorage : uint8_t { Device = 0, Host = 1, None = 2 };

class BlockAllocator {
public:
    BlockAllocator(int num_blocks, int block_size, int num_kv_heads, int head_dim,
                   PrefixCachePolicy policy = PrefixCachePolicy::Hash,
                   DType kv_dtype = DType::F32, PoolStorage storage = PoolStorage::Device);

    /// Pages of (K + V) pools that fit in budget_bytes for this element type (new; the
    /// reference's engine sizes pools as fp32 in EngineServer's constructor,
    /// src/engine/engine_server.cpp:418-422 and :470-476).  At 288 GB and 16-token pages of
    /// 8 kv heads x 128 dims in fp16 that is 4.4 million pages; clamped to INT32_MAX.
    static int blocks_for_budget(size_t budget_bytes, int block_size, int num_kv_heads, int head_dim,
                                 DType kv_dtype);

    int allocate(uint64_t token_hash = 0);
    int allocate_tokens(const int* tokens, int n_tokens, int start_pos,
                        std::vector<int>& out_blocks);
    void release(int block_id);

    int find_by_hash(uint64_t token_hash) const;
    PrefixCacheResult find_cached_prefix(const std::vector<int>& tokens, int start_pos) const;
    void insert_cached_blocks(const std::vector<int>& tokens, int start_pos,
                              const std::vector<int>& block_ids);
    int evict_lru();
    void increment_ref(int block_id);
    void reset();

    void* k_data(int block_id);
    void* v_data(int block_id);
    const void* k_storage_raw() const { return k_storage_.raw(); }
    const void* v_storage_raw() const { return v_storage_.raw(); }
    size_t k_storage_bytes() const { return k_storage_.nbytes(); }
    size_t v_storage_bytes() const { return v_storage_.nbytes(); }

    int num_blocks() const { return num_blocks_; }
    int block_size() const { return block_size_; }
    int num_free() const { return static_cast<int>(free_list_.size()); }
    int num_kv_heads() const { return num_kv_heads_; }
    int head_dim() const { return head_dim_; }
    DType kv_dtype() const { return kv_dtype_; }
    PoolStorage storage() const { return storage_; }

    PrefixCachePolicy policy() const { return policy_; }
    const PrefixCache* prefix_cache() const { return prefix_cache_.get(); }

    /// Metadata of one block (ref count, hash) for inspection.
    const Block& block(int block_id) const { return blocks_[static_cast<size_t>(block_id)]; }
    /// Bytes of one block-layer of K (or V).
    size_t block_bytes() const;

private:
    int num_blocks_, block_size_, num_kv_heads_, head_dim_;
    DType kv_dtype_ = DType::F32;
    PrefixCachePolicy policy_;
    PoolStorage storage_;
    std::vector<Block> blocks_;
    std::deque<int> free_list_;
    // The prefix cache is logically const for lookups but updates LRU stamps.
    mutable std::unique_ptr<PrefixCache> prefix_cache_;
    Tensor k_storage_, v_storage_;

    int allocate_free_block();
    int allocate_with_eviction();
    void free_block_physical(int block_id);
    void zero_pools();
};

class BlockTable {
public:
    explicit BlockTable(int max_blocks);
    void append(int physical_id);
    int operator[](int pos) const;
    int size() const { return static_cast<int>(blocks_.size()); }
    const int* data() const { return blocks_.data(); }

private:
    int max_blocks_;
    std::vector<int> blocks_;
};

}  // namespace kv_cache
}  // namespace lightllm
