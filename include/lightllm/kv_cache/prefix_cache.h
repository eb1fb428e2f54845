#pragma once
/// Prefix caches for the MI355X build of the paged KV-cache path.
///
/// Public interface identical to the reference's
/// include/lightllm/kv_cache/prefix_cache.h:28-325 (wjb554/lightllm), so the
/// reference's own prefix-cache tests compile against this header unchanged.
/// The implementation (src: lightllm_amd/csrc/prefix_cache_*.cpp) is this
/// build's own: nodes live in an index arena with generation counters, so
/// stale block->node entries are detected instead of dereferenced.
///
///   HashPrefixCache  -- FNV-1a 64 per full block, first-miss lookup, LRU by
///                       access counter (hash_prefix_cache.cpp:23-236 semantics)
///   RadixPrefixCache -- Patricia trie keyed by first token, split on insert,
///                       LRU eviction of childless unreferenced value nodes
///                       with single-child merge (radix_prefix_cache.cpp:30-696
///                       semantics)
///
/// Not thread-safe: one caller (the step loop) serialises access.

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

namespace lightllm {
namespace kv_cache {

struct PrefixCacheResult {
    /// Tokens matched from start_pos (a multiple of block_size).
    int matched_tokens = 0;
    /// Physical block ids of the matched blocks, in order.
    std::vector<int> matched_block_ids;
};

enum class PrefixCachePolicy { Hash, Radix };

/// LIGHTLLM_PREFIX_CACHE = "radix" | "Radix" selects Radix; anything else Hash.
PrefixCachePolicy prefix_cache_policy_from_env();
const char* prefix_cache_policy_name(PrefixCachePolicy policy);

class PrefixCache {
public:
    virtual ~PrefixCache() = default;
    virtual PrefixCacheResult lookup(const std::vector<int>& tokens, int start_pos) = 0;
    virtual void insert(const std::vector<int>& tokens, int start_pos,
                        const std::vector<int>& block_ids) = 0;
    virtual void remove(int block_id) = 0;
    virtual int evict_lru() = 0;
    virtual size_t size() const = 0;
    virtual void increment_ref(int block_id) = 0;
    virtual int block_size() const = 0;
};

class HashPrefixCache : public PrefixCache {
public:
    explicit HashPrefixCache(int block_size);

    PrefixCacheResult lookup(const std::vector<int>& tokens, int start_pos) override;
    void insert(const std::vector<int>& tokens, int start_pos,
                const std::vector<int>& block_ids) override;
    void remove(int block_id) override;
    int evict_lru() override;
    size_t size() const override;
    void increment_ref(int block_id) override;
    int block_size() const override { return block_size_; }

    int find_by_hash(uint64_t token_hash) const;
    static uint64_t hash_tokens(const int* tokens, int n);

private:
    struct Entry {
        uint64_t hash;
        int refs;
        uint64_t last_access;
        size_t slot;   // position in order_
    };
    int block_size_;
    uint64_t clock_ = 0;
    std::unordered_map<uint64_t, int> by_hash_;   // hash -> block id
    std::unordered_map<int, Entry> entries_;      // block id -> entry
    std::vector<int> order_;                      // block ids, swap-pop on erase
};

/// Trie node as published by the reference header; kept for interface
/// parity.  RadixPrefixCache stores its nodes in an internal arena.
struct RadixNode {
    std::vector<int> token_segment;
    int block_id = -1;
    int ref_count = 0;
    uint64_t last_access = 0;
    std::map<int, std::unique_ptr<RadixNode>> children;
    bool is_leaf() const { return block_id >= 0; }
};

class RadixPrefixCache : public PrefixCache {
public:
    explicit RadixPrefixCache(int block_size);
    ~RadixPrefixCache() override;

    PrefixCacheResult lookup(const std::vector<int>& tokens, int start_pos) override;
    void insert(const std::vector<int>& tokens, int start_pos,
                const std::vector<int>& block_ids) override;
    void remove(int block_id) override;
    int evict_lru() override;
    size_t size() const override;
    void increment_ref(int block_id) override;
    int block_size() const override { return block_size_; }

private:
    struct Arena;
    int block_size_;
    uint64_t clock_ = 0;
    std::unique_ptr<Arena> arena_;
};

std::unique_ptr<PrefixCache> create_prefix_cache(PrefixCachePolicy policy, int block_size);

}  // namespace kv_cache
}  // namespace lightllm
