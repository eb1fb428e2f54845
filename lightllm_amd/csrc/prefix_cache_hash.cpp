// HashPrefixCache: one FNV-1a 64 hash per full block.
//
// Semantics of the reference's src/kv_cache/hash_prefix_cache.cpp:23-236:
//  * hash_tokens: FNV-1a 64 over (uint32)token (offset basis 14695981039346656037,
//    prime 1099511628211) -- a published constant pair, kept so hashes agree;
//  * lookup walks full blocks from start_pos and stops at the first miss,
//    touching each hit's LRU stamp;
//  * insert skips blocks that would run past the token array, drops a stale
//    hash of a re-inserted block, sets the block's ref count to 1 and stamps it;
//  * remove decrements the ref count (never below 0) without touching the stamp;
//  * evict_lru picks the unreferenced entry with the oldest stamp and erases it
//    everywhere;
//  * increment_ref bumps the count of a cached block and stamps it.
// Storage is this build's own: one entry record per block id plus a dense id
// vector (swap-pop on erase) scanned on eviction.
#include <cstdlib>
#include <cstring>

#include "lightllm/kv_cache/prefix_cache.h"

namespace lightllm {
namespace kv_cache {

uint64_t HashPrefixCache::hash_tokens(const int* tokens, int n) {
    uint64_t h = 14695981039346656037ULL;
    for (int i = 0; i < n; ++i) {
        h ^= static_cast<uint64_t>(static_cast<uint32_t>(tokens[i]));
        h *= 1099511628211ULL;
    }
    return h;
}

HashPrefixCache::HashPrefixCache(int block_size) : block_size_(block_size) {}

PrefixCacheResult HashPrefixCache::lookup(const std::vector<int>& tokens, int start_pos) {
    PrefixCacheResult r;
    const int n = static_cast<int>(tokens.size());
    for (int pos = start_pos; pos >= 0 && pos + block_size_ <= n; pos += block_size_) {
        auto it = by_hash_.find(hash_tokens(tokens.data() + pos, block_size_));
        if (it == by_hash_.end()) break;
        r.matched_block_ids.push_back(it->second);
        r.matched_tokens += block_size_;
        auto e = entries_.find(it->second);
        if (e != entries_.end()) e->second.last_access = ++clock_;
    }
    return r;
}

void HashPrefixCache::insert(const std::vector<int>& tokens, int start_pos,
                             const std::vector<int>& block_ids) {
    const int n = static_cast<int>(tokens.size());
    for (size_t i = 0; i < block_ids.size(); ++i) {
        const int pos = start_pos + static_cast<int>(i) * block_size_;
        if (pos < 0 || pos + block_size_ > n) continue;
        const uint64_t h = hash_tokens(tokens.data() + pos, block_size_);
        const int id = block_ids[i];
        auto e = entries_.find(id);
        if (e != entries_.end() && e->second.hash != h) {
            auto stale = by_hash_.find(e->second.hash);
            if (stale != by_hash_.end() && stale->second == id) by_hash_.erase(stale);
        }
        by_hash_[h] = id;
        if (e == entries_.end()) {
            entries_[id] = Entry{h, 1, ++clock_, order_.size()};
            order_.push_back(id);
        } else {
            e->second.hash = h;
            e->second.refs = 1;
            e->second.last_access = ++clock_;
        }
    }
}

void HashPrefixCache::remove(int block_id) {
    auto e = entries_.find(block_id);
    if (e != entries_.end() && e->second.refs > 0) --e->second.refs;
}

int HashPrefixCache::evict_lru() {
    int victim = -1;
    uint64_t oldest = UINT64_MAX;
    for (int id : order_) {
        const Entry& e = entries_.at(id);
        if (e.refs > 0) continue;
        if (e.last_access < oldest) {
            oldest = e.last_access;
            victim = id;
        }
    }
    if (victim < 0) return -1;
    Entry e = entries_.at(victim);
    auto h = by_hash_.find(e.hash);
    if (h != by_hash_.end() && h->second == victim) by_hash_.erase(h);
    const size_t slot = e.slot;
    if (slot + 1 != order_.size()) {
        order_[slot] = order_.back();
        entries_.at(order_[slot]).slot = slot;
    }
    order_.pop_back();
    entries_.erase(victim);
    return victim;
}

size_t HashPrefixCache::size() const { return by_hash_.size(); }

void HashPrefixCache::increment_ref(int block_id) {
    auto e = entries_.find(block_id);
    if (e == entries_.end()) return;
    ++e->second.refs;
    e->second.last_access = ++clock_;
}

int HashPrefixCache::find_by_hash(uint64_t token_hash) const {
    auto it = by_hash_.find(token_hash);
    return it == by_hash_.end() ? -1 : it->second;
}

// ---- policy helpers and factory --------------------------------------------

PrefixCachePolicy prefix_cache_policy_from_env() {
    const char* v = std::getenv("LIGHTLLM_PREFIX_CACHE");
    if (v && (std::strcmp(v, "radix") == 0 || std::strcmp(v, "Radix") == 0))
        return PrefixCachePolicy::Radix;
    return PrefixCachePolicy::Hash;
}

const char* prefix_cache_policy_name(PrefixCachePolicy policy) {
    switch (policy) {
        case PrefixCachePolicy::Hash: return "hash";
        case PrefixCachePolicy::Radix: return "radix";
    }
    return "unknown";
}

std::unique_ptr<PrefixCache> create_prefix_cache(PrefixCachePolicy policy, int block_size) {
    if (policy == PrefixCachePolicy::Radix) return std::make_unique<RadixPrefixCache>(block_size);
    return std::make_unique<HashPrefixCache>(block_size);
}

}  // namespace kv_cache
}  // namespace lightllm
