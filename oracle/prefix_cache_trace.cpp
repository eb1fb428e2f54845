// Prefix-cache trace driver -- TEST INFRASTRUCTURE ONLY.
//
// Drives the PrefixCache public API (include/lightllm/kv_cache/prefix_cache.h,
// identical in the reference and in this build) through an engine-like,
// seeded sequence of operations and prints every observable result.  Built
// twice by oracle/Makefile: against the reference's sources
// (src/kv_cache/{hash,radix}_prefix_cache.cpp of wjb554/lightllm, into
// oracle/_ref/) and against this build's (lightllm_amd/csrc); the tests
// compare the two outputs line by line.
//
// The protocol mirrors the reference engine (src/engine/engine_server.cpp:
// 1403-1439 lookup + adopt + allocate; :1886-1914 insert; :694-704 release
// -> BlockAllocator::release -> PrefixCache::remove at ref 0,
// src/kv_cache/block_allocator.cpp:138-147; eviction on exhaustion :66-75).
//
// The reference build is compiled with AddressSanitizer: its radix cache keeps
// block -> node pointers to nodes it has freed (RadixPrefixCache::remove,
// src/kv_cache/radix_prefix_cache.cpp:373-377, reached through stale entries
// after prune/merge), so a trace is an oracle only up to the first reported
// use-after-free.
//
// usage: trace <hash|radix> <block_size> <seed> <n_ops> <pool_blocks>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <vector>

#include "lightllm/kv_cache/prefix_cache.h"

using namespace lightllm::kv_cache;

namespace {

struct Rng {
    uint64_t s;
    uint32_t next() {
        s = s * 6364136223846793005ULL + 1442695040888963407ULL;
        return static_cast<uint32_t>(s >> 33);
    }
    int below(int n) { return n <= 0 ? 0 : static_cast<int>(next() % static_cast<uint32_t>(n)); }
};

struct Seq {
    std::vector<int> tokens;
    std::vector<int> blocks;   // blocks this sequence holds a reference on
};

void print_ids(const char* tag, const std::vector<int>& ids) {
    std::printf("%s[", tag);
    for (size_t i = 0; i < ids.size(); ++i) std::printf(i ? ",%d" : "%d", ids[i]);
    std::printf("]");
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 6) {
        std::fprintf(stderr, "usage: %s <hash|radix> <block_size> <seed> <n_ops> <pool>\n", argv[0]);
        return 2;
    }
    // Line-buffered: when the reference build aborts on undefined behaviour
    // (AddressSanitizer), every completed op line before it is still emitted.
    std::setvbuf(stdout, nullptr, _IOLBF, 0);
    const bool radix = std::strcmp(argv[1], "radix") == 0;
    const int bs = std::atoi(argv[2]);
    Rng rng{static_cast<uint64_t>(std::strtoull(argv[3], nullptr, 10)) * 2654435761ULL + 7};
    const int n_ops = std::atoi(argv[4]);
    const int pool = std::atoi(argv[5]);

    std::unique_ptr<PrefixCache> cache =
        create_prefix_cache(radix ? PrefixCachePolicy::Radix : PrefixCachePolicy::Hash, bs);
    std::printf("policy=%s bs=%d\n", prefix_cache_policy_name(radix ? PrefixCachePolicy::Radix
                                                                      : PrefixCachePolicy::Hash),
                cache->block_size());

    std::vector<int> refs(static_cast<size_t>(pool), 0);   // allocator-level ref counts
    std::vector<int> free_list;
    for (int i = 0; i < pool; ++i) free_list.push_back(i);
    size_t free_head = 0;
    std::vector<Seq> live;
    // A few shared prompt prefixes so lookups hit, split and diverge.
    std::vector<std::vector<int>> prefixes(4);
    for (auto& p : prefixes) {
        int len = bs * (1 + rng.below(4)) + rng.below(bs);
        for (int i = 0; i < len; ++i) p.push_back(rng.below(6));
    }

    auto take_free = [&]() -> int {
        if (free_head < free_list.size()) return free_list[free_head++];
        int ev = cache->evict_lru();
        std::printf(" evict=%d", ev);
        if (ev < 0) return -1;
        return ev;   // evicted blocks have ref 0 and were already returned below
    };
    auto give_back = [&](int id) {
        // release to ref 0: cache->remove then back to the free list (FIFO)
        cache->remove(id);
        free_list.push_back(id);
    };

    for (int op = 0; op < n_ops; ++op) {
        int kind = rng.below(10);
        std::printf("op%d ", op);
        if (kind <= 3 || live.empty()) {
            // new request: shared prefix + random suffix
            Seq s;
            const auto& pre = prefixes[static_cast<size_t>(rng.below(4))];
            int keep = rng.below(static_cast<int>(pre.size()) + 1);
            s.tokens.assign(pre.begin(), pre.begin() + keep);
            int extra = rng.below(3 * bs);
            for (int i = 0; i < extra; ++i) s.tokens.push_back(rng.below(6));
            PrefixCacheResult r = cache->lookup(s.tokens, 0);
            std::printf("new n=%zu matched=%d ", s.tokens.size(), r.matched_tokens);
            print_ids("ids", r.matched_block_ids);
            for (int id : r.matched_block_ids) {
                cache->increment_ref(id);
                if (id >= 0 && id < pool) refs[id]++;
                s.blocks.push_back(id);
            }
            int full = static_cast<int>(s.tokens.size()) / bs;
            std::vector<int> fresh;
            for (int b = static_cast<int>(s.blocks.size()); b < full; ++b) {
                int id = take_free();
                if (id < 0) break;
                refs[id] = 1;
                fresh.push_back(id);
            }
            if (!fresh.empty()) {
                cache->insert(s.tokens, static_cast<int>(s.blocks.size()) * bs, fresh);
                for (int id : fresh) s.blocks.push_back(id);
            }
            print_ids(" fresh", fresh);
            live.push_back(s);
        } else if (kind <= 5) {
            // extend a live request by up to two blocks and insert its new full blocks
            Seq& s = live[static_cast<size_t>(rng.below(static_cast<int>(live.size())))];
            int extra = rng.below(2 * bs + 1);
            for (int i = 0; i < extra; ++i) s.tokens.push_back(rng.below(6));
            int start = static_cast<int>(s.blocks.size()) * bs;
            PrefixCacheResult r = cache->lookup(s.tokens, start);
            std::printf("extend n=%zu start=%d matched=%d ", s.tokens.size(), start, r.matched_tokens);
            print_ids("ids", r.matched_block_ids);
            int full = static_cast<int>(s.tokens.size()) / bs;
            std::vector<int> fresh;
            for (int b = static_cast<int>(s.blocks.size()); b < full; ++b) {
                int id = take_free();
                if (id < 0) break;
                refs[id] = 1;
                fresh.push_back(id);
            }
            if (!fresh.empty()) {
                cache->insert(s.tokens, start, fresh);
                for (int id : fresh) s.blocks.push_back(id);
            }
            print_ids(" fresh", fresh);
        } else if (kind <= 7) {
            // release a live request
            size_t i = static_cast<size_t>(rng.below(static_cast<int>(live.size())));
            std::printf("release ");
            print_ids("ids", live[i].blocks);
            for (int id : live[i].blocks) {
                if (id < 0 || id >= pool || refs[id] <= 0) continue;
                if (--refs[id] == 0) give_back(id);
            }
            live.erase(live.begin() + static_cast<long>(i));
        } else if (kind == 8) {
            // probe lookup at a random start
            const auto& pre = prefixes[static_cast<size_t>(rng.below(4))];
            std::vector<int> t(pre.begin(), pre.end());
            int extra = rng.below(2 * bs);
            for (int i = 0; i < extra; ++i) t.push_back(rng.below(6));
            int start = bs * rng.below(static_cast<int>(t.size()) / bs + 1);
            PrefixCacheResult r = cache->lookup(t, start);
            std::printf("probe n=%zu start=%d matched=%d ", t.size(), start, r.matched_tokens);
            print_ids("ids", r.matched_block_ids);
        } else {
            int ev = cache->evict_lru();
            std::printf("evict=%d", ev);
            if (ev >= 0) {
                // the evicted block is already on the free list (ref 0); nothing else to do
            }
        }
        std::printf(" size=%zu\n", cache->size());
    }
    return 0;
}
