// Host-side driver for AddressSanitizer + UndefinedBehaviorSanitizer runs of
// this build's own host C++: BlockAllocator / BlockTable
// (lightllm_amd/csrc/block_allocator.cpp), HashPrefixCache and
// RadixPrefixCache (prefix_cache_hash.cpp, prefix_cache_radix.cpp), the C
// handle API (allocator_capi.cpp) and the host Tensor (tensor.cpp).  Built
// from those sources with -fsanitize=address,undefined (tests/cpp/Makefile,
// target san); no GPU is touched (host or metadata-only pools).
//
// A seeded random serving workload: requests with shared prefixes look up
// their cached prefix, allocate the rest (with LRU eviction when the pool
// runs dry), publish their blocks to the prefix cache, write every byte of
// their pages, and release them in random order; plus direct allocate /
// increment_ref / evict_lru / reset calls and bad arguments.  It follows the
// semantics of the reference's src/kv_cache/block_allocator.cpp:16-248,
// hash_prefix_cache.cpp:23-236 and radix_prefix_cache.cpp:30-696, and checks
// the invariants that hold whatever the eviction order:
//   * every id returned is -1 or in [0, num_blocks);
//   * a lookup matches at most the tokens given, with valid ids (whole blocks
//     for the hash cache);
//   * a reset frees every block exactly once.
// The reference does not keep a block off the free list while its prefix
// cache still holds it: release() at ref 0 frees a cached block at once
// (block_allocator.cpp:138-147) and a later evict_lru() frees it again
// (:185-191), so the free list can hold an id twice and hand one page to two
// owners.  This build keeps that behaviour (reference_double_free below
// checks it), so the driver asserts no owner exclusivity.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <stdexcept>
#include <vector>

#include "lightllm/kv_cache/block_allocator.h"
#include "lightllm_kv.h"

using namespace lightllm;
using namespace lightllm::kv_cache;

static int passed = 0, failed = 0;
static void CHECK(const char* name, bool cond) {
    if (cond) {
        ++passed;
    } else {
        ++failed;
        if (failed < 20) std::fprintf(stderr, "  FAIL: %s\n", name);
    }
}

struct Request {
    std::vector<int> tokens;
    std::vector<int> blocks;   // one reference held on each
};

static void workload(PrefixCachePolicy policy, PoolStorage storage, uint32_t seed) {
    const int nb = 96, bs = 16, hkv = 2, d = 8;
    BlockAllocator a(nb, bs, hkv, d, policy, DType::F16, storage);
    std::mt19937 rng(seed);
    // a few shared prompt stems, so that lookups hit and radix nodes split
    std::vector<std::vector<int>> stems;
    for (int s = 0; s < 6; ++s) {
        std::vector<int> t(static_cast<size_t>(16 + rng() % 80));
        for (int& x : t) x = static_cast<int>(rng() % 50);
        stems.push_back(t);
    }
    std::vector<Request> live;
    for (int step = 0; step < 4000; ++step) {
        const int op = static_cast<int>(rng() % 10);
        if (op < 5) {
            // a new request: stem prefix + own tail
            Request r;
            const auto& stem = stems[rng() % stems.size()];
            const size_t keep = rng() % (stem.size() + 1);
            r.tokens.assign(stem.begin(), stem.begin() + static_cast<long>(keep));
            const int tail = static_cast<int>(rng() % 60);
            for (int i = 0; i < tail; ++i) r.tokens.push_back(static_cast<int>(rng() % 50));
            const int n = static_cast<int>(r.tokens.size());
            const PrefixCacheResult hit = a.find_cached_prefix(r.tokens, 0);
            CHECK("lookup within the tokens", hit.matched_tokens >= 0 && hit.matched_tokens <= n);
            // Hash matches whole blocks; Radix also records a value node that ends
            // inside a block, when a partial last block was published (the
            // reference's radix_prefix_cache.cpp:120-131)
            if (policy == PrefixCachePolicy::Hash)
                CHECK("hash lookup: whole blocks",
                      hit.matched_tokens % bs == 0 &&
                          static_cast<int>(hit.matched_block_ids.size()) * bs == hit.matched_tokens);
            CHECK("lookup ids cover the match",
                  static_cast<int>(hit.matched_block_ids.size()) == (hit.matched_tokens + bs - 1) / bs ||
                      policy == PrefixCachePolicy::Radix);
            for (int id : hit.matched_block_ids) CHECK("lookup id valid", id >= 0 && id < nb);
            std::vector<int> out;
            const int fresh = a.allocate_tokens(r.tokens.data(), n, 0, out);
            CHECK("fresh count", fresh >= 0 && fresh <= static_cast<int>(out.size()));
            bool ok = true;
            for (int id : out) ok = ok && id >= 0 && id < nb;
            CHECK("allocate_tokens ids valid", ok);
            if (storage == PoolStorage::Host)
                for (int id : out) {   // every byte of the request's pages
                    std::memset(a.k_data(id), step & 0xFF, a.block_bytes());
                    std::memset(a.v_data(id), ~step & 0xFF, a.block_bytes());
                }
            r.blocks = out;
            if (rng() % 2) a.insert_cached_blocks(r.tokens, 0, r.blocks);
            live.push_back(std::move(r));
        } else if (op < 8 && !live.empty()) {
            const size_t i = rng() % live.size();
            for (int id : live[i].blocks) a.release(id);
            live.erase(live.begin() + static_cast<long>(i));
        } else if (op == 8) {
            const uint64_t h = rng() % 3 ? 0 : (uint64_t)(rng() % 7 + 1);
            const int id = a.allocate(h);
            CHECK("allocate id valid", id >= -1 && id < nb);
            if (id >= 0) {
                Request r;
                r.blocks.push_back(id);
                if (rng() % 2 && !live.empty()) {   // a second reference on a live block
                    const Request& o = live[rng() % live.size()];
                    if (!o.blocks.empty()) {
                        a.increment_ref(o.blocks.front());
                        r.blocks.push_back(o.blocks.front());
                    }
                }
                live.push_back(std::move(r));
            }
        } else {
            const int victim = a.evict_lru();
            CHECK("evict id valid", victim >= -1 && victim < nb);
        }
        CHECK("free count non-negative", a.num_free() >= 0);
        if (step % 997 == 996) {   // reset drops every reference
            a.reset();
            live.clear();
            CHECK("reset frees every block", a.num_free() == nb);
        }
    }
    for (auto& r : live)
        for (int id : r.blocks) a.release(id);
    // out-of-range and double releases are ignored, as the reference's guards
    a.release(-1);
    a.release(nb);
    a.increment_ref(nb + 5);
    CHECK("block table throws past max", [] {
        BlockTable t(2);
        t.append(1);
        t.append(2);
        try {
            t.append(3);
        } catch (const std::runtime_error&) {
            return t.size() == 2 && t[1] == 2;
        }
        return false;
    }());
}

// The reference's release-then-evict sequence: a block of a cached prefix,
// released to ref 0, is on the free list and still in the cache; evicting it
// frees it a second time (block_allocator.cpp:138-147, 185-191 of the
// reference).  This build behaves the same, so engines see the same ids.
static void reference_double_free(PrefixCachePolicy policy) {
    const int nb = 4, bs = 16;
    BlockAllocator a(nb, bs, 1, 8, policy, DType::F16, PoolStorage::None);
    std::vector<int> tokens(bs);
    for (int i = 0; i < bs; ++i) tokens[i] = i + 1;
    std::vector<int> out;
    CHECK("one fresh block", a.allocate_tokens(tokens.data(), bs, 0, out) == 1 && out.size() == 1);
    const int id = out[0];
    a.release(id);
    CHECK("released to the free list", a.num_free() == nb);
    CHECK("and still cached", a.find_cached_prefix(tokens, 0).matched_tokens == bs);
    CHECK("evicted", a.evict_lru() == id);
    CHECK("freed a second time", a.num_free() == nb + 1);
    a.reset();
    CHECK("reset restores the count", a.num_free() == nb);
}

static void c_api(uint32_t seed) {
    llkv_allocator* h = nullptr;
    CHECK("create rejects bad geometry", llkv_allocator_create(-1, 16, 2, 8, 0, 1, 2, &h) != LLKV_OK);
    CHECK("create rejects null out", llkv_allocator_create(8, 16, 2, 8, 0, 1, 2, nullptr) != LLKV_OK);
    for (int policy = 0; policy < 2; ++policy) {
        CHECK("create", llkv_allocator_create(40, 16, 2, 8, policy, 1, 1, &h) == LLKV_OK && h);
        std::mt19937 rng(seed + policy);
        std::vector<int> tokens(200);
        for (int& t : tokens) t = static_cast<int>(rng() % 9);
        int blocks[64], n = 0;
        const int fresh = llkv_allocator_allocate_tokens(h, tokens.data(), 200, 0, blocks, 4, &n);
        CHECK("allocate_tokens through the handle", fresh == 13 && n == 13);   // capacity 4: 4 written
        std::vector<int> ids(blocks, blocks + 4);
        int n_ids = 0, got[64];
        llkv_allocator_insert_cached_blocks(h, tokens.data(), 64, 0, ids.data(), 4);
        const int matched = llkv_allocator_find_cached_prefix(h, tokens.data(), 200, 0, got, 2, &n_ids);
        CHECK("find_cached_prefix bounded by capacity", matched >= 0 && matched <= 200 && n_ids >= 0);
        CHECK("hash of a block", llkv_hash_tokens(tokens.data(), 16) != 0);
        CHECK("allocate_tokens null tokens", llkv_allocator_allocate_tokens(h, nullptr, 5, 0, blocks, 64, &n) == -1);
        for (int i = 0; i < 40; ++i) llkv_allocator_allocate(h, 0);
        CHECK("exhausted pool evicts or fails", llkv_allocator_allocate(h, 0) >= -1);
        CHECK("storage pointer", llkv_allocator_k_storage(h) != nullptr);
        CHECK("reset", llkv_allocator_reset(h) == LLKV_OK && llkv_allocator_num_free(h) == 40);
        llkv_allocator_release(h, 1000);
        llkv_allocator_destroy(h);
        h = nullptr;
    }
    llkv_allocator_destroy(nullptr);
    CHECK("budget", llkv_blocks_for_budget(1 << 20, 16, 2, 8, 1) == 1024);
    CHECK("budget bad args", llkv_blocks_for_budget(1 << 20, 0, 2, 8, 1) == -1);
}

static void tensors() {
    Tensor t({3, 5, 7}, DType::F16, Device::CPU);
    std::vector<uint16_t> src(105, 0x3C00), dst(105, 0);
    t.copy_from(src.data(), src.size() * 2);
    t.copy_to(dst.data(), dst.size() * 2);
    CHECK("host tensor round trip", src == dst);
    Tensor u = std::move(t);
    CHECK("move leaves the source empty", !t.defined() && u.defined() && u.numel() == 105);
    u.fill_zeros();
    u.copy_to(dst.data(), dst.size() * 2);
    CHECK("fill_zeros", dst == std::vector<uint16_t>(105, 0));
    Tensor v = u.view({15, 7});
    CHECK("view shares the data", v.raw() == u.raw() && v.size(0) == 15 && v.size(-1) == 7);
    bool threw = false;
    try {
        Tensor bad({-1, 4}, DType::F32, Device::CPU);
    } catch (const std::exception&) {
        threw = true;
    }
    CHECK("negative dimension throws", threw);
}

int main(int argc, char** argv) {
    const uint32_t seed = argc > 1 ? static_cast<uint32_t>(std::strtoul(argv[1], nullptr, 10)) : 1u;
    for (uint32_t s = seed; s < seed + 4; ++s) {
        workload(PrefixCachePolicy::Hash, PoolStorage::Host, s);
        workload(PrefixCachePolicy::Radix, PoolStorage::Host, s);
        workload(PrefixCachePolicy::Hash, PoolStorage::None, s + 100);
        workload(PrefixCachePolicy::Radix, PoolStorage::None, s + 100);
    }
    reference_double_free(PrefixCachePolicy::Hash);
    reference_double_free(PrefixCachePolicy::Radix);
    c_api(seed);
    tensors();
    std::printf("test_host_san: %d passed, %d failed\n", passed, failed);
    return failed == 0 ? 0 : 1;
}
