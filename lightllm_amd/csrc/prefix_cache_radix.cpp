// RadixPrefixCache: Patricia trie over token ids, one value node per cached
// block.
//
// Observable semantics follow the reference's src/kv_cache/radix_prefix_cache.cpp
// (lookup :51-134, insert :150-361, remove/increment_ref :371-395,
// evict_lru :408-434, pre-order LRU search :512-534, prune + single-child
// merge :563-630), including its corner cases:
//  * lookup first walks tokens[0, start_pos) without recording; if the tree
//    cannot reach start_pos it restarts matching at the root from start_pos;
//    value nodes fully matched beyond start_pos are recorded;
//  * insert re-walks to start_pos (falling back to the root), then per block
//    creates a leaf, descends through full matches (bumping a matched value
//    node's ref count), or splits a partially matched node -- the new
//    intermediate takes over the split node's children, and becomes the
//    block's value node when the block ends exactly at the split point;
//  * evict_lru takes the unreferenced, childless value node with the oldest
//    stamp (first in pre-order on ties), unlinks it and merges a valueless
//    non-root parent left with one child into that child.
//
// Representation (this build's own): nodes live in an index arena with
// parent links and a generation counter per slot.  The block -> node map
// stores (index, generation); entries whose node was freed by an eviction or
// merge are detected as stale and ignored instead of being dereferenced.
#include <algorithm>
#include <cstdint>
#include <utility>

#include "lightllm/kv_cache/prefix_cache.h"

namespace lightllm {
namespace kv_cache {

struct RadixPrefixCache::Arena {
    struct Node {
        std::vector<int> seg;
        int block = -1;
        int refs = 0;
        uint64_t stamp = 0;
        int parent = -1;
        uint32_t gen = 0;
        bool live = false;
        std::map<int, int> kids;   // first token of the child's segment -> node
    };
    struct Ref {
        int node;
        uint32_t gen;
    };

    std::vector<Node> nodes;
    std::vector<int> free_slots;
    std::unordered_map<int, Ref> by_block;   // block id -> value node

    int make() {
        int id;
        if (!free_slots.empty()) {
            id = free_slots.back();
            free_slots.pop_back();
        } else {
            id = static_cast<int>(nodes.size());
            nodes.emplace_back();
        }
        Node& n = nodes[id];
        uint32_t gen = n.gen;
        n = Node();
        n.gen = gen;
        n.live = true;
        return id;
    }
    void free_subtree(int id) {
        std::vector<int> stack{id};
        while (!stack.empty()) {
            int x = stack.back();
            stack.pop_back();
            for (auto& kv : nodes[x].kids) stack.push_back(kv.second);
            release(x);
        }
    }
    void release(int id) {
        Node& n = nodes[id];
        n.live = false;
        n.kids.clear();
        n.seg.clear();
        ++n.gen;
        free_slots.push_back(id);
    }
    void map_block(int block, int node) { by_block[block] = Ref{node, nodes[node].gen}; }
    // Live node of a block id, or -1 (unknown or stale).
    int node_of(int block) const {
        auto it = by_block.find(block);
        if (it == by_block.end()) return -1;
        const Node& n = nodes[it->second.node];
        return (n.live && n.gen == it->second.gen) ? it->second.node : -1;
    }
    void link(int parent, int key, int child) {
        auto it = nodes[parent].kids.find(key);
        if (it != nodes[parent].kids.end() && it->second != child) free_subtree(it->second);
        nodes[parent].kids[key] = child;
        nodes[child].parent = parent;
    }
    int find_child(int node, int token) const {
        auto it = nodes[node].kids.find(token);
        return it == nodes[node].kids.end() ? -1 : it->second;
    }
};

static int common_prefix(const std::vector<int>& tokens, int pos, const std::vector<int>& seg,
                         int limit) {
    int k = 0;
    while (k < limit && tokens[pos + k] == seg[k]) ++k;
    return k;
}

RadixPrefixCache::RadixPrefixCache(int block_size)
    : block_size_(block_size), arena_(std::make_unique<Arena>()) {
    arena_->make();   // node 0: the root, a pure routing node
}

RadixPrefixCache::~RadixPrefixCache() = default;

PrefixCacheResult RadixPrefixCache::lookup(const std::vector<int>& tokens, int start_pos) {
    PrefixCacheResult r;
    Arena& A = *arena_;
    const int n = static_cast<int>(tokens.size());
    const uint64_t now = ++clock_;
    int node = 0, pos = 0;
    bool reached = start_pos == 0;
    if (start_pos > 0) {
        while (pos < start_pos && pos < n) {
            int c = A.find_child(node, tokens[pos]);
            if (c < 0) break;
            const int seg_len = static_cast<int>(A.nodes[c].seg.size());
            const int lim = std::min(seg_len, start_pos - pos);
            if (pos + lim > n) break;
            const int k = common_prefix(tokens, pos, A.nodes[c].seg, lim);
            if (k < lim) break;
            pos += k;
            node = c;
            A.nodes[node].stamp = now;
            if (k < seg_len) break;
        }
        reached = pos == start_pos;
    }
    if (!reached) {
        node = 0;
        pos = start_pos;
    }
    while (pos >= 0 && pos < n) {
        int c = A.find_child(node, tokens[pos]);
        if (c < 0) break;
        const int seg_len = static_cast<int>(A.nodes[c].seg.size());
        const int k = common_prefix(tokens, pos, A.nodes[c].seg, std::min(seg_len, n - pos));
        if (k < seg_len) {
            A.nodes[c].stamp = now;
            break;
        }
        pos += k;
        node = c;
        A.nodes[node].stamp = now;
        if (A.nodes[node].block >= 0 && pos > start_pos) {
            r.matched_tokens = pos - start_pos;
            r.matched_block_ids.push_back(A.nodes[node].block);
        }
    }
    return r;
}

void RadixPrefixCache::insert(const std::vector<int>& tokens, int start_pos,
                              const std::vector<int>& block_ids) {
    Arena& A = *arena_;
    const int n = static_cast<int>(tokens.size());
    const uint64_t now = ++clock_;
    int node = 0, pos = 0;
    // Position the cursor at start_pos by walking from the root; any failure
    // restarts from the root at start_pos.
    while (pos < start_pos) {
        int c = pos < n ? A.find_child(node, tokens[pos]) : -1;
        if (c < 0) { node = 0; pos = start_pos; break; }
        const int seg_len = static_cast<int>(A.nodes[c].seg.size());
        const int lim = std::min(seg_len, start_pos - pos);
        if (pos + lim > n) { node = 0; pos = start_pos; break; }
        const int k = common_prefix(tokens, pos, A.nodes[c].seg, lim);
        if (k < lim) { node = 0; pos = start_pos; break; }
        pos += k;
        node = c;
        A.nodes[c].stamp = now;
        if (k < seg_len) { node = 0; pos = start_pos; break; }
    }

    for (int id : block_ids) {
        int remaining = block_size_;
        if (pos < 0 || pos + remaining > n) return;   // block not backed by tokens
        while (remaining > 0) {
            const int first = tokens[pos];
            const int c = A.find_child(node, first);
            int k = 0;
            if (c >= 0) {
                const int seg_len = static_cast<int>(A.nodes[c].seg.size());
                k = common_prefix(tokens, pos, A.nodes[c].seg, std::min(remaining, seg_len));
            }
            if (c < 0 || k == 0) {
                // New leaf holding the rest of the block.
                const int leaf = A.make();
                A.nodes[leaf].seg.assign(tokens.begin() + pos, tokens.begin() + pos + remaining);
                A.nodes[leaf].block = id;
                A.nodes[leaf].refs = 1;
                A.nodes[leaf].stamp = now;
                A.map_block(id, leaf);
                A.link(node, first, leaf);
                pos += remaining;
                remaining = 0;
                node = leaf;
                break;
            }
            const int seg_len = static_cast<int>(A.nodes[c].seg.size());
            if (k == seg_len) {
                // Whole segment matched: descend.
                pos += k;
                remaining -= k;
                node = c;
                A.nodes[c].stamp = now;
                if (A.nodes[c].block >= 0) {
                    ++A.nodes[c].refs;
                    if (remaining == 0) {
                        A.map_block(id, c);
                        break;
                    }
                }
                continue;
            }
            // Partial match: split c at k.  The new intermediate takes c's
            // prefix and c's children; c keeps the suffix, childless, under it.
            const int mid = A.make();
            Arena::Node& cn = A.nodes[c];
            A.nodes[mid].seg.assign(cn.seg.begin(), cn.seg.begin() + k);
            A.nodes[mid].stamp = cn.stamp;
            A.nodes[mid].kids = std::move(cn.kids);
            cn.kids.clear();
            for (auto& kv : A.nodes[mid].kids) A.nodes[kv.second].parent = mid;
            A.nodes[c].seg.erase(A.nodes[c].seg.begin(), A.nodes[c].seg.begin() + k);
            A.link(mid, A.nodes[c].seg[0], c);   // replaces (frees) a clashing child, as the reference
            if (A.nodes[c].block >= 0) A.map_block(A.nodes[c].block, c);
            pos += k;
            remaining -= k;
            A.nodes[node].kids[first] = mid;
            A.nodes[mid].parent = node;
            node = mid;
            if (remaining == 0) {
                A.nodes[mid].block = id;
                A.nodes[mid].refs = 1;
                A.nodes[mid].stamp = now;
                A.map_block(id, mid);
                break;
            }
        }
    }
}

void RadixPrefixCache::remove(int block_id) {
    const int x = arena_->node_of(block_id);
    if (x >= 0 && arena_->nodes[x].refs > 0) --arena_->nodes[x].refs;
}

void RadixPrefixCache::increment_ref(int block_id) {
    const int x = arena_->node_of(block_id);
    if (x >= 0) ++arena_->nodes[x].refs;
}

int RadixPrefixCache::evict_lru() {
    Arena& A = *arena_;
    int best = -1;
    uint64_t best_stamp = UINT64_MAX;
    // Pre-order walk, children in ascending key order.
    std::vector<int> stack{0};
    while (!stack.empty()) {
        const int x = stack.back();
        stack.pop_back();
        const Arena::Node& nd = A.nodes[x];
        if (nd.block >= 0 && nd.refs == 0 && nd.kids.empty() && nd.stamp < best_stamp) {
            best = x;
            best_stamp = nd.stamp;
        }
        for (auto it = nd.kids.rbegin(); it != nd.kids.rend(); ++it) stack.push_back(it->second);
    }
    if (best < 0) return -1;
    const int block = A.nodes[best].block;
    const int parent = A.nodes[best].parent;
    if (parent < 0) {
        A.nodes[best].block = -1;
        A.nodes[best].refs = 0;
        A.nodes[best].seg.clear();
    } else {
        Arena::Node& p = A.nodes[parent];
        const int key = A.nodes[best].seg.empty() ? 0 : A.nodes[best].seg[0];
        auto it = p.kids.find(key);
        if (it != p.kids.end() && it->second == best) {
            p.kids.erase(it);
            A.release(best);
            if (p.block == -1 && p.kids.size() == 1 && parent != 0) {
                // Merge the valueless parent with its only child.
                const int only = p.kids.begin()->second;
                Arena::Node& ch = A.nodes[only];
                p.seg.insert(p.seg.end(), ch.seg.begin(), ch.seg.end());
                p.block = ch.block;
                p.refs = ch.refs;
                p.stamp = ch.stamp;
                std::map<int, int> grand = std::move(ch.kids);
                ch.kids.clear();
                A.release(only);
                Arena::Node& p2 = A.nodes[parent];
                p2.kids = std::move(grand);
                for (auto& kv : p2.kids) A.nodes[kv.second].parent = parent;
                if (p2.block >= 0) A.map_block(p2.block, parent);
            }
        }
    }
    A.by_block.erase(block);
    return block;
}

size_t RadixPrefixCache::size() const { return arena_->by_block.size(); }

}  // namespace kv_cache
}  // namespace lightllm
