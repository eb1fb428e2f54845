// Shared definitions of the paged attention kernels (decode, split merge,
// generic row kernel used for odd shapes / fp32 prefill / first prefill).
#pragma once

#include "common.h"

namespace llkv {

// Arguments of the decode kernels.  Partials: part_o [B, Hq, S_max, D] fp32
// holding the normalised split output, part_lse [B, Hq, S_max] holding the
// split's log2-sum-exp2 (in the base-2 domain of the scaled scores);
// counters [B, Hq] int32 count finished splits (zero between calls: the split
// that completes a head group merges the partials and resets its counter).
struct DecodeArgs {
    void* out;
    const void* q;
    const void* k;
    const void* v;
    const int* bt;
    const int* lens;
    float* part_o;
    float* part_lse;
    int* counters;
    int B, Hq, Hkv, D, bs, max_blocks;
    int S_max;      // splits allocated per (seq, head)
    int pps_auto;   // pages per split in automatic mode
    int fixed_S;    // > 0: reference split rule (S ranges of ceil(n/S) pages)
    float scale_log2;
};

// Split geometry of one sequence; identical in the split and merge kernels.
struct SplitGeo {
    int L;        // keys attended (clamped to the table's capacity)
    int npages;
    int pps;      // pages per split
    int nsplit;   // non-empty splits
};

__device__ inline SplitGeo split_geo(const DecodeArgs& a, int b) {
    SplitGeo g;
    int L = a.lens[b];
    int cap = a.max_blocks * a.bs;
    L = L < 0 ? 0 : (L > cap ? cap : L);
    g.L = L;
    g.npages = (L + a.bs - 1) / a.bs;
    if (a.fixed_S > 0)
        g.pps = (g.npages + a.fixed_S - 1) / a.fixed_S;
    else
        g.pps = a.pps_auto;
    if (g.pps < 1) g.pps = 1;
    g.nsplit = (g.npages + g.pps - 1) / g.pps;
    if (g.nsplit > a.S_max) {   // caller's max_seq_len hint was too small
        g.pps = (g.npages + a.S_max - 1) / a.S_max;
        g.nsplit = (g.npages + g.pps - 1) / g.pps;
    }
    return g;
}

constexpr float kNegBig = -1e30f;   // finite "minus infinity" for running maxima

// Split completion: called by every lane of the wave after it stored its
// partial.  Returns true in exactly one wave per counter -- the last split to
// finish -- after making the other splits' partials visible to it.  Release /
// acquire are at agent scope, so partials written through another XCD's L2
// are written back before the count and re-read from memory after it.
__device__ inline bool split_arrive_last(int* counter, int nsplit) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    int prev = 0;
    if (threadIdx.x == 0)
        prev = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = __shfl(prev, 0, 64);
    if (prev != nsplit - 1) return false;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    return true;
}

// Merge of the nsplit partials of `heads` consecutive q heads starting at
// (b, hq0) into `out` (the reference's paged_attention_reduce_kernel,
// src/kv_cache/paged_attention.cu:477-532, in normalised form:
// out = sum_s 2^(lse_s - M) o_s / sum_s 2^(lse_s - M)).  One wave; lanes own
// output dims.  Resets the counter for the next call.
template <typename T>
__device__ inline void split_merge(const DecodeArgs& a, int b, int hq0, int heads, int nsplit,
                                   int* counter) {
    const int lane = threadIdx.x;
    for (int g = 0; g < heads; ++g) {
        const int64_t bh = (int64_t)b * a.Hq + hq0 + g;
        const float* lse = a.part_lse + bh * a.S_max;
        const float* po = a.part_o + bh * a.S_max * a.D;
        float M = -INFINITY;
        for (int s = 0; s < nsplit; ++s) M = fmaxf(M, lse[s]);
        float wsum = 0.0f;
        for (int s = 0; s < nsplit; ++s) wsum += fast_exp2(lse[s] - M);
        const float inv = 1.0f / wsum;
        T* out = reinterpret_cast<T*>(a.out) + bh * a.D;
        for (int d = lane; d < a.D; d += 64) {
            float o = 0.0f;
            for (int s = 0; s < nsplit; ++s)
                o = fmaf(fast_exp2(lse[s] - M),
                         po[(int64_t)s * a.D + d], o);
            out[d] = Elem<T>::from_f32(o * inv);
        }
    }
    if (lane == 0) *counter = 0;
}

}  // namespace llkv
