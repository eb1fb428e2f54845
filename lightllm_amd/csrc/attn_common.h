// Shared definitions of the paged attention kernels (decode, split merge,
// generic row kernel used for odd shapes / fp32 prefill / first prefill).
#pragma once

#include "common.h"

namespace llkv {

// Arguments of the decode kernels.  Partials: part_o [B, Hq, S_max, D] fp32
// holding the normalised split output, part_lse [B, Hq, S_max] holding the
// split's log2-sum-exp2 (in the base-2 domain of the scaled scores).
struct DecodeArgs {
    void* out;
    const void* q;
    const void* k;
    const void* v;
    const int* bt;
    const int* lens;
    float* part_o;
    float* part_lse;
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

// Optional per-work-group timeline for experiments: a build may define
// LLKV_TRACE_POINT(k) to record a timestamp at point k; by default it compiles
// to nothing.
#ifndef LLKV_TRACE_POINT
#define LLKV_TRACE_POINT(k)
#endif

}  // namespace llkv
