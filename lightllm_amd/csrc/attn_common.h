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
    // Balanced schedule (nwg > 0): nwg work-groups share the batch's pages
    // equally; plan receives the per-sequence page prefix sums [B + 1].
    int nwg;
    int* plan;
    // Fused append (both non-null): the step's new K/V rows [B, Hkv, D].  The
    // new token of sequence b is position len(b) - 1; the work-group whose
    // segment holds it stores the row into the pools (k / v, written through)
    // and reads that token from here instead of the pool.
    const void* knew;
    const void* vnew;
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

// Barrier for LDS hand-offs only: waits for this wave's LDS operations, not
// for its global stores (which __syncthreads would also wait for).
__device__ inline void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);   // no compiler motion of memory operations across
    __builtin_amdgcn_s_waitcnt(0xC07F);        // lgkmcnt(0); vmcnt / expcnt unconstrained
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

constexpr int kDecodeWaves = 4;   // waves per decode work-group
constexpr int kUnitWaves = 16;    // waves per work-group of the unit schedule (one work-group per unit)

constexpr float kNegBig = -1e30f;   // finite "minus infinity" for running maxima

// A segment: pages [pg_begin, pg_begin + npages) of (sequence b, kv head
// kvh), keys below tok_end.  Its result goes straight to the output rows of
// the G query heads (direct) or to fp32 partials: rows part_o + po_off +
// h * po_stride (D floats) and part_lse[pl_off + h * pl_stride], h < G.
// cum = pages of the earlier segments of the same round.
struct SegDesc {
    int b, kvh, pg_begin, npages, cum, tok_end, direct;
    int new_tok;   // fused append: position of the new token if in this segment, else -1
    int64_t po_off, pl_off;
};

// Position of sequence b's new token when a fused append is on, the segment
// [pg_begin, tok_end) holds it and the table has a page for it, else -1 (with
// no page the append writes nothing and the decode reads the pool, as the two
// separate calls would).
__device__ inline int seg_new_tok(const DecodeArgs& a, int b, int pg_begin, int tok_end, int L) {
    if (a.knew == nullptr || L <= 0 || tok_end != L || pg_begin * kPage > L - 1) return -1;
    return a.bt[(int64_t)b * a.max_blocks + (L - 1) / kPage] >= 0 ? L - 1 : -1;
}

// Fused append: store the new K/V row of segment d's (sequence, kv head) into
// its pool slot (skipped when the table has no page there, as llkv_append skips
// a negative slot).  Called by every thread of the work-group.
template <typename T, int D>
__device__ inline void store_new_row(const DecodeArgs& a, const SegDesc& d) {
    if (d.new_tok < 0) return;
    const int phys = a.bt[(int64_t)d.b * a.max_blocks + d.new_tok / kPage];
    if (phys < 0) return;
    const int64_t dst = (((int64_t)phys * kPage + d.new_tok % kPage) * a.Hkv + d.kvh) * D;
    const int64_t src = ((int64_t)d.b * a.Hkv + d.kvh) * D;
    constexpr int U = D * (int)sizeof(T) / 16;   // 16-byte units per head row
    for (int i = threadIdx.x; i < 2 * U; i += blockDim.x) {
        const bool isv = i >= U;
        const int u = isv ? i - U : i;
        const uint4* from = reinterpret_cast<const uint4*>(
                                reinterpret_cast<const T*>(isv ? a.vnew : a.knew) + src) + u;
        uint4* to = reinterpret_cast<uint4*>(
                        const_cast<T*>(reinterpret_cast<const T*>(isv ? a.v : a.k)) + dst) + u;
        *to = *from;
    }
}

// ---------------------------------------------------------------------------
// Balanced schedule.  Page-units are (sequence b, kv head) pairs in the order
// u = b * Hkv + kvh; unit u holds npages(b) pages and the batch holds
// T = Hkv * sum_b npages(b) page-units.  Work-group w of nwg takes positions
// [floor(w T / nwg), floor((w + 1) T / nwg)), cut at unit boundaries into
// segments.  The segment of (w, u) has id w + u: along increasing positions
// both w and u never decrease and at least one grows at each cut, so ids are
// unique and below nwg + B * Hkv.  A unit inside one work-group is written
// directly; otherwise its segments' partials are merged afterwards.
// ---------------------------------------------------------------------------
constexpr int kBalanceMaxB = 1024;    // sequences (prefix sums staged in LDS)
constexpr int kBalanceMaxWG = 2048;   // work-groups (bounds the partial storage)

__device__ inline int clamp_len(const DecodeArgs& a, int b) {
    int L = a.lens[b];
    const int cap = a.max_blocks * a.bs;
    return L < 0 ? 0 : (L > cap ? cap : L);
}

__device__ inline int wave_incl_scan(int v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(v, off, 64);
        if (lane >= off) v += t;
    }
    return v;
}

// sP[b] = pages of sequences [0, b), b = 0..B, and sL[b] = clamped length,
// computed by wave 0; ends with a barrier.
__device__ inline void scan_pages(const DecodeArgs& a, int* sP, int* sL) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        int run = 0;
        for (int c0 = 0; c0 < a.B; c0 += 64) {
            const int b = c0 + lane;
            const int L = b < a.B ? clamp_len(a, b) : 0;
            const int np = (L + a.bs - 1) / a.bs;
            const int incl = wave_incl_scan(np);
            if (b < a.B) {
                sP[b + 1] = run + incl;
                sL[b] = L;
            }
            run += __shfl(incl, 63, 64);
        }
        if (lane == 0) sP[0] = 0;
    }
    __syncthreads();
}

// floor(x / y) for 0 <= x < 2^53, 0 < y: a double quotient corrected by
// integer products (64-bit integer division is a long software sequence).
__device__ inline int64_t div_floor(int64_t x, int64_t y) {
    int64_t q = (int64_t)((double)x / (double)y);
    if (q * y > x) --q;
    else if ((q + 1) * y <= x) ++q;
    return q;
}

// First position of work-group w's share: floor(w T / nwg).
__device__ inline int64_t share_begin(int64_t w, int64_t T, int nwg) {
    return div_floor(w * T, nwg);
}

// Work-group holding position p (0 <= p < T): the largest w with
// floor(w T / nwg) <= p.
__device__ inline int64_t wg_of(int64_t p, int64_t T, int nwg) {
    return div_floor((p + 1) * nwg - 1, T);
}

// Every share holds at least one position when T >= nwg.
__device__ inline bool wg_nonempty(int64_t w, int64_t T, int nwg) {
    return T >= nwg || share_begin(w, T, nwg) < share_begin(w + 1, T, nwg);
}

// Segments of work-group wg's positions [p, r1), at most maxseg of them, into
// segs[]; returns the position after the last one.  Partial rows of segment
// id w + u start at row (w + u) * G.
__device__ inline int64_t build_segments(const DecodeArgs& a, const int* sP, const int* sL,
                                         int64_t p, int64_t r1, int64_t wg, int maxseg,
                                         SegDesc* segs, int* nseg) {
    const int G = a.Hq / a.Hkv;
    int lo = 0, hi = a.B;   // Hkv * sP[lo] <= p < Hkv * sP[hi]
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if ((int64_t)a.Hkv * sP[mid] <= p) lo = mid;
        else hi = mid;
    }
    int b = lo;
    int np = sP[b + 1] - sP[b];
    int64_t base = (int64_t)a.Hkv * sP[b];
    const int off = (int)(p - base);   // < Hkv * np
    int kvh = off / np;
    int pg = off - kvh * np;
    int n = 0, cum = 0;
    while (p < r1 && n < maxseg) {
        const int64_t unit_end = base + (int64_t)(kvh + 1) * np;
        const int64_t seg_end = r1 < unit_end ? r1 : unit_end;
        SegDesc& d = segs[n];
        d.b = b;
        d.kvh = kvh;
        d.pg_begin = pg;
        d.npages = (int)(seg_end - p);
        d.cum = cum;
        const int te = (pg + d.npages) * kPage;
        d.tok_end = te < sL[b] ? te : sL[b];
        d.direct = pg == 0 && seg_end == unit_end;
        d.new_tok = seg_new_tok(a, b, pg, d.tok_end, sL[b]);
        const int64_t seg = wg + (int64_t)b * a.Hkv + kvh;
        d.po_off = seg * G * a.D;
        d.pl_off = seg * G;
        cum += d.npages;
        ++n;
        p = seg_end;
        if (p >= r1) break;
        // next non-empty unit
        pg = 0;
        if (++kvh == a.Hkv) {
            kvh = 0;
            do {
                ++b;
            } while (sP[b + 1] == sP[b]);
            np = sP[b + 1] - sP[b];
        }
        base = (int64_t)a.Hkv * sP[b];
    }
    *nseg = n;
    return p;
}

// Optional per-work-group timeline for experiments: a build may define
// LLKV_TRACE_POINT(k) to record a timestamp at point k; by default it compiles
// to nothing.
#ifndef LLKV_TRACE_POINT
#define LLKV_TRACE_POINT(k)
#endif

}  // namespace llkv
