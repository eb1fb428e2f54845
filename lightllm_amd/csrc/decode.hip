// Paged decode attention for gfx950 (one new query token per sequence).
//
// Replaces the reference's decode kernels (src/kv_cache/paged_attention.cu:
// baseline :104-170, v2 :186-310, Split-K :324-460, reduce :477-532) and the
// host dispatcher (:537-626).  Math is the same online softmax; the mapping
// to the hardware is new:
//
//  * A work-group of 4 waves runs a segment: a page range of one (sequence,
//    kv head).  All G = Hq/Hkv query heads of the kv head are computed
//    together, so every K/V byte is read from HBM once (the reference
//    launches one block per query head and re-reads K/V G times).
//  * Scores and the weighted V sum are two small matrix products per page on
//    the MFMA units (decode_mfma.h), with K/V loaded straight into the
//    operand registers (16-byte K loads, 8- or 16-byte V loads); the 4 waves
//    take interleaved pages and merge their softmax states through LDS.
//  * Schedules.  Fixed split (num_splits = S > 0): the reference's S ranges
//    of ceil(n/S) pages per sequence, one work-group per (split, kv head,
//    sequence).  Automatic (num_splits = 0): fixed splits sized from the
//    resident work-group count when the batch has few (sequence, kv head)
//    units, else the balanced schedule -- as many work-groups as the GPU
//    holds at once, each taking an equal share of the batch's pages whatever
//    the length mix (attn_common.h).  Partials are merged by log-sum-exp in a
//    small second kernel; a unit computed by one work-group writes its
//    output directly.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <map>
#include <mutex>
#include <utility>

#include "attn_common.h"
#include "decode_kernels.h"

namespace llkv {
namespace {

// Generic decode kernel: any head_dim <= 256, any group size, any page size.
// One wave per (split, q_head, sequence); 64 keys per iteration, one key per
// lane (dot product over D from an LDS copy of q), then p broadcast through
// LDS for the V pass where lanes own output dims.
template <typename T>
__global__ __launch_bounds__(64) void decode_generic_kernel(DecodeArgs a) {
    __shared__ float q_s[256];
    __shared__ float p_s[64];
    __shared__ int64_t row_s[64];
    const int lane = threadIdx.x;
    const int split = blockIdx.x, hq = blockIdx.y, b = blockIdx.z;
    const int D = a.D;
    const int G = a.Hq / a.Hkv;
    const int kvh = hq / G;
    const SplitGeo geo = split_geo(a, b);
    T* out = reinterpret_cast<T*>(a.out);
    const int64_t bh = (int64_t)b * a.Hq + hq;
    if (geo.npages == 0) {
        if (split == 0)
            for (int d = lane; d < D; d += 64) out[bh * D + d] = Elem<T>::from_f32(0.0f);
        return;
    }
    if (split >= geo.nsplit) return;
    const int tok_begin = split * geo.pps * a.bs;
    const int tok_end = min(tok_begin + geo.pps * a.bs, geo.L);

    const T* qp = reinterpret_cast<const T*>(a.q) + bh * D;
    for (int d = lane; d < D; d += 64) q_s[d] = Elem<T>::to_f32(qp[d]) * a.scale_log2;
    __syncthreads();

    const T* kp = reinterpret_cast<const T*>(a.k);
    const T* vp = reinterpret_cast<const T*>(a.v);
    const int64_t row_elems = (int64_t)a.Hkv * D;
    const int* bt = a.bt + (int64_t)b * a.max_blocks;
    float m = kNegBig, l = 0.0f, acc[4] = {0.f, 0.f, 0.f, 0.f};

    for (int t0 = tok_begin; t0 < tok_end; t0 += 64) {
        const int t = t0 + lane;
        const bool valid = t < tok_end;
        int64_t row = 0;
        float s = -INFINITY;
        if (valid) {
            row = ((int64_t)max(bt[t / a.bs], 0) * a.bs + t % a.bs) * row_elems + (int64_t)kvh * D;
            // four interleaved running sums, added pairwise: a quarter of the
            // rounding steps of one sum over D terms
            float d0 = 0.0f, d1 = 0.0f, d2 = 0.0f, d3 = 0.0f;
            int d = 0;
            for (; d + 3 < D; d += 4) {
                d0 = fmaf(q_s[d], Elem<T>::to_f32(kp[row + d]), d0);
                d1 = fmaf(q_s[d + 1], Elem<T>::to_f32(kp[row + d + 1]), d1);
                d2 = fmaf(q_s[d + 2], Elem<T>::to_f32(kp[row + d + 2]), d2);
                d3 = fmaf(q_s[d + 3], Elem<T>::to_f32(kp[row + d + 3]), d3);
            }
            for (; d < D; ++d) d0 = fmaf(q_s[d], Elem<T>::to_f32(kp[row + d]), d0);
            s = (d0 + d1) + (d2 + d3);
        }
        const float mx = fmaxf(m, wave_max(s));
        const float corr = fast_exp2(m - mx);
        const float p = valid ? fast_exp2(s - mx) : 0.0f;
        l = l * corr + wave_sum(p);
        m = mx;
        p_s[lane] = p;
        row_s[lane] = row;
        __syncthreads();
        const int n = min(64, tok_end - t0);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] *= corr;
        for (int j = 0; j < n; ++j) {
            const float pj = p_s[j];
            const int64_t rj = row_s[j];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = lane + 64 * i;
                if (d < D) acc[i] = fmaf(pj, Elem<T>::to_f32(vp[rj + d]), acc[i]);
            }
        }
        __syncthreads();
    }

    const float inv = 1.0f / l;
    if (geo.nsplit == 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = lane + 64 * i;
            if (d < D) out[bh * D + d] = Elem<T>::from_f32(acc[i] * inv);
        }
        return;
    }
    float* pp = a.part_o + (bh * a.S_max + split) * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = lane + 64 * i;
        if (d < D) pp[d] = acc[i] * inv;
    }
    if (lane == 0) a.part_lse[bh * a.S_max + split] = m + fast_log2(l);
}

// Log-sum-exp merge of `count` partials of one (sequence, q head): entry j
// is the normalised row po + j * po_step (D floats) with log2-sum-exp2
// pl[j * pl_step]; live(j) false skips an entry.  One wave; lane owns dims
// lane + 64 i; entries are fetched kMergeBatch at a time with a running
// maximum, so a merge costs ceil(count / kMergeBatch) memory round trips.
// The reference's paged_attention_reduce_kernel
// (src/kv_cache/paged_attention.cu:477-532) computes the same sum in
// unnormalised form: out = sum_j 2^(lse_j - M) o_j / sum_j 2^(lse_j - M).
constexpr int kMergeBatch = 16;

template <typename T, int MD, class Live>
__device__ inline void merge_partials(const float* po, int64_t po_step, const float* pl,
                                      int64_t pl_step, int count, int D, Live live, T* out) {
    const int lane = threadIdx.x & 63;
    float M = -INFINITY, W = 0.0f, o[MD];
#pragma unroll
    for (int i = 0; i < MD; ++i) o[i] = 0.0f;
    for (int j0 = 0; j0 < count; j0 += kMergeBatch) {
        float lv[kMergeBatch], pv[kMergeBatch][MD];
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j) {
            const bool ok = j0 + j < count && live(j0 + j);
            const int64_t jj = j0 + j;
            lv[j] = ok ? pl[jj * pl_step] : -INFINITY;
#pragma unroll
            for (int i = 0; i < MD; ++i)
                pv[j][i] = ok ? po[jj * po_step + min(lane + 64 * i, D - 1)] : 0.0f;
        }
        float mb = -INFINITY;
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j) mb = fmaxf(mb, lv[j]);
        const float Mn = fmaxf(M, mb);
        if (Mn == -INFINITY) continue;
        const float sc = fast_exp2(M - Mn);
        W *= sc;
#pragma unroll
        for (int i = 0; i < MD; ++i) o[i] *= sc;
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j) {
            const float w = fast_exp2(lv[j] - Mn);
            W += w;
#pragma unroll
            for (int i = 0; i < MD; ++i) o[i] = fmaf(w, pv[j][i], o[i]);
        }
        M = Mn;
    }
    const float inv = 1.0f / W;
#pragma unroll
    for (int i = 0; i < MD; ++i)
        if (lane + 64 * i < D) out[lane + 64 * i] = Elem<T>::from_f32(o[i] * inv);
}

struct AllLive {
    __device__ bool operator()(int) const { return true; }
};

// Merge of the fixed split schedule: grid (Hq, B), one wave each.
template <typename T, int MD>
__global__ __launch_bounds__(64) void decode_merge_kernel(DecodeArgs a) {
    const int hq = blockIdx.x, b = blockIdx.y;
    const SplitGeo geo = split_geo(a, b);
    if (geo.nsplit <= 1) return;   // written directly by the split kernel
    const int64_t bh = (int64_t)b * a.Hq + hq;
    merge_partials<T, MD>(a.part_o + bh * a.S_max * a.D, a.D, a.part_lse + bh * a.S_max, 1,
                          geo.nsplit, a.D, AllLive(), reinterpret_cast<T*>(a.out) + bh * a.D);
}

// Work-groups of the balanced schedule that hold pages (a work-group's share
// is empty when the batch has fewer page-units than work-groups).
struct LiveWG {
    int64_t w0, T;
    int nwg;
    __device__ bool operator()(int j) const { return wg_nonempty(w0 + j, T, nwg); }
};

// Merge of the balanced schedule.  Unit
// (b, kvh) spans positions [s, e); its segments are those of work-groups
// wg_of(s) .. wg_of(e - 1), with ids w + u.
// Grid (Hkv, B), one wave per q head of the kv head (G waves): the unit's
// schedule is read once per work-group and units inside one share exit
// together.
template <typename T, int MD>
__global__ __launch_bounds__(1024) void decode_merge_balanced_kernel(DecodeArgs a) {
    const int kvh = blockIdx.x, b = blockIdx.y;
    const int G = a.Hq / a.Hkv;
    const int h = threadIdx.x >> 6, hq = kvh * G + h;
    const int D = a.D;
    const int Pb = a.plan[b];
    const int np = a.plan[b + 1] - Pb;
    if (np == 0) return;   // zeros written by the split kernel
    const int64_t T_ = (int64_t)a.Hkv * a.plan[a.B];
    const int64_t s = (int64_t)a.Hkv * Pb + (int64_t)kvh * np;
    const int64_t wf = wg_of(s, T_, a.nwg), wl = wg_of(s + np - 1, T_, a.nwg);
    if (wf == wl) return;   // written directly
    const int64_t seg0 = wf + (int64_t)b * a.Hkv + kvh;
    T* out = reinterpret_cast<T*>(a.out) + ((int64_t)b * a.Hq + hq) * D;
    const float* po = a.part_o + (seg0 * G + h) * D;
    const float* pl = a.part_lse + seg0 * G + h;
    const int cnt = (int)(wl - wf + 1);
    if (T_ >= a.nwg)   // every work-group holds pages: all entries live
        merge_partials<T, MD>(po, (int64_t)G * D, pl, G, cnt, D, AllLive(), out);
    else
        merge_partials<T, MD>(po, (int64_t)G * D, pl, G, cnt, D, LiveWG{wf, T_, a.nwg}, out);
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------
// The tuned kernels of a pool type, plain or fused-append (decode_tuned_*.hip).
Kernels pick_tuned(int dtype, int D, int G, bool append) {
    if (dtype == LLKV_DTYPE_F32) return tuned_kernels_f32(D, G, append);
    if (dtype == LLKV_DTYPE_F16) return tuned_kernels_f16(D, G, append);
    if (dtype == LLKV_DTYPE_BF16) return tuned_kernels_bf16(D, G, append);
    return Kernels();
}

struct Plan {
    int S_max;
    int pps_auto;
    int fixed_S;
};

// Split size of the fixed schedule when num_splits = 0 but the balanced one
// does not apply (odd shapes, more than kBalanceMaxB sequences): 8 pages per
// split, larger for long contexts so one sequence has at most kMaxAutoSplits
// partials to merge.
constexpr int kAutoPps = 8;
constexpr int kMaxAutoSplits = 64;

Plan make_plan(int bs, int max_seq_len, int num_splits) {
    Plan p;
    int max_pages = (std::max(max_seq_len, 1) + bs - 1) / bs;
    if (num_splits > 0) {
        p.fixed_S = num_splits;
        p.pps_auto = 1;
        p.S_max = std::min(num_splits, max_pages);
    } else {
        p.fixed_S = 0;
        const int pps = std::max(kAutoPps, (max_pages + kMaxAutoSplits - 1) / kMaxAutoSplits);
        p.pps_auto = pps;
        p.S_max = (max_pages + pps - 1) / pps;
    }
    if (p.S_max < 1) p.S_max = 1;
    return p;
}

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Fixed schedule workspace: [lse B*Hq*S_max, 256 B aligned][o B*Hq*S_max*D], fp32.
size_t fixed_workspace(int B, int Hq, int D, const Plan& p) {
    if (p.S_max <= 1) return 0;
    size_t n = (size_t)B * Hq * p.S_max;
    return align256(n * sizeof(float)) + n * D * sizeof(float);
}

// Balanced schedule workspace: [plan int32 B+1][lse E*G][o E*G*D], each part
// 256 B aligned, E = kBalanceMaxWG + B*Hkv segments (the largest id + 1).
struct BalancedWs {
    size_t plan_off, lse_off, o_off, total;
};

BalancedWs balanced_workspace(int B, int Hq, int Hkv, int D) {
    const size_t E = (size_t)kBalanceMaxWG + (size_t)B * Hkv;
    const size_t G = Hq / Hkv;
    BalancedWs w;
    w.plan_off = 0;
    w.lse_off = align256((size_t)(B + 1) * sizeof(int));
    w.o_off = w.lse_off + align256(E * G * sizeof(float));
    w.total = w.o_off + E * G * D * sizeof(float);
    return w;
}

bool balanced_eligible(int B) { return B <= kBalanceMaxB; }

int resident_wgs(DecodeFn fn) {
    return resident_workgroups(reinterpret_cast<const void*>(fn), 64 * kDecodeWaves);
}

// Work-groups of the balanced schedule: one resident set (more only adds a
// second, partly idle round), capped by kBalanceMaxWG and by one page-unit
// per wave.
int balanced_wgs(DecodeFn fn, int64_t page_units_bound) {
    const int cap = std::min(kBalanceMaxWG, resident_wgs(fn));
    const int64_t by_work = std::max<int64_t>(1, (page_units_bound + kDecodeWaves - 1) / kDecodeWaves);
    return (int)std::max<int64_t>(1, std::min<int64_t>(cap, by_work));
}

// Automatic schedule.  With few (sequence, kv head) units against the
// resident work-group count, fixed splits of each unit fill the GPU in one
// pass (S ~ resident / units, or 0.8 x that when the longest sequence gives
// each wave more than kShortChainPages pages), and at most one split per 4
// pages; with many units (a large batch of uneven lengths) the balanced
// schedule shares the pages equally instead.
constexpr int kAutoMaxSplits = 64;
constexpr int kShortChainPages = 4;   // pages per wave up to which a split is latency-bound

struct AutoChoice {
    bool balanced;
    bool wide;    // one split on the kUnitWaves-wave kernel (unit schedule)
    int splits;   // fixed schedule: S
};

// Choice of the automatic schedule, from a sweep of batch size (16 .. 1024),
// context (64 .. 1024 tokens, lengths uniform in [L/2, L]) and two head layouts
// (14/2/64 fp32, 32/8/128 fp16), every shape timed under each schedule:
//  * one split per (sequence, kv head) on 4-wave work-groups, no merge, when
//    every sequence is short (<= kOneSplitShortPages pages), or when there are
//    many units and no sequence is long (the balanced schedule's scan, segment
//    bookkeeping and merge cost more than the page chain it shortens):
//    e.g. 512 x 128 tokens fp32 31.5 -> 13.7 us, 1024 x 64 Llama-3 fp16
//    87 -> 52 us, 256 x 1024 fp32 45 -> 37 us;
//  * the unit schedule (one split on 16-wave work-groups) for a middle range of
//    units with up to 4 pages per wave: 32 x 1024 Llama-3 fp16 30.6 -> 23.4 us,
//    128 x 1024 fp32 24.7 -> 20.9 us;
//  * otherwise the balanced schedule for many units (long or uneven contexts:
//    configuration 5) and fixed splits for few (configurations 1-3).
constexpr int kOneSplitShortPages = 8;
constexpr int kOneSplitMaxPages = 64;
constexpr int kOneSplitMinUnits = 384;        // up to kOneSplitMaxPages pages
constexpr int kOneSplitMinUnitsShort = 256;   // up to 16 pages
constexpr int kUnitMaxChain = 4;              // pages per wave of the unit schedule
constexpr int kUnitMinUnits = 64;             // units per page of a wave's chain

bool unit_schedule(const Kernels& ks, int B, int Hkv, int max_pages) {
    const int64_t units = (int64_t)B * Hkv;
    const int chain = (std::max(1, max_pages) + kUnitWaves - 1) / kUnitWaves;   // pages per wave
    if (ks.unit == nullptr || chain > kUnitMaxChain || units < (int64_t)kUnitMinUnits * chain)
        return false;
    const int cap = resident_workgroups(reinterpret_cast<const void*>(ks.unit), 64 * kUnitWaves);
    return units <= cap;
}

AutoChoice auto_schedule(const Kernels& ks, int B, int Hkv, int max_pages) {
    AutoChoice c{false, false, 0};
    const int64_t units = (int64_t)B * Hkv;
    if (max_pages <= kOneSplitShortPages ||
        (max_pages <= kOneSplitMaxPages && units >= kOneSplitMinUnits) ||
        (max_pages <= 16 && units >= kOneSplitMinUnitsShort)) {
        c.splits = 1;
        return c;
    }
    if (unit_schedule(ks, B, Hkv, max_pages)) {
        c.wide = true;
        c.splits = 1;
        return c;
    }
    const int cap = resident_wgs(ks.split);
    if (ks.balanced != nullptr && balanced_eligible(B) && units * 4 >= cap) {
        c.balanced = true;
        return c;
    }
    // One resident set of work-groups when each wave's chain of pages stays short
    // (latency-bound: every extra work-group adds loads in flight); 0.8 of it when
    // the chains are long (bandwidth-bound: extra work-groups only contend).
    int64_t S = (cap + units - 1) / units;
    if ((int64_t)max_pages > S * kDecodeWaves * kShortChainPages) {
        // Long chains: the 16-wave kernel at its full resident count (one
        // work-group per CU), a quarter as many splits (and partials to merge)
        // for the same waves.  Full rather than 0.8 x (which left a fifth of
        // the CUs idle): configuration 3 55.6 -> 55.2 us, 8 x 32k tokens 29.9 ->
        // 29.0 us, 32/8/128 fp16 4 x 32k 112.6 -> 110.1 us, equal on the other
        // long-chain shapes swept; twice the resident count was slower.
        if (ks.unit != nullptr) {
            const int cap16 = resident_workgroups(reinterpret_cast<const void*>(ks.unit), 64 * kUnitWaves);
            const int64_t S16 = std::min<int64_t>((cap16 + units - 1) / units, kAutoMaxSplits);
            if (S16 > 1 && (int64_t)max_pages > S16 * kUnitWaves * kShortChainPages) {
                c.wide = true;
                c.splits = (int)S16;
                return c;
            }
        }
        S = (cap * 4 / 5 + units - 1) / units;
    }
    // at least one page per wave of a split (smaller splits only add partials to merge)
    const int64_t by_pages = (std::max(1, max_pages) + kDecodeWaves - 1) / kDecodeWaves;
    S = std::max<int64_t>(1, std::min<int64_t>({S, (int64_t)kAutoMaxSplits, by_pages}));
    c.splits = (int)S;
    return c;
}

template <typename T, int MD>
void launch_merge_md(bool balanced, dim3 grid, hipStream_t st, const DecodeArgs& a) {
    if (balanced)
        decode_merge_balanced_kernel<T, MD><<<dim3(a.Hkv, a.B), 64 * (a.Hq / a.Hkv), 0, st>>>(a);
    else decode_merge_kernel<T, MD><<<grid, 64, 0, st>>>(a);
}

template <typename T>
void launch_merge(bool balanced, int D, dim3 grid, hipStream_t st, const DecodeArgs& a) {
    if (D <= 64) launch_merge_md<T, 1>(balanced, grid, st, a);
    else if (D <= 128) launch_merge_md<T, 2>(balanced, grid, st, a);
    else launch_merge_md<T, 4>(balanced, grid, st, a);
}

}  // namespace
}  // namespace llkv

using namespace llkv;

extern "C" size_t llkv_paged_decode_workspace_size(int num_seqs, int num_q_heads,
                                                   int num_kv_heads, int head_dim,
                                                   int block_size, int max_seq_len,
                                                   int num_splits) {
    if (num_seqs <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 ||
        block_size <= 0 || num_q_heads % num_kv_heads != 0)
        return 0;
    Plan p = make_plan(block_size, max_seq_len, num_splits);
    size_t need = fixed_workspace(num_seqs, num_q_heads, head_dim, p);
    if (num_splits == 0) {
        // the automatic choice may be any fixed split up to kAutoMaxSplits, or balanced
        const int max_pages = (std::max(max_seq_len, 1) + block_size - 1) / block_size;
        Plan f = make_plan(block_size, max_seq_len, std::min(kAutoMaxSplits, max_pages));
        need = std::max(need, fixed_workspace(num_seqs, num_q_heads, head_dim, f));
        if (balanced_eligible(num_seqs))
            need = std::max(need, balanced_workspace(num_seqs, num_q_heads, num_kv_heads, head_dim).total);
    }
    return need;
}

namespace llkv {
namespace {

// Fused append on the generic path: the new K/V row of (sequence, kv head) =
// (blockIdx.y, blockIdx.x) goes to position len - 1 before the decode kernel
// runs (any head_dim and page size).
template <typename T>
__global__ __launch_bounds__(64) void append_new_rows_kernel(DecodeArgs a) {
    const int kvh = blockIdx.x, b = blockIdx.y;
    const int L = clamp_len(a, b);
    if (L <= 0) return;
    const int phys = a.bt[(int64_t)b * a.max_blocks + (L - 1) / a.bs];
    if (phys < 0) return;
    const int64_t dst = (((int64_t)phys * a.bs + (L - 1) % a.bs) * a.Hkv + kvh) * a.D;
    const int64_t src = ((int64_t)b * a.Hkv + kvh) * a.D;
    T* kp = const_cast<T*>(reinterpret_cast<const T*>(a.k));
    T* vp = const_cast<T*>(reinterpret_cast<const T*>(a.v));
    for (int d = threadIdx.x; d < a.D; d += blockDim.x) {
        kp[dst + d] = reinterpret_cast<const T*>(a.knew)[src + d];
        vp[dst + d] = reinterpret_cast<const T*>(a.vnew)[src + d];
    }
}

// The schedule of a call: balanced, or fixed splits (num_splits updated to
// the automatic choice) with wide = the 16-wave unit kernel for one split.
void decide_schedule(const Kernels& ks, int num_seqs, int num_kv_heads, int block_size, int max_seq_len,
                     int& num_splits, bool& balanced, bool& wide) {
    const int max_pages_hint = (max_seq_len + block_size - 1) / block_size;
    balanced = false;
    wide = false;
    if (num_splits == 0 && ks.split != nullptr) {
        const AutoChoice c = auto_schedule(ks, num_seqs, num_kv_heads, max_pages_hint);
        balanced = c.balanced;
        wide = c.wide;
        if (!balanced) num_splits = c.splits;
    } else if (num_splits == 1 && ks.split != nullptr) {
        wide = unit_schedule(ks, num_seqs, num_kv_heads, max_pages_hint);
    }
}

int paged_decode_impl(const char* fn, void* out, const void* q, const void* k_new,
                      const void* v_new, const void* k_pool, const void* v_pool,
                      const int* block_table, const int* seq_lens, int num_seqs, int num_q_heads,
                      int num_kv_heads, int head_dim, int block_size, int max_blocks_per_seq,
                      int max_seq_len, int num_splits, float scale, int dtype, void* workspace,
                      size_t workspace_bytes, void* stream) {
    if (num_seqs == 0) return LLKV_OK;
    if (num_seqs < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 ||
        block_size <= 0 || max_blocks_per_seq <= 0 || num_splits < 0)
        return set_error(LLKV_ERR_INVALID, "%s: bad shape arguments", fn);
    if (head_dim > 256)
        return set_error(LLKV_ERR_UNSUPPORTED, "%s: head_dim too large (%d > 256)", fn, head_dim);
    if (num_q_heads % num_kv_heads != 0)
        return set_error(LLKV_ERR_INVALID, "%s: num_q_heads %d not a multiple of num_kv_heads %d",
                         fn, num_q_heads, num_kv_heads);
    if (dtype_bytes(dtype) == 0) return set_error(LLKV_ERR_INVALID, "%s: unsupported dtype %d", fn, dtype);
    if (!out || !q || !k_pool || !v_pool || !block_table || !seq_lens)
        return set_error(LLKV_ERR_INVALID, "%s: null pointer", fn);
    if (max_seq_len < 0) max_seq_len = 0;
    // token positions (max_blocks_per_seq * block_size) are int on the device
    if ((int64_t)num_seqs * max_blocks_per_seq > INT32_MAX ||
        (int64_t)max_blocks_per_seq * block_size > INT32_MAX)
        return set_error(LLKV_ERR_UNSUPPORTED, "%s: block table too large", fn);
    if (max_seq_len > max_blocks_per_seq * block_size) max_seq_len = max_blocks_per_seq * block_size;

    const int G = num_q_heads / num_kv_heads;
    // The tuned bodies need 16-token pages, 16-byte aligned rows and pointers.
    const size_t es = dtype_bytes(dtype);
    const bool aligned = (((uintptr_t)q | (uintptr_t)out | (uintptr_t)k_pool |
                           (uintptr_t)v_pool | (uintptr_t)k_new | (uintptr_t)v_new) & 15) == 0 &&
                         ((size_t)num_kv_heads * head_dim * es) % 16 == 0;
    Kernels ks;
    if (block_size == kPage && aligned) {
        ks = pick_tuned(dtype, head_dim, G, k_new != nullptr);
    }
    const int max_pages_hint = (max_seq_len + block_size - 1) / block_size;
    bool balanced = false, wide = false;
    // The fused-append call takes the plain call's schedule (from the plain
    // kernels' resident counts), so that its results equal append + decode
    // bit for bit.
    const Kernels sched = (k_new != nullptr && ks.split != nullptr) ? pick_tuned(dtype, head_dim, G, false) : ks;
    decide_schedule(sched, num_seqs, num_kv_heads, block_size, max_seq_len, num_splits, balanced, wide);

    DecodeArgs a;
    a.out = out;
    a.q = q;
    a.k = k_pool;
    a.v = v_pool;
    a.bt = block_table;
    a.lens = seq_lens;
    a.B = num_seqs;
    a.Hq = num_q_heads;
    a.Hkv = num_kv_heads;
    a.D = head_dim;
    a.bs = block_size;
    a.max_blocks = max_blocks_per_seq;
    a.scale_log2 = scale * kLog2e;
    a.nwg = 0;
    a.plan = nullptr;
    a.knew = k_new;
    a.vnew = v_new;
    char* ws = reinterpret_cast<char*>(workspace);
    hipStream_t st = (hipStream_t)stream;

    if (balanced) {
        const BalancedWs w = balanced_workspace(num_seqs, num_q_heads, num_kv_heads, head_dim);
        if (workspace == nullptr || workspace_bytes < w.total)
            return set_error(LLKV_ERR_WORKSPACE, "%s: workspace %zu bytes < required %zu", fn,
                             workspace_bytes, w.total);
        a.nwg = balanced_wgs(sched.balanced, (int64_t)num_seqs * num_kv_heads * max_pages_hint);   // as the plain call
        a.plan = reinterpret_cast<int*>(ws + w.plan_off);
        a.part_lse = reinterpret_cast<float*>(ws + w.lse_off);
        a.part_o = reinterpret_cast<float*>(ws + w.o_off);
        a.S_max = 0;
        a.pps_auto = 0;
        a.fixed_S = 0;
        ks.balanced<<<dim3(a.nwg), 64 * kDecodeWaves, 0, st>>>(a);
        if (int e = check_launch(fn)) return e;
    } else {
        Plan p = make_plan(block_size, max_seq_len, num_splits);
        size_t need = fixed_workspace(num_seqs, num_q_heads, head_dim, p);
        if (need > 0 && (workspace == nullptr || workspace_bytes < need))
            return set_error(LLKV_ERR_WORKSPACE, "%s: workspace %zu bytes < required %zu", fn,
                             workspace_bytes, need);
        size_t n = (size_t)num_seqs * num_q_heads * p.S_max;
        a.part_lse = need ? reinterpret_cast<float*>(ws) : nullptr;
        a.part_o = need ? reinterpret_cast<float*>(ws + align256(n * sizeof(float))) : nullptr;
        a.S_max = p.S_max;
        a.pps_auto = p.pps_auto;
        a.fixed_S = p.fixed_S;
        if (ks.split) {
            dim3 grid(p.S_max, num_kv_heads, num_seqs);
            if (wide)   // the 16-wave work-groups (one split, or long chains)
                ks.unit<<<grid, 64 * kUnitWaves, 0, st>>>(a);
            else
                ks.split<<<grid, 64 * kDecodeWaves, 0, st>>>(a);
        } else {
            if (k_new != nullptr) {   // append first, then the plain generic decode
                dim3 agrid(num_kv_heads, num_seqs);
                if (dtype == LLKV_DTYPE_F32) append_new_rows_kernel<float><<<agrid, 64, 0, st>>>(a);
                else if (dtype == LLKV_DTYPE_F16) append_new_rows_kernel<_Float16><<<agrid, 64, 0, st>>>(a);
                else append_new_rows_kernel<bf16_t><<<agrid, 64, 0, st>>>(a);
                a.knew = a.vnew = nullptr;
            }
            dim3 grid(p.S_max, num_q_heads, num_seqs);
            if (dtype == LLKV_DTYPE_F32) decode_generic_kernel<float><<<grid, 64, 0, st>>>(a);
            else if (dtype == LLKV_DTYPE_F16) decode_generic_kernel<_Float16><<<grid, 64, 0, st>>>(a);
            else decode_generic_kernel<bf16_t><<<grid, 64, 0, st>>>(a);
        }
        if (int e = check_launch(fn)) return e;
        if (p.S_max <= 1) return LLKV_OK;
    }
    dim3 grid(num_q_heads, num_seqs);
    if (dtype == LLKV_DTYPE_F32) launch_merge<float>(balanced, head_dim, grid, st, a);
    else if (dtype == LLKV_DTYPE_F16) launch_merge<_Float16>(balanced, head_dim, grid, st, a);
    else launch_merge<bf16_t>(balanced, head_dim, grid, st, a);
    return check_launch(fn);
}

}  // namespace
}  // namespace llkv

extern "C" int llkv_paged_decode(void* out, const void* q, const void* k_pool,
                                 const void* v_pool, const int* block_table,
                                 const int* seq_lens, int num_seqs, int num_q_heads,
                                 int num_kv_heads, int head_dim, int block_size,
                                 int max_blocks_per_seq, int max_seq_len, int num_splits,
                                 float scale, int dtype, void* workspace,
                                 size_t workspace_bytes, void* stream) {
    return paged_decode_impl("llkv_paged_decode", out, q, nullptr, nullptr, k_pool, v_pool,
                             block_table, seq_lens, num_seqs, num_q_heads, num_kv_heads, head_dim,
                             block_size, max_blocks_per_seq, max_seq_len, num_splits, scale, dtype,
                             workspace, workspace_bytes, stream);
}

extern "C" int llkv_paged_decode_schedule(int num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                                          int block_size, int max_seq_len, int num_splits, int dtype,
                                          int with_append, int* kind, int* splits) {
    using namespace llkv;
    const char* fn = "llkv_paged_decode_schedule";
    if (!kind || !splits) return set_error(LLKV_ERR_INVALID, "%s: null pointer", fn);
    if (num_seqs < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
        num_splits < 0 || num_q_heads % num_kv_heads != 0 || dtype_bytes(dtype) == 0)
        return set_error(LLKV_ERR_INVALID, "%s: bad shape arguments", fn);
    if (max_seq_len < 0) max_seq_len = 0;
    Kernels ks;
    const size_t es = dtype_bytes(dtype);
    if (block_size == kPage && ((size_t)num_kv_heads * head_dim * es) % 16 == 0 && head_dim <= 256)
        ks = pick_tuned(dtype, head_dim, num_q_heads / num_kv_heads, false);   // as the fused call
    (void)with_append;
    bool balanced = false, wide = false;
    decide_schedule(ks, num_seqs, num_kv_heads, block_size, max_seq_len, num_splits, balanced, wide);
    if (balanced) {
        *kind = LLKV_SCHED_BALANCED;
        *splits = 0;
        return LLKV_OK;
    }
    const Plan p = make_plan(block_size, max_seq_len, num_splits);
    *splits = p.S_max;
    if (ks.split == nullptr) *kind = LLKV_SCHED_GENERIC;
    else if (wide) *kind = LLKV_SCHED_UNIT;
    else *kind = p.S_max > 1 ? LLKV_SCHED_SPLITS : LLKV_SCHED_ONE_SPLIT;
    return LLKV_OK;
}

extern "C" int llkv_paged_decode_append(void* out, const void* q, const void* k_new,
                                        const void* v_new, void* k_pool, void* v_pool,
                                        const int* block_table, const int* seq_lens, int num_seqs,
                                        int num_q_heads, int num_kv_heads, int head_dim,
                                        int block_size, int max_blocks_per_seq, int max_seq_len,
                                        int num_splits, float scale, int dtype, void* workspace,
                                        size_t workspace_bytes, void* stream) {
    const char* fn = "llkv_paged_decode_append";
    if (num_seqs > 0 && (!k_new || !v_new))
        return set_error(LLKV_ERR_INVALID, "%s: null pointer", fn);
    return paged_decode_impl(fn, out, q, k_new, v_new, k_pool, v_pool, block_table, seq_lens,
                             num_seqs, num_q_heads, num_kv_heads, head_dim, block_size,
                             max_blocks_per_seq, max_seq_len, num_splits, scale, dtype, workspace,
                             workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// Decode without a caller workspace: the split partials go to a file-scope
// device array (kNoAllocScratchBytes per GPU, held until the process ends),
// for callers that cannot allocate.  Its device address is looked up once per
// device (hipGetSymbolAddress) and kept; kernels receive that address, never
// the array's host-side name.  The decode kernels write every partial before
// reading it within a call, so nothing needs clearing; calls that overlap on
// one GPU share the array and race.
// ---------------------------------------------------------------------------
namespace llkv {
namespace {

constexpr size_t kNoAllocScratchBytes = 16u << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

int scratch_address(const char* fn, void** out) {
    static std::mutex mu;
    static void* ptrs[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return set_error(LLKV_ERR_HIP, "%s: no current device", fn);
    std::lock_guard<std::mutex> lock(mu);
    if (ptrs[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr)
            return set_error(LLKV_ERR_HIP, "%s: hipGetSymbolAddress(scratch): %s", fn,
                             hipGetErrorString(e));
        ptrs[dev] = p;
    }
    *out = ptrs[dev];
    return LLKV_OK;
}

}  // namespace
}  // namespace llkv

extern "C" size_t llkv_paged_decode_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int llkv_paged_decode_noalloc(void* out, const void* q, const void* k_pool,
                                         const void* v_pool, const int* block_table,
                                         const int* seq_lens, int num_seqs, int num_q_heads,
                                         int num_kv_heads, int head_dim, int block_size,
                                         int max_blocks_per_seq, int max_seq_len, int num_splits,
                                         float scale, int dtype, void* stream) {
    // (the schedule chosen for this call decides the bytes it needs; a shape
    // beyond the array fails the impl's workspace check with LLKV_ERR_WORKSPACE)
    const char* fn = "llkv_paged_decode_noalloc (16 MiB device scratch array)";
    if (num_seqs == 0) return LLKV_OK;
    void* ws = nullptr;
    if (int e = scratch_address(fn, &ws)) return e;
    return paged_decode_impl(fn, out, q, nullptr, nullptr, k_pool, v_pool, block_table, seq_lens,
                             num_seqs, num_q_heads, num_kv_heads, head_dim, block_size,
                             max_blocks_per_seq, max_seq_len, num_splits, scale, dtype, ws,
                             kNoAllocScratchBytes, stream);
}
