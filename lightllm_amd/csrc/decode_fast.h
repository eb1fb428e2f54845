// VALU paged decode body for gfx950 (16-token pages, head_dim 64 / 128,
// group sizes 1, 2, 4, 7, 8; fp16 / bf16, also usable for fp32).  Included by
// decode.hip, which instantiates it under the fixed-split and the balanced
// schedules.
//
// A segment (token range of one (sequence, kv head)) runs on a work-group of
// 4 waves:
//  * every wave computes all G = Hq/Hkv query heads of the KV head, so each
//    K/V byte is read from HBM once (the reference launches one block per
//    query head and re-reads K/V G times, src/kv_cache/paged_attention.cu:580);
//  * the 4 waves take interleaved tiles of the segment, each with a two-deep
//    software pipeline of 16-byte global_load_dwordx4 loads;
//  * a token's row is spread over LPT = D/8 lanes (8 dims per lane); the dot
//    products finish with DPP row reductions; every token group of a wave
//    keeps its own running (max, sum, acc) until the end of the segment;
//  * the groups of a wave merge with shuffles and the 4 waves through LDS.
#pragma once

#include "attn_common.h"

namespace llkv {

constexpr int kDecodeWaves = 4;

// Where a segment's result goes: straight to the output rows of its G query
// heads (direct), or to fp32 partials (po: G rows of D, row stride po_stride;
// pl: G log2-sum-exp2 values, stride pl_stride).
struct SegOut {
    bool direct;
    float* po;
    int64_t po_stride;
    float* pl;
    int64_t pl_stride;
};

template <typename TT, int D, int G>
struct FastDecode {
    using T = TT;
    static constexpr int VEC = Chunk<T>::VEC;          // elements per 16 B
    static constexpr int NJ = sizeof(T) == 4 ? 2 : 1;   // 16 B chunks per lane
    static constexpr int DPL = NJ * VEC;                // dims per lane (8)
    static constexpr int LPT = D / DPL;                 // lanes per token
    static constexpr int TPS = 64 / LPT;                // tokens per step
    static constexpr int U = 4 / NJ;                    // steps per tile (two tiles in flight)
    static constexpr int TILE = U * TPS;
    static constexpr int MD = (D + 63) / 64;            // output dims per lane in the merges
    static constexpr int W = kDecodeWaves;
    static constexpr int GQ = G, HD = D;
    static constexpr int kWavesPerEU = 1;
    static constexpr int kSegMax = 1;   // segments of a round run one after another
    static_assert(D % DPL == 0, "head_dim must be a multiple of 8");
    static_assert(TPS >= 1 && TPS <= 16 && 16 % TPS == 0, "step must stay inside a page");

    struct Smem {
        float acc[W][G][D];
        float ml[W][G][2];
    };

    // Tokens [tok_begin, tok_end) of (b, kvh), 0 <= tok_begin < tok_end.
    // Ends with a barrier, so the caller may run another segment.
    __device__ static void segment(const DecodeArgs& a, Smem& sm, int b, int kvh, int tok_begin,
                                   int tok_end, const SegOut& so) {
        const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
        const int hq0 = kvh * G;
        const int last_page = (tok_end - 1) >> 4;
        const int grp = lane / LPT, part = lane % LPT;

        // Query rows of the G heads, pre-scaled into the exp2 domain.
        float qf[G][DPL];
        const T* qb = reinterpret_cast<const T*>(a.q) + ((int64_t)b * a.Hq + hq0) * D;
#pragma unroll
        for (int g = 0; g < G; ++g) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                uint4 c = *reinterpret_cast<const uint4*>(qb + g * D + (j * LPT + part) * VEC);
                Chunk<T>::unpack(c, &qf[g][j * VEC]);
            }
#pragma unroll
            for (int e = 0; e < DPL; ++e) qf[g][e] *= a.scale_log2;
        }

        float m[G], l[G], acc[G][DPL];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            m[g] = kNegBig;
            l[g] = 0.0f;
#pragma unroll
            for (int e = 0; e < DPL; ++e) acc[g][e] = 0.0f;
        }

        const int64_t row_elems = (int64_t)a.Hkv * D;
        const T* kbase = reinterpret_cast<const T*>(a.k) + kvh * D + part * VEC;
        const T* vbase = reinterpret_cast<const T*>(a.v) + kvh * D + part * VEC;
        const int* bt = a.bt + (int64_t)b * a.max_blocks;

        // Page ids, 64 at a time, one per lane; steps read them with v_readlane,
        // so no K/V load waits behind a block-table load.
        const int first = tok_begin + w * TILE;   // this wave's first tile
        int tbl_base = min(first, tok_end - 1) >> 4;
        int tbl = bt[min(tbl_base + lane, last_page)];
        constexpr int TILE_PAGES = (TILE + 15) / 16;

        auto load_tile = [&](int t0, uint4 (&kr)[U][NJ], uint4 (&vr)[U][NJ]) {
            if ((t0 >> 4) + TILE_PAGES > tbl_base + 64) {   // uniform; at most every 64 pages
                tbl_base = t0 >> 4;
                tbl = bt[min(tbl_base + lane, last_page)];
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int ts = t0 + u * TPS;                  // first token of the step (uniform)
                const int page = min(ts >> 4, last_page);     // steps past the end re-read a valid page
                const int64_t phys = max(__builtin_amdgcn_readlane(tbl, page - tbl_base), 0);
                const int64_t row = phys * kPage + (ts & 15) + grp;
                const T* kp = kbase + row * row_elems;
                const T* vp = vbase + row * row_elems;
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    kr[u][j] = *reinterpret_cast<const uint4*>(kp + j * LPT * VEC);
                    vr[u][j] = *reinterpret_cast<const uint4*>(vp + j * LPT * VEC);
                }
            }
        };

        auto compute_tile = [&](int t0, const uint4 (&kr)[U][NJ], const uint4 (&vr)[U][NJ]) {
            float s[U][G];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                float kf[DPL];
#pragma unroll
                for (int j = 0; j < NJ; ++j) Chunk<T>::unpack(kr[u][j], &kf[j * VEC]);
                const bool valid = (t0 + u * TPS + grp) < tok_end;
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    float d = 0.0f;
#pragma unroll
                    for (int e = 0; e < DPL; ++e) d = fmaf(qf[g][e], kf[e], d);
                    d = group_sum<LPT>(d);
                    s[u][g] = valid ? d : -INFINITY;
                }
            }
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float mx = m[g];
#pragma unroll
                for (int u = 0; u < U; ++u) mx = fmaxf(mx, s[u][g]);
                const float corr = fast_exp2(m[g] - mx);
                m[g] = mx;
                l[g] *= corr;
#pragma unroll
                for (int e = 0; e < DPL; ++e) acc[g][e] *= corr;
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                float vf[DPL];
#pragma unroll
                for (int j = 0; j < NJ; ++j) Chunk<T>::unpack(vr[u][j], &vf[j * VEC]);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float p = fast_exp2(s[u][g] - m[g]);
                    l[g] += p;
#pragma unroll
                    for (int e = 0; e < DPL; ++e) acc[g][e] = fmaf(p, vf[e], acc[g][e]);
                }
            }
        };

        // Wave w owns tiles w, w+W, w+2W, ... of the segment.  Two register
        // buffers: tile i+1's loads are in flight while tile i is computed;
        // sched_barrier keeps the scheduler from sinking the prefetch.
        constexpr int STRIDE = W * TILE;
        uint4 ka[U][NJ], va[U][NJ], kb[U][NJ], vb[U][NJ];
        if (first < tok_end) load_tile(first, ka, va);
        for (int t0 = first; t0 < tok_end; t0 += 2 * STRIDE) {
            const int t1 = t0 + STRIDE;
            if (t1 < tok_end) load_tile(t1, kb, vb);
            __builtin_amdgcn_sched_barrier(0);
            compute_tile(t0, ka, va);
            if (t1 >= tok_end) break;
            if (t1 + STRIDE < tok_end) load_tile(t1 + STRIDE, ka, va);
            __builtin_amdgcn_sched_barrier(0);
            compute_tile(t1, kb, vb);
        }

        // Token groups of the wave (lanes with equal `part`) merge by shuffles.
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float M = m[g];
#pragma unroll
            for (int off = LPT; off < 64; off <<= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
            const float f = fast_exp2(m[g] - M);
            l[g] *= f;
#pragma unroll
            for (int e = 0; e < DPL; ++e) acc[g][e] *= f;
#pragma unroll
            for (int off = LPT; off < 64; off <<= 1) {
                l[g] += __shfl_xor(l[g], off, 64);
#pragma unroll
                for (int e = 0; e < DPL; ++e) acc[g][e] += __shfl_xor(acc[g][e], off, 64);
            }
            m[g] = M;
        }

        // The 4 waves merge through LDS; wave 0 finishes.
        if (grp == 0) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
#pragma unroll
                for (int j = 0; j < NJ; ++j)
#pragma unroll
                    for (int e4 = 0; e4 < VEC; e4 += 4)
                        *reinterpret_cast<float4*>(&sm.acc[w][g][(j * LPT + part) * VEC + e4]) =
                            make_float4(acc[g][j * VEC + e4], acc[g][j * VEC + e4 + 1],
                                        acc[g][j * VEC + e4 + 2], acc[g][j * VEC + e4 + 3]);
                if (part == 0) {
                    sm.ml[w][g][0] = m[g];
                    sm.ml[w][g][1] = l[g];
                }
            }
        }
        __syncthreads();
        {
            T* out = reinterpret_cast<T*>(a.out) + ((int64_t)b * a.Hq + hq0) * D;
            for (int g = w; g < G; g += W) {   // heads spread over the waves
                float M = sm.ml[0][g][0];
#pragma unroll
                for (int ww = 1; ww < W; ++ww) M = fmaxf(M, sm.ml[ww][g][0]);
                float f[W], L = 0.0f;
#pragma unroll
                for (int ww = 0; ww < W; ++ww) {
                    f[ww] = fast_exp2(sm.ml[ww][g][0] - M);
                    L = fmaf(f[ww], sm.ml[ww][g][1], L);
                }
                const float inv = 1.0f / L;
#pragma unroll
                for (int i = 0; i < MD; ++i) {
                    const int d = lane + 64 * i;
                    if (d >= D) continue;
                    float o = 0.0f;
#pragma unroll
                    for (int ww = 0; ww < W; ++ww) o = fmaf(f[ww], sm.acc[ww][g][d], o);
                    o *= inv;
                    if (so.direct) out[g * D + d] = Elem<T>::from_f32(o);
                    else so.po[g * so.po_stride + d] = o;
                }
                if (!so.direct && lane == 0) so.pl[g * so.pl_stride] = M + fast_log2(L);
            }
        }
        lds_barrier();   // the partial / output stores need not complete here
    }

    __device__ static void round(const DecodeArgs& a, Smem& sm, const SegDesc* segs, int nseg,
                                 int64_t po_stride, int64_t pl_stride) {
        for (int s = 0; s < nseg; ++s) {
            const SegDesc d = segs[s];
            SegOut so;
            so.direct = d.direct != 0;
            so.po = a.part_o + d.po_off;
            so.po_stride = po_stride;
            so.pl = a.part_lse + d.pl_off;
            so.pl_stride = pl_stride;
            segment(a, sm, d.b, d.kvh, d.pg_begin * kPage, d.tok_end, so);
        }
    }
};

}  // namespace llkv
