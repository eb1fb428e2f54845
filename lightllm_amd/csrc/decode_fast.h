// Fast paged decode kernel for gfx950 (16-token pages, head_dim 64 / 128,
// group sizes 1, 2, 4, 7, 8; fp32 / fp16 / bf16).  Included by decode.hip.
//
// Work-group = 4 waves for one (chunk of pages, kv_head, sequence):
//  * every wave computes all G = Hq/Hkv query heads of the KV head, so each
//    K/V byte is read from HBM once (the reference launches one block per
//    query head and re-reads K/V G times, src/kv_cache/paged_attention.cu:580);
//  * the 4 waves take interleaved tiles of the chunk (equal work), each with a
//    two-deep software pipeline of 16-byte global_load_dwordx4 loads;
//  * a token's row is spread over LPT = D/8 lanes (8 dims per lane); the dot
//    products finish with DPP row reductions; every token group of a wave
//    keeps its own running (max, sum, acc) until the end of the chunk;
//  * the groups of a wave merge with shuffles, the 4 waves through LDS, and
//    the chunks of a sequence through the split-merge kernel (decode.hip).
#pragma once

#include "attn_common.h"

namespace llkv {

constexpr int kDecodeWaves = 4;

template <typename T, int D, int G>
struct FastCfg {
    static constexpr int VEC = Chunk<T>::VEC;          // elements per 16 B
    static constexpr int NJ = sizeof(T) == 4 ? 2 : 1;   // 16 B chunks per lane
    static constexpr int DPL = NJ * VEC;                // dims per lane (8)
    static constexpr int LPT = D / DPL;                 // lanes per token
    static constexpr int TPS = 64 / LPT;                // tokens per step
    static constexpr int U = 4 / NJ;                    // steps per tile (two tiles in flight)
    static constexpr int TILE = U * TPS;
    static constexpr int MD = (D + 63) / 64;            // output dims per lane in the merges
    static_assert(D % DPL == 0, "head_dim must be a multiple of 8");
    static_assert(TPS >= 1 && TPS <= 16 && 16 % TPS == 0, "step must stay inside a page");
};

template <typename T, int D, int G>
__global__ __launch_bounds__(64 * kDecodeWaves) void decode_fast_kernel(DecodeArgs a) {
    using C = FastCfg<T, D, G>;
    constexpr int VEC = C::VEC, NJ = C::NJ, DPL = C::DPL, LPT = C::LPT;
    constexpr int TPS = C::TPS, U = C::U, TILE = C::TILE, MD = C::MD;
    constexpr int W = kDecodeWaves;
    __shared__ float s_acc[W][G][D];
    __shared__ float s_ml[W][G][2];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const SplitGeo geo = split_geo(a, b);
    const int hq0 = kvh * G;
    T* out = reinterpret_cast<T*>(a.out);

    if (geo.npages == 0) {   // empty sequence: zeros, as the reference (:224-227)
        if (split == 0)
            for (int i = tid; i < G * D; i += 64 * W)
                out[((int64_t)b * a.Hq + hq0) * D + i] = Elem<T>::from_f32(0.0f);
        return;
    }
    if (split >= geo.nsplit) return;

    const int tok_begin = split * geo.pps * kPage;
    const int tok_end = min(tok_begin + geo.pps * kPage, geo.L);
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

    // Wave w owns tiles w, w+W, w+2W, ... of the chunk.  Two register
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
                    *reinterpret_cast<float4*>(&s_acc[w][g][(j * LPT + part) * VEC + e4]) =
                        make_float4(acc[g][j * VEC + e4], acc[g][j * VEC + e4 + 1],
                                    acc[g][j * VEC + e4 + 2], acc[g][j * VEC + e4 + 3]);
            if (part == 0) {
                s_ml[w][g][0] = m[g];
                s_ml[w][g][1] = l[g];
            }
        }
    }
    __syncthreads();
    if (w != 0) return;

    const bool direct = geo.nsplit == 1;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float M = s_ml[0][g][0];
#pragma unroll
        for (int ww = 1; ww < W; ++ww) M = fmaxf(M, s_ml[ww][g][0]);
        float f[W], L = 0.0f;
#pragma unroll
        for (int ww = 0; ww < W; ++ww) {
            f[ww] = fast_exp2(s_ml[ww][g][0] - M);
            L = fmaf(f[ww], s_ml[ww][g][1], L);
        }
        const float inv = 1.0f / L;
        const int64_t bh = (int64_t)b * a.Hq + hq0 + g;
#pragma unroll
        for (int i = 0; i < MD; ++i) {
            const int d = lane + 64 * i;
            if (d >= D) continue;
            float o = 0.0f;
#pragma unroll
            for (int ww = 0; ww < W; ++ww) o = fmaf(f[ww], s_acc[ww][g][d], o);
            o *= inv;
            if (direct) out[bh * D + d] = Elem<T>::from_f32(o);
            else a.part_o[(bh * a.S_max + split) * D + d] = o;
        }
        if (!direct && lane == 0) a.part_lse[bh * a.S_max + split] = M + fast_log2(L);
    }
}

}  // namespace llkv
