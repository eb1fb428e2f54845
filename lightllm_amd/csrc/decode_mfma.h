// MFMA paged decode body for fp32 K/V on gfx950 (16-token pages, head_dim
// 64 / 128, up to 16 query heads per KV head).  Included by decode.hip, which
// instantiates it under the fixed-split and the balanced schedules.
//
// Per KV head the decode step is two small matrix products:
//     S^T [tokens x G] = K [tokens x D] . Q^T [D x G]
//     O^T [D x G]      = V^T [D x tokens] . P^T [tokens x G]
// both run on v_mfma_f32_16x16x4_f32 (full fp32 products and sums), with the
// G query heads as the 16-wide N dimension.  Operand layouts are chosen so
// that nothing goes through LDS:
//   * K: lane (g = lane/16, c = lane%16) holds token c of the page and, for
//     k-step ks, dim 16*(ks/4) + 4*g + ks%4 -- four 16-byte loads per page;
//   * S^T lands in lane (g, c) as tokens 4g+i (i < 4) of query c, which is
//     exactly the B operand P^T of the second product for k-step i;
//   * V^T: lane (g, c) loads V[token 4g+i][dims 64h + 4c .. 64h + 4c+3] as one
//     16-byte load (16 lanes of a group read a 256-byte row segment); element
//     j of that vector is the A operand of output tile dt = 4h + j, so tile dt
//     row r holds dim 64h + 4r + j (a permutation undone when the tiles are
//     written to LDS).
// Softmax state (max, sum) is per query column, kept in every lane of the
// column; the running max needs two cross-row shuffles per page.
// A work-group runs a round of up to kSegMax segments (page ranges of
// different (sequence, kv head) units) at once: the 4 waves take interleaved
// pages of the round's concatenated page list, so every wave issues its first
// loads at the start whatever the segment boundaries; a wave that crosses into
// the next segment parks its softmax state in LDS and loads the next query
// rows.  Afterwards the waves merge each segment's states through LDS, the
// query heads spread over the waves.
#pragma once

#include "attn_common.h"

namespace llkv {

typedef float mf32x4 __attribute__((ext_vector_type(4)));

template <int D, int G>
struct MfmaF32Decode {
    static_assert(G >= 1 && G <= 16, "up to 16 query heads per KV head");
    static_assert(D % 64 == 0, "head_dim multiple of 64");
    using T = float;
    static constexpr int W = 4;               // waves per work-group
    static constexpr int KC = D / 16;         // 16-byte K chunks per lane per page
    static constexpr int KS = D / 4;          // k-steps of S^T = K Q^T
    static constexpr int DT = D / 16;         // 16-dim tiles of O^T
    static constexpr int VH = D / 64;         // 16-byte V vectors per lane per token
    static constexpr int MD = (D + 63) / 64;
    static constexpr int GQ = G, HD = D;
    // Resident waves per SIMD the register budget is held to: 5 (<= 96
    // registers) for head_dim 64; head_dim 128 needs more and gets 4.
    static constexpr int kWavesPerEU = D == 64 ? 5 : 4;
    // Segments per round: two where the LDS for the parked states stays small.
    static constexpr int kSegMax = G * D <= 512 ? 2 : 1;

    struct Smem {
        float acc[kSegMax][W][G][D];
        float ml[kSegMax][W][G][2];   // (max, sum); sum 0: the wave had no page
    };

    __device__ static void round(const DecodeArgs& a, Smem& sm, const SegDesc* segs, int nseg,
                                 int64_t po_stride, int64_t pl_stride) {
        const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
        const int g = lane >> 4, c = lane & 15;
        const int np_total = segs[nseg - 1].cum + segs[nseg - 1].npages;
        const int64_t row_elems = (int64_t)a.Hkv * D;

        // Empty states for this wave's slots (a wave may own no page of a segment).
        for (int s = 0; s < nseg; ++s) {
            for (int i = lane; i < G * D; i += 64) (&sm.acc[s][w][0][0])[i] = 0.0f;
            if (lane < G) {
                sm.ml[s][w][lane][0] = kNegBig;
                sm.ml[s][w][lane][1] = 0.0f;
            }
        }

        // Physical page of this wave's k-th page (k = lane + tbl_k0), j = w + 4k.
        int tbl = 0, tbl_k0 = 0;
        auto load_tbl = [&](int k0) {
            const int j = w + W * (k0 + lane);
            int v = 0;
            if (j < np_total) {
                int s = 0;
                while (s + 1 < nseg && j >= segs[s + 1].cum) ++s;
                const SegDesc& d = segs[s];
                v = a.bt[(int64_t)d.b * a.max_blocks + d.pg_begin + (j - d.cum)];
            }
            tbl = v;
        };
        load_tbl(0);

        // State of the current segment.
        int cur = -1, sb = 0, skvh = 0, spg = 0, scum = 0, stok = 0;
        int next_cum = 0;   // first page of the next segment (register copy)
        float qop[KS];
        mf32x4 o[DT];
        float m = kNegBig, lsum = 0.0f;

        auto flush = [&](int s) {
            float ls = lsum;
            ls += __shfl_xor(ls, 16, 64);
            ls += __shfl_xor(ls, 32, 64);
            if (c < G) {
                // tile 4h + j, row 4g + i  ->  dim 64h + 16g + 4i + j
#pragma unroll
                for (int h = 0; h < VH; ++h)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        *reinterpret_cast<float4*>(&sm.acc[s][w][c][64 * h + 16 * g + 4 * i]) =
                            make_float4(o[4 * h][i], o[4 * h + 1][i], o[4 * h + 2][i], o[4 * h + 3][i]);
                if (g == 0) {
                    sm.ml[s][w][c][0] = m;
                    sm.ml[s][w][c][1] = ls;
                }
            }
        };

        float4 kr[KC];
        float4 vr[VH][4];
        for (int k = 0;; ++k) {
            const int j = w + W * k;
            if (j >= np_total) break;
            if (k - tbl_k0 >= 64) {
                tbl_k0 = k;
                load_tbl(k);
            }
            if (j >= next_cum) {   // uniform: park the previous state, start the next segment
                int s = cur < 0 ? 0 : cur;
                while (s + 1 < nseg && j >= segs[s + 1].cum) ++s;
                if (cur >= 0) flush(cur);
                cur = s;
                next_cum = s + 1 < nseg ? segs[s + 1].cum : INT_MAX;
                sb = segs[s].b;
                skvh = segs[s].kvh;
                spg = segs[s].pg_begin;
                scum = segs[s].cum;
                stok = segs[s].tok_end;
                // Q^T operand: column c is query head kvh*G + c (zero beyond G), pre-scaled.
                const float* qrow = reinterpret_cast<const float*>(a.q) +
                                    ((int64_t)sb * a.Hq + skvh * G + c) * D;
#pragma unroll
                for (int cc = 0; cc < KC; ++cc) {
                    float4 v = c < G ? *reinterpret_cast<const float4*>(qrow + 16 * cc + 4 * g)
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
                    qop[4 * cc + 0] = v.x * a.scale_log2;
                    qop[4 * cc + 1] = v.y * a.scale_log2;
                    qop[4 * cc + 2] = v.z * a.scale_log2;
                    qop[4 * cc + 3] = v.w * a.scale_log2;
                }
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) o[dt] = mf32x4{0.f, 0.f, 0.f, 0.f};
                m = kNegBig;
                lsum = 0.0f;
            }
            const int pg = spg + (j - scum);
            const int64_t phys = max(__builtin_amdgcn_readlane(tbl, k - tbl_k0), 0);

            // K rows: lane (g, c) holds token c, dims 16 cc + 4 g .. + 3.
            const float* kp = reinterpret_cast<const float*>(a.k) + (int64_t)skvh * D +
                              (phys * kPage + c) * row_elems + 4 * g;
#pragma unroll
            for (int cc = 0; cc < KC; ++cc) kr[cc] = *reinterpret_cast<const float4*>(kp + 16 * cc);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float* vp = reinterpret_cast<const float*>(a.v) + (int64_t)skvh * D +
                                  (phys * kPage + 4 * g + i) * row_elems + 4 * c;
#pragma unroll
                for (int h = 0; h < VH; ++h) vr[h][i] = *reinterpret_cast<const float4*>(vp + 64 * h);
            }

            mf32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int cc = 0; cc < KC; ++cc) {
                sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[cc].x, qop[4 * cc + 0], sacc, 0, 0, 0);
                sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[cc].y, qop[4 * cc + 1], sacc, 0, 0, 0);
                sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[cc].z, qop[4 * cc + 2], sacc, 0, 0, 0);
                sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[cc].w, qop[4 * cc + 3], sacc, 0, 0, 0);
            }
            const int t0 = pg * kPage + 4 * g;
            float x[4];
            float mt = kNegBig;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[i] = (t0 + i < stok) ? sacc[i] : -INFINITY;
                mt = fmaxf(mt, x[i]);
            }
            mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
            mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
            const float mnew = fmaxf(m, mt);
            const float corr = fast_exp2(m - mnew);
            m = mnew;
            float p[4];
            float ps = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                p[i] = fast_exp2(x[i] - mnew);
                ps += p[i];
            }
            lsum = fmaf(lsum, corr, ps);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[dt] *= corr;
#pragma unroll
            for (int h = 0; h < VH; ++h)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    o[4 * h + 0] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[h][i].x, p[i], o[4 * h + 0], 0, 0, 0);
                    o[4 * h + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[h][i].y, p[i], o[4 * h + 1], 0, 0, 0);
                    o[4 * h + 2] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[h][i].z, p[i], o[4 * h + 2], 0, 0, 0);
                    o[4 * h + 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[h][i].w, p[i], o[4 * h + 3], 0, 0, 0);
                }
        }
        if (cur >= 0) flush(cur);
        LLKV_TRACE_POINT(1);
        __syncthreads();

        // Merge the 4 waves' states of each segment; heads spread over the waves.
        for (int s = 0; s < nseg; ++s) {
            const SegDesc& d = segs[s];
            for (int h = w; h < G; h += W) {
                float M = sm.ml[s][0][h][0];
#pragma unroll
                for (int ww = 1; ww < W; ++ww) M = fmaxf(M, sm.ml[s][ww][h][0]);
                float f[W], L = 0.0f;
#pragma unroll
                for (int ww = 0; ww < W; ++ww) {
                    f[ww] = fast_exp2(sm.ml[s][ww][h][0] - M);
                    L = fmaf(f[ww], sm.ml[s][ww][h][1], L);
                }
                const float inv = 1.0f / L;
#pragma unroll
                for (int i = 0; i < MD; ++i) {
                    const int dd = lane + 64 * i;
                    float ov = 0.0f;
#pragma unroll
                    for (int ww = 0; ww < W; ++ww) ov = fmaf(f[ww], sm.acc[s][ww][h][dd], ov);
                    ov *= inv;
                    if (d.direct)
                        reinterpret_cast<float*>(a.out)[((int64_t)d.b * a.Hq + d.kvh * G + h) * D + dd] = ov;
                    else
                        a.part_o[d.po_off + h * po_stride + dd] = ov;
                }
                if (!d.direct && lane == 0) a.part_lse[d.pl_off + h * pl_stride] = M + fast_log2(L);
            }
        }
        lds_barrier();   // the partial / output stores need not complete here
        LLKV_TRACE_POINT(2);
    }
};

}  // namespace llkv
