// MFMA paged decode kernel for fp32 K/V on gfx950 (16-token pages, head_dim
// 64 / 128, up to 16 query heads per KV head).  Included by decode.hip.
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
//   * V^T: lane (g, c) of k-step i holds V[token 4g+i][dim 16*dt + c], a
//     4-byte load whose 16 lanes of a group read 64 contiguous bytes.
// Softmax state (max, sum) is per query column, kept in every lane of the
// column; the running max needs two cross-row shuffles per page.
// Work-group = 4 waves on one (chunk, kv_head, sequence); waves take
// interleaved pages and merge through LDS; the chunks of a sequence merge in
// the split-merge kernel (decode.hip).
#pragma once

#include "attn_common.h"

namespace llkv {

typedef float mf32x4 __attribute__((ext_vector_type(4)));

template <int D, int G>
__global__ __launch_bounds__(64 * 4) void decode_mfma_f32_kernel(DecodeArgs a) {
    static_assert(G >= 1 && G <= 16, "up to 16 query heads per KV head");
    static_assert(D % 16 == 0, "head_dim multiple of 16");
    constexpr int W = 4;               // waves per work-group
    constexpr int KC = D / 16;         // 16-byte K chunks per lane per page
    constexpr int KS = D / 4;          // k-steps of S^T = K Q^T
    constexpr int DT = D / 16;         // 16-dim tiles of O^T
    constexpr int MD = (D + 63) / 64;
    __shared__ float s_acc[W][G][D];
    __shared__ float s_ml[W][G][2];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    LLKV_TRACE_POINT(0);
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const SplitGeo geo = split_geo(a, b);
    const int hq0 = kvh * G;
    float* out = reinterpret_cast<float*>(a.out);

    if (geo.npages == 0) {   // empty sequence: zeros, as the reference (:224-227)
        if (split == 0)
            for (int i = tid; i < G * D; i += 64 * W) out[((int64_t)b * a.Hq + hq0) * D + i] = 0.0f;
        return;
    }
    if (split >= geo.nsplit) return;

    const int tok_begin = split * geo.pps * kPage;
    const int tok_end = min(tok_begin + geo.pps * kPage, geo.L);
    const int page_begin = tok_begin >> 4;
    const int last_page = (tok_end - 1) >> 4;

    // Q^T operand: column c is query head hq0 + c (zero beyond G), pre-scaled.
    float qop[KS];
    {
        const float* qrow = reinterpret_cast<const float*>(a.q) + ((int64_t)b * a.Hq + hq0 + c) * D;
#pragma unroll
        for (int cc = 0; cc < KC; ++cc) {
            float4 v = c < G ? *reinterpret_cast<const float4*>(qrow + 16 * cc + 4 * g)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
            qop[4 * cc + 0] = v.x * a.scale_log2;
            qop[4 * cc + 1] = v.y * a.scale_log2;
            qop[4 * cc + 2] = v.z * a.scale_log2;
            qop[4 * cc + 3] = v.w * a.scale_log2;
        }
    }

    mf32x4 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = mf32x4{0.f, 0.f, 0.f, 0.f};
    float m = kNegBig, lsum = 0.0f;

    const int64_t row_elems = (int64_t)a.Hkv * D;
    const float* kg = reinterpret_cast<const float*>(a.k) + (int64_t)kvh * D;
    const float* vg = reinterpret_cast<const float*>(a.v) + (int64_t)kvh * D;
    const int* bt = a.bt + (int64_t)b * a.max_blocks;

    // Page ids, 64 at a time, one per lane, read back with v_readlane.
    const int first = page_begin + w;          // this wave's first page
    int tbl_base = min(first, last_page);
    int tbl = bt[min(tbl_base + lane, last_page)];

    auto load_page = [&](int pg, float4 (&kr)[KC], float (&vr)[DT][4]) {
        if (pg + 1 > tbl_base + 64) {   // uniform
            tbl_base = pg;
            tbl = bt[min(tbl_base + lane, last_page)];
        }
        const int64_t phys = max(__builtin_amdgcn_readlane(tbl, pg - tbl_base), 0);
        const float* kp = kg + (phys * kPage + c) * row_elems + 4 * g;
#pragma unroll
        for (int cc = 0; cc < KC; ++cc) kr[cc] = *reinterpret_cast<const float4*>(kp + 16 * cc);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float* vp = vg + (phys * kPage + 4 * g + i) * row_elems + c;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) vr[dt][i] = vp[16 * dt];
        }
    };

    auto compute_page = [&](int pg, const float4 (&kr)[KC], const float (&vr)[DT][4]) {
        mf32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int cc = 0; cc < KC; ++cc) {
            s = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[cc].x, qop[4 * cc + 0], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[cc].y, qop[4 * cc + 1], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[cc].z, qop[4 * cc + 2], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[cc].w, qop[4 * cc + 3], s, 0, 0, 0);
        }
        const int t0 = pg * kPage + 4 * g;
        float x[4];
        float mt = kNegBig;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[i] = (t0 + i < tok_end) ? s[i] : -INFINITY;
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
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[dt][i], p[i], o[dt], 0, 0, 0);
    };

    // Wave w owns pages w, w+W, ... of the chunk.  One page of registers per
    // wave keeps the kernel at <= 128 VGPRs (4 waves per SIMD); the other
    // resident waves hide the load latency.
    float4 ka[KC];
    float va[DT][4];
    for (int pg = first; pg <= last_page; pg += W) {
        load_page(pg, ka, va);
        compute_page(pg, ka, va);
    }

    LLKV_TRACE_POINT(1);
    // Column sums over the 4 lane groups; then the 4 waves merge through LDS.
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    if (c < G) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
            *reinterpret_cast<float4*>(&s_acc[w][c][dt * 16 + 4 * g]) =
                make_float4(o[dt][0], o[dt][1], o[dt][2], o[dt][3]);
        if (g == 0) {
            s_ml[w][c][0] = m;
            s_ml[w][c][1] = lsum;
        }
    }
    __syncthreads();
    if (w != 0) return;

    const bool direct = geo.nsplit == 1;
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float M = s_ml[0][h][0];
#pragma unroll
        for (int ww = 1; ww < W; ++ww) M = fmaxf(M, s_ml[ww][h][0]);
        float f[W], L = 0.0f;
#pragma unroll
        for (int ww = 0; ww < W; ++ww) {
            f[ww] = fast_exp2(s_ml[ww][h][0] - M);
            L = fmaf(f[ww], s_ml[ww][h][1], L);
        }
        const float inv = 1.0f / L;
        const int64_t bh = (int64_t)b * a.Hq + hq0 + h;
#pragma unroll
        for (int i = 0; i < MD; ++i) {
            const int d = lane + 64 * i;
            if (d >= D) continue;
            float ov = 0.0f;
#pragma unroll
            for (int ww = 0; ww < W; ++ww) ov = fmaf(f[ww], s_acc[ww][h][d], ov);
            ov *= inv;
            if (direct) out[bh * D + d] = ov;
            else a.part_o[(bh * a.S_max + split) * D + d] = ov;
        }
        if (!direct && lane == 0) a.part_lse[bh * a.S_max + split] = M + fast_log2(L);
    }
    LLKV_TRACE_POINT(2);
}

}  // namespace llkv
