// Decode schedules over an MFMA body (decode_mfma.h): the fixed-split and
// balanced kernels, and the group-size table of the tuned instantiations.
// Included by the per-pool-type translation units only.
#pragma once

#include <hip/hip_runtime.h>

#include "decode_kernels.h"
#include "decode_mfma.h"

namespace llkv {
namespace {

// Fixed split schedule: grid (S_max, Hkv, B), Body::W waves per work-group,
// one segment each.
template <class Body>
__global__ __launch_bounds__(Body::kThreads) __attribute__((amdgpu_waves_per_eu(Body::kWavesPerEU)))
void decode_split_kernel(DecodeArgs a) {
    __shared__ typename Body::Smem sm;
    __shared__ SegDesc segs[1];
    using T = typename Body::T;
    LLKV_TRACE_POINT(0);
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const SplitGeo geo = split_geo(a, b);
    const int hq0 = kvh * Body::GQ;
    if (geo.npages == 0) {   // empty sequence: zeros, as the reference (:224-227)
        if (split == 0) {
            T* out = reinterpret_cast<T*>(a.out) + ((int64_t)b * a.Hq + hq0) * Body::HD;
            for (int i = threadIdx.x; i < Body::GQ * Body::HD; i += blockDim.x)
                out[i] = Elem<T>::from_f32(0.0f);
        }
        return;
    }
    if (split >= geo.nsplit) return;
    if (threadIdx.x == 0) {
        SegDesc& d = segs[0];
        d.b = b;
        d.kvh = kvh;
        d.pg_begin = split * geo.pps;
        d.npages = min(geo.pps, geo.npages - d.pg_begin);
        d.cum = 0;
        d.tok_end = min((d.pg_begin + d.npages) * kPage, geo.L);
        d.direct = geo.nsplit == 1;
        d.new_tok = seg_new_tok(a, b, d.pg_begin, d.tok_end, geo.L);
        const int64_t bh0 = (int64_t)b * a.Hq + hq0;
        d.po_off = (bh0 * a.S_max + split) * a.D;
        d.pl_off = bh0 * a.S_max + split;
    }
    __syncthreads();
    store_new_row<T, Body::HD>(a, segs[0]);
    Body::round(a, sm, segs, 1, (int64_t)a.S_max * a.D, a.S_max);
}

// Balanced schedule: grid (nwg), 4 waves per work-group.  Every work-group
// scans the lengths itself (the batch is at most kBalanceMaxB sequences) and
// cuts its share into segments, run kSegMax segments per round.  A unit
// (sequence, kv head) inside one share is written directly; the others are
// merged by decode_merge_balanced_kernel.  Work-group 0 stores the page
// prefix sums for that kernel; empty sequences get zeros from the work-group
// with their index modulo nwg.
template <class Body>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(Body::kWavesPerEU)))
void decode_balanced_kernel(DecodeArgs a) {
    using T = typename Body::T;
    constexpr int D = Body::HD;
    __shared__ typename Body::Smem sm;
    __shared__ int sP[kBalanceMaxB + 1];
    __shared__ int sL[kBalanceMaxB];
    __shared__ SegDesc segs[Body::kSegMax];
    __shared__ int s_n;
    __shared__ int64_t s_next;
    LLKV_TRACE_POINT(0);
    scan_pages(a, sP, sL);
    LLKV_TRACE_POINT(4);
    const int tid = threadIdx.x;
    if (blockIdx.x == 0)
        for (int i = tid; i <= a.B; i += blockDim.x) a.plan[i] = sP[i];
    const int64_t T_ = (int64_t)a.Hkv * sP[a.B];
    const int64_t wg = blockIdx.x;
    for (int b = (int)wg; b < a.B; b += a.nwg) {   // the reference's seq_len == 0 rule (:224-227)
        if (sP[b + 1] != sP[b]) continue;
        T* out = reinterpret_cast<T*>(a.out) + (int64_t)b * a.Hq * D;
        for (int i = tid; i < a.Hq * D; i += blockDim.x) out[i] = Elem<T>::from_f32(0.0f);
    }
    const int64_t r1 = share_begin(wg + 1, T_, a.nwg);
    int64_t p = share_begin(wg, T_, a.nwg);
    while (p < r1) {
        if (tid == 0) {
            int n = 0;
            s_next = build_segments(a, sP, sL, p, r1, wg, Body::kSegMax, segs, &n);
            s_n = n;
        }
        __syncthreads();
        const int n = s_n;
        p = s_next;
        for (int i = 0; i < n; ++i) store_new_row<T, D>(a, segs[i]);
        Body::round(a, sm, segs, n, D, 1);   // ends with a barrier
    }
}

template <class Body>
Kernels kernels_of() {
    Kernels k;
    k.split = decode_split_kernel<Body>;
    k.balanced = decode_balanced_kernel<Body>;
    return k;
}

// head_dim 64 / 128 also get the unit schedule's kUnitWaves-wave kernel,
// except fp32 at head_dim 128, whose body does not fit the 128 registers of
// four waves per SIMD (~50 would spill).
template <typename T, int D, int G, bool A>
Kernels kernels_with_unit() {
    Kernels k = kernels_of<MfmaDecode<T, D, G, A>>();
    if constexpr (!(Elem<T>::kDtype == LLKV_DTYPE_F32 && D == 128))
        k.unit = decode_split_kernel<MfmaDecode<T, D, G, A, kUnitWaves>>;
    return k;
}

template <typename T, int D, bool A>
Kernels tuned_g(int G) {
    switch (G) {
        case 1: return kernels_with_unit<T, D, 1, A>();
        case 2: return kernels_with_unit<T, D, 2, A>();
        case 3: return kernels_with_unit<T, D, 3, A>();
        case 4: return kernels_with_unit<T, D, 4, A>();
        case 5: return kernels_with_unit<T, D, 5, A>();
        case 6: return kernels_with_unit<T, D, 6, A>();
        case 7: return kernels_with_unit<T, D, 7, A>();
        case 8: return kernels_with_unit<T, D, 8, A>();
        case 12: return kernels_with_unit<T, D, 12, A>();
        case 16: return kernels_with_unit<T, D, 16, A>();
    }
    return Kernels();
}

// head_dim 96 (Phi-3 layouts) and 256 (Gemma-2 / Gemma-3 layouts): group
// sizes 1, 2, 4, 8.
template <typename T, int D, bool A>
Kernels tuned_g_few(int G) {
    switch (G) {
        case 1: return kernels_of<MfmaDecode<T, D, 1, A>>();
        case 2: return kernels_of<MfmaDecode<T, D, 2, A>>();
        case 4: return kernels_of<MfmaDecode<T, D, 4, A>>();
        case 8: return kernels_of<MfmaDecode<T, D, 8, A>>();
    }
    return Kernels();
}

template <typename T>
Kernels tuned(int D, int G, bool append) {
    if (D == 64) return append ? tuned_g<T, 64, true>(G) : tuned_g<T, 64, false>(G);
    if (D == 128) return append ? tuned_g<T, 128, true>(G) : tuned_g<T, 128, false>(G);
    if (D == 256) return append ? tuned_g_few<T, 256, true>(G) : tuned_g_few<T, 256, false>(G);
    if (D == 96) return append ? tuned_g_few<T, 96, true>(G) : tuned_g_few<T, 96, false>(G);
    return Kernels();
}

}  // namespace
}  // namespace llkv
