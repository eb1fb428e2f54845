// Paged decode attention for gfx950 (one new query token per sequence).
//
// Replaces the reference's decode kernels (src/kv_cache/paged_attention.cu:
// baseline :104-170, v2 :186-310, Split-K :324-460, reduce :477-532) and the
// host dispatcher (:537-626).  Math is the same online softmax; the mapping
// to the hardware is new:
//
//  * One wave64 per (split, kv_head, sequence).  All G = Hq/Hkv query heads of
//    the KV head are computed by that wave, so every K/V byte is read from
//    HBM once (the reference launches one block per query head and re-reads
//    K/V G times).
//  * A token's row (D elements) is spread over LPT = D/8 lanes, 8 dims per
//    lane, loaded as 16-byte global_load_dwordx4; 64/LPT tokens per step,
//    8 (fp16/bf16) or 4 (fp32) steps in flight per tile: 16 outstanding
//    dwordx4 loads per lane, no LDS round trip.
//  * The per-token dot product is finished with DPP row reductions
//    (quad_perm, row_half_mirror, row_mirror); each token group keeps its own
//    running (max, sum, acc) so no cross-group traffic happens until the end
//    of the split, where the groups are merged by log-sum-exp with shuffles.
//  * Split-K is per sequence: a sequence of n pages gets ceil(n/pps) splits
//    (automatic) or the reference's S ranges of ceil(n/S) pages (fixed), so
//    short sequences in a mixed batch launch no idle split.  Partials are
//    merged by log-sum-exp in a small second kernel; a sequence with one
//    split writes the output directly.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "attn_common.h"
#include "decode_fast.h"
#include "decode_mfma.h"

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
            float d0 = 0.0f;
            for (int d = 0; d < D; ++d) d0 = fmaf(q_s[d], Elem<T>::to_f32(kp[row + d]), d0);
            s = d0;
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

// Merge of the split partials of one (sequence, q head), launched after the
// split kernel (the reference's paged_attention_reduce_kernel,
// src/kv_cache/paged_attention.cu:477-532, in normalised form:
// out = sum_s 2^(lse_s - M) o_s / sum_s 2^(lse_s - M)).  One wave; lane owns
// dims lane + 64 i (i < MD); partials are fetched 8 splits at a time so a
// merge costs ceil(nsplit / 8) memory round trips.
template <typename T, int MD>
__global__ __launch_bounds__(64) void decode_merge_kernel(DecodeArgs a) {
    const int hq = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
    const SplitGeo geo = split_geo(a, b);
    if (geo.nsplit <= 1) return;   // written directly by the split kernel
    const int D = a.D, nsplit = geo.nsplit;
    const int64_t bh = (int64_t)b * a.Hq + hq;
    const float* lse = a.part_lse + bh * a.S_max;
    const float* po = a.part_o + bh * a.S_max * D;
    float mx = -INFINITY;
    for (int s = lane; s < nsplit; s += 64) mx = fmaxf(mx, lse[s]);
    const float M = wave_max(mx);
    constexpr int SC = 8;
    float W = 0.0f, o[MD];
#pragma unroll
    for (int i = 0; i < MD; ++i) o[i] = 0.0f;
    for (int s0 = 0; s0 < nsplit; s0 += SC) {
        float lv[SC], pv[SC][MD];
#pragma unroll
        for (int j = 0; j < SC; ++j) {
            const int s = min(s0 + j, nsplit - 1);   // clamped reads; weight zeroed below
            lv[j] = lse[s];
#pragma unroll
            for (int i = 0; i < MD; ++i) pv[j][i] = po[(int64_t)s * D + min(lane + 64 * i, D - 1)];
        }
#pragma unroll
        for (int j = 0; j < SC; ++j) {
            const float w = s0 + j < nsplit ? fast_exp2(lv[j] - M) : 0.0f;
            W += w;
#pragma unroll
            for (int i = 0; i < MD; ++i) o[i] = fmaf(w, pv[j][i], o[i]);
        }
    }
    T* out = reinterpret_cast<T*>(a.out) + bh * D;
    const float inv = 1.0f / W;
#pragma unroll
    for (int i = 0; i < MD; ++i)
        if (lane + 64 * i < D) out[lane + 64 * i] = Elem<T>::from_f32(o[i] * inv);
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------
typedef void (*DecodeFn)(DecodeArgs);

template <typename T, int D>
DecodeFn pick_fast_g(int G) {
    switch (G) {
        case 1: return decode_fast_kernel<T, D, 1>;
        case 2: return decode_fast_kernel<T, D, 2>;
        case 4: return decode_fast_kernel<T, D, 4>;
        case 7: return decode_fast_kernel<T, D, 7>;
        case 8: return decode_fast_kernel<T, D, 8>;
    }
    return nullptr;
}

template <typename T>
DecodeFn pick_fast(int D, int G) {
    if (D == 64) return pick_fast_g<T, 64>(G);
    if (D == 128) return pick_fast_g<T, 128>(G);
    return nullptr;
}

template <int D>
DecodeFn pick_mfma_f32_g(int G) {
    switch (G) {
        case 1: return decode_mfma_f32_kernel<D, 1>;
        case 2: return decode_mfma_f32_kernel<D, 2>;
        case 4: return decode_mfma_f32_kernel<D, 4>;
        case 7: return decode_mfma_f32_kernel<D, 7>;
        case 8: return decode_mfma_f32_kernel<D, 8>;
        case 16: return decode_mfma_f32_kernel<D, 16>;
    }
    return nullptr;
}

// fp32 pools: the MFMA kernel (decode_mfma.h).
DecodeFn pick_f32(int D, int G) {
    if (D == 64) return pick_mfma_f32_g<64>(G);
    if (D == 128) return pick_mfma_f32_g<128>(G);
    return nullptr;
}

struct Plan {
    int S_max;
    int pps_auto;
    int fixed_S;
};

// Automatic split size (pages per split).  Only the longest length is known
// on the host, so the batch is sized as if sequences averaged half of it:
// about 4096 splits in total (16 waves per CU over 256 CUs), at least 4
// pages (64 tokens) per split so partials stay a few percent of the KV
// bytes, and at most kMaxAutoSplits splits per sequence so the merge that
// closes a sequence stays short.
constexpr int kMaxAutoSplits = 64;

Plan make_plan(int B, int Hkv, int bs, int max_seq_len, int num_splits) {
    Plan p;
    int max_pages = (std::max(max_seq_len, 1) + bs - 1) / bs;
    if (num_splits > 0) {
        p.fixed_S = num_splits;
        p.pps_auto = 1;
        p.S_max = std::min(num_splits, max_pages);
    } else {
        p.fixed_S = 0;
        // Split-kernel work-groups are 4 waves; aim for ~1280 of them (5 per
        // CU, all resident at once), assuming sequences average half the
        // longest.
        const int64_t units = (int64_t)B * Hkv;
        int64_t pps = ((int64_t)max_pages * units / 2 + 1279) / 1280;
        const int64_t lo = std::max<int64_t>(4, (max_pages + kMaxAutoSplits - 1) / kMaxAutoSplits);
        // At most 32 pages (512 tokens) per chunk unless the split cap forces
        // it: a few long sequences in a batch of short ones (a lognormal mix)
        // must still be spread over many work-groups.
        const int64_t hi = std::max<int64_t>(lo, 32);
        pps = std::min(std::max(pps, lo), hi);
        p.pps_auto = (int)pps;
        p.S_max = (int)((max_pages + pps - 1) / pps);
    }
    if (p.S_max < 1) p.S_max = 1;
    return p;
}

// Workspace: [lse B*Hq*S_max, 256 B aligned][o B*Hq*S_max*D], fp32.
size_t lse_bytes(size_t n) { return (n * sizeof(float) + 255) & ~(size_t)255; }

size_t workspace_for(int B, int Hq, int D, const Plan& p) {
    if (p.S_max <= 1) return 0;
    size_t n = (size_t)B * Hq * p.S_max;
    return lse_bytes(n) + n * D * sizeof(float);
}

}  // namespace
}  // namespace llkv

using namespace llkv;

extern "C" size_t llkv_paged_decode_workspace_size(int num_seqs, int num_q_heads,
                                                   int num_kv_heads, int head_dim,
                                                   int block_size, int max_seq_len,
                                                   int num_splits) {
    if (num_seqs <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 ||
        block_size <= 0)
        return 0;
    Plan p = make_plan(num_seqs, num_kv_heads, block_size, max_seq_len, num_splits);
    return workspace_for(num_seqs, num_q_heads, head_dim, p);
}

extern "C" int llkv_paged_decode(void* out, const void* q, const void* k_pool,
                                 const void* v_pool, const int* block_table,
                                 const int* seq_lens, int num_seqs, int num_q_heads,
                                 int num_kv_heads, int head_dim, int block_size,
                                 int max_blocks_per_seq, int max_seq_len, int num_splits,
                                 float scale, int dtype, void* workspace,
                                 size_t workspace_bytes, void* stream) {
    const char* fn = "llkv_paged_decode";
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
    if (max_seq_len > max_blocks_per_seq * block_size) max_seq_len = max_blocks_per_seq * block_size;

    Plan p = make_plan(num_seqs, num_kv_heads, block_size, max_seq_len, num_splits);
    size_t need = workspace_for(num_seqs, num_q_heads, head_dim, p);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
        return set_error(LLKV_ERR_WORKSPACE, "%s: workspace %zu bytes < required %zu", fn,
                         workspace_bytes, need);

    DecodeArgs a;
    a.out = out;
    a.q = q;
    a.k = k_pool;
    a.v = v_pool;
    a.bt = block_table;
    a.lens = seq_lens;
    size_t n = (size_t)num_seqs * num_q_heads * p.S_max;
    char* ws = reinterpret_cast<char*>(workspace);
    a.part_lse = need ? reinterpret_cast<float*>(ws) : nullptr;
    a.part_o = need ? reinterpret_cast<float*>(ws + lse_bytes(n)) : nullptr;
    a.B = num_seqs;
    a.Hq = num_q_heads;
    a.Hkv = num_kv_heads;
    a.D = head_dim;
    a.bs = block_size;
    a.max_blocks = max_blocks_per_seq;
    a.S_max = p.S_max;
    a.pps_auto = p.pps_auto;
    a.fixed_S = p.fixed_S;
    a.scale_log2 = scale * kLog2e;

    const int G = num_q_heads / num_kv_heads;
    hipStream_t st = (hipStream_t)stream;
    // The fast kernel needs 16-token pages, 16-byte aligned rows and pointers.
    const size_t es = dtype_bytes(dtype);
    const bool aligned = (((uintptr_t)q | (uintptr_t)out | (uintptr_t)k_pool |
                           (uintptr_t)v_pool) & 15) == 0 &&
                         ((size_t)num_kv_heads * head_dim * es) % 16 == 0;
    DecodeFn fast = nullptr;
    if (block_size == kPage && aligned) {
        if (dtype == LLKV_DTYPE_F32) fast = pick_f32(head_dim, G);
        else if (dtype == LLKV_DTYPE_F16) fast = pick_fast<_Float16>(head_dim, G);
        else if (dtype == LLKV_DTYPE_BF16) fast = pick_fast<bf16_t>(head_dim, G);
    }
    if (fast) {
        dim3 grid(p.S_max, num_kv_heads, num_seqs);
        fast<<<grid, 64 * kDecodeWaves, 0, st>>>(a);
    } else {
        dim3 grid(p.S_max, num_q_heads, num_seqs);
        if (dtype == LLKV_DTYPE_F32) decode_generic_kernel<float><<<grid, 64, 0, st>>>(a);
        else if (dtype == LLKV_DTYPE_F16) decode_generic_kernel<_Float16><<<grid, 64, 0, st>>>(a);
        else decode_generic_kernel<bf16_t><<<grid, 64, 0, st>>>(a);
    }
    if (int e = check_launch(fn)) return e;
    if (p.S_max > 1) {
        dim3 grid(num_q_heads, num_seqs);
        const bool wide = head_dim > 128;
        if (dtype == LLKV_DTYPE_F32) {
            if (wide) decode_merge_kernel<float, 4><<<grid, 64, 0, st>>>(a);
            else decode_merge_kernel<float, 2><<<grid, 64, 0, st>>>(a);
        } else if (dtype == LLKV_DTYPE_F16) {
            if (wide) decode_merge_kernel<_Float16, 4><<<grid, 64, 0, st>>>(a);
            else decode_merge_kernel<_Float16, 2><<<grid, 64, 0, st>>>(a);
        } else {
            if (wide) decode_merge_kernel<bf16_t, 4><<<grid, 64, 0, st>>>(a);
            else decode_merge_kernel<bf16_t, 2><<<grid, 64, 0, st>>>(a);
        }
        if (int e = check_launch(fn)) return e;
    }
    return LLKV_OK;
}

