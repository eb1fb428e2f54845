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
//    short sequences in a mixed batch launch no idle split.  The split that
//    finishes last for a (sequence, kv_head) -- detected with an agent-scope
//    atomic counter -- merges the partials by log-sum-exp in the same launch;
//    a sequence with one split writes the output directly.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "attn_common.h"

namespace llkv {
namespace {

template <typename T, int D, int G>
struct FastCfg {
    static constexpr int VEC = Chunk<T>::VEC;          // elements per 16 B
    static constexpr int NJ = sizeof(T) == 4 ? 2 : 1;   // 16 B chunks per lane
    static constexpr int DPL = NJ * VEC;                // dims per lane (8)
    static constexpr int LPT = D / DPL;                 // lanes per token
    static constexpr int TPS = 64 / LPT;                // tokens per step
    static constexpr int U = 8 / NJ;                    // steps per tile
    static constexpr int TILE = U * TPS;
    static_assert(D % DPL == 0, "head_dim must be a multiple of 8");
    static_assert(TPS >= 1 && TPS <= 16 && 16 % TPS == 0, "step must stay inside a page");
};

template <typename T, int D, int G>
__global__ __launch_bounds__(64) void decode_fast_kernel(DecodeArgs a) {
    using C = FastCfg<T, D, G>;
    constexpr int VEC = C::VEC, NJ = C::NJ, DPL = C::DPL, LPT = C::LPT;
    constexpr int TPS = C::TPS, U = C::U, TILE = C::TILE;

    const int lane = threadIdx.x;
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const SplitGeo geo = split_geo(a, b);
    const int hq0 = kvh * G;
    T* out = reinterpret_cast<T*>(a.out);

    if (geo.npages == 0) {   // empty sequence: zeros, as the reference (:224-227)
        if (split == 0) {
            for (int i = lane; i < G * D; i += 64)
                out[((int64_t)b * a.Hq + hq0) * D + i] = Elem<T>::from_f32(0.0f);
        }
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

    for (int t0 = tok_begin; t0 < tok_end; t0 += TILE) {
        uint4 kr[U][NJ], vr[U][NJ];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int ts = t0 + u * TPS;                  // first token of the step (uniform)
            const int page = min(ts >> 4, last_page);     // steps past the end re-read a valid page
            const int64_t phys = max(bt[page], 0);          // a -1 hole reads page 0, never faults
            const int64_t row = phys * kPage + (ts & 15) + grp;
            const T* kp = kbase + row * row_elems;
            const T* vp = vbase + row * row_elems;
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                kr[u][j] = *reinterpret_cast<const uint4*>(kp + j * LPT * VEC);
                vr[u][j] = *reinterpret_cast<const uint4*>(vp + j * LPT * VEC);
            }
        }

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
    }

    // Merge the TPS token groups of the wave (lanes with equal `part`).
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

    const bool direct = geo.nsplit == 1;
    if (grp == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float inv = 1.0f / l[g];
            float o[DPL];
#pragma unroll
            for (int e = 0; e < DPL; ++e) o[e] = acc[g][e] * inv;
            const int64_t bh = (int64_t)b * a.Hq + hq0 + g;
            if (direct) {
                T* op = out + bh * D;
#pragma unroll
                for (int j = 0; j < NJ; ++j)
                    *reinterpret_cast<uint4*>(op + (j * LPT + part) * VEC) = Chunk<T>::pack(&o[j * VEC]);
            } else {
                float* pp = a.part_o + (bh * a.S_max + split) * D;
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
#pragma unroll
                    for (int e4 = 0; e4 < VEC; e4 += 4)
                        *reinterpret_cast<float4*>(pp + (j * LPT + part) * VEC + e4) =
                            make_float4(o[j * VEC + e4], o[j * VEC + e4 + 1], o[j * VEC + e4 + 2],
                                        o[j * VEC + e4 + 3]);
                }
                if (part == 0) a.part_lse[bh * a.S_max + split] = m[g] + fast_log2(l[g]);
            }
        }
    }
    if (direct) return;
    // The split that completes this (sequence, kv_head) merges all its partials.
    int* counter = a.counters + (int64_t)b * a.Hq + hq0;
    if (split_arrive_last(counter, geo.nsplit)) split_merge<T>(a, b, hq0, G, geo.nsplit, counter);
}

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
    int* counter = a.counters + bh;
    if (split_arrive_last(counter, geo.nsplit)) split_merge<T>(a, b, hq, 1, geo.nsplit, counter);
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

struct Plan {
    int S_max;
    int pps_auto;
    int fixed_S;
};

// Automatic split size: aim for roughly 8 resident waves per CU over the
// whole batch (256 CUs), never below 4 pages (64 tokens) per split so that
// partial traffic stays a few percent of the KV bytes.
Plan make_plan(int B, int Hkv, int bs, int max_seq_len, int num_splits) {
    Plan p;
    int max_pages = (std::max(max_seq_len, 1) + bs - 1) / bs;
    if (num_splits > 0) {
        p.fixed_S = num_splits;
        p.pps_auto = 1;
        p.S_max = std::min(num_splits, max_pages);
    } else {
        p.fixed_S = 0;
        const int64_t target_items = 256 * 8;
        int64_t units = (int64_t)B * Hkv;
        int64_t want = (target_items + units - 1) / units;   // splits per (seq, kv_head)
        int pps = (int)std::max<int64_t>(4, (max_pages + want - 1) / want);
        p.pps_auto = pps;
        p.S_max = (max_pages + pps - 1) / pps;
    }
    if (p.S_max < 1) p.S_max = 1;
    return p;
}

// Workspace: [counters: fixed kCounterBytes][lse B*Hq*S_max][o B*Hq*S_max*D].
// The counter region has the same size and place for every call, so a
// workspace reused across batch shapes never finds partial data where a
// counter is expected (the counters are zero between calls).
constexpr size_t kCounterBytes = 256 * 1024;
constexpr int kMaxHeadRows = (int)(kCounterBytes / sizeof(int));   // B * Hq limit
size_t counter_bytes(int, int) { return kCounterBytes; }

size_t workspace_for(int B, int Hq, int D, const Plan& p) {
    if (p.S_max <= 1) return 0;
    size_t n = (size_t)B * Hq * p.S_max;
    return counter_bytes(B, Hq) + ((n * sizeof(float) + 255) & ~(size_t)255) + n * D * sizeof(float);
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
    if (p.S_max > 1 && (int64_t)num_seqs * num_q_heads > kMaxHeadRows)
        return set_error(LLKV_ERR_UNSUPPORTED, "%s: num_seqs * num_q_heads %lld exceeds %d", fn,
                         (long long)num_seqs * num_q_heads, kMaxHeadRows);
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
    a.counters = need ? reinterpret_cast<int*>(ws) : nullptr;
    a.part_lse = need ? reinterpret_cast<float*>(ws + counter_bytes(num_seqs, num_q_heads)) : nullptr;
    a.part_o = need ? reinterpret_cast<float*>(ws + counter_bytes(num_seqs, num_q_heads) +
                                               ((n * sizeof(float) + 255) & ~(size_t)255))
                    : nullptr;
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
        if (dtype == LLKV_DTYPE_F32) fast = pick_fast<float>(head_dim, G);
        else if (dtype == LLKV_DTYPE_F16) fast = pick_fast<_Float16>(head_dim, G);
        else if (dtype == LLKV_DTYPE_BF16) fast = pick_fast<bf16_t>(head_dim, G);
    }
    if (fast) {
        dim3 grid(p.S_max, num_kv_heads, num_seqs);
        fast<<<grid, 64, 0, st>>>(a);
    } else {
        dim3 grid(p.S_max, num_q_heads, num_seqs);
        if (dtype == LLKV_DTYPE_F32) decode_generic_kernel<float><<<grid, 64, 0, st>>>(a);
        else if (dtype == LLKV_DTYPE_F16) decode_generic_kernel<_Float16><<<grid, 64, 0, st>>>(a);
        else decode_generic_kernel<bf16_t><<<grid, 64, 0, st>>>(a);
    }
    return check_launch(fn);
}

