// Paged prefill attention (varlen, causal or not) and batched first prefill
// over contiguous K/V, for gfx950.
//
// Kernels:
//  * prefill_mfma_kernel / prefill_f32_kernel (prefill_mfma.hip): fp16/bf16
//    and fp32 at head_dim 64/96/128/256, 16-token pages -- MFMA QK^T and PV
//    tiles; the fast path.
//  * rows_generic_kernel (this file): any dtype, any head_dim <= 256, any
//    page size, paged or contiguous K/V.  One wave per (query row, q_head),
//    64 keys per iteration with one key per lane, then the probabilities are
//    broadcast through LDS for the V pass where lanes own output dims.
//
// Masking rules follow the reference kernels: paged prefill
// (src/kv_cache/paged_attention.cu:641-796, causal break at pos > abs_q_pos
// with abs_q_pos = total_seq - P + i) and first prefill (:1230-1325, keys of
// the entry with start+pos <= start+local).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "attn_common.h"
#include "prefill_mfma.h"

namespace llkv {
namespace {

struct RowArgs {
    void* out;
    const void* q;
    const void* k;
    const void* v;
    // paged mode
    const int* bt;
    const int* cu_q;
    const int* lens;
    int max_blocks, bs;
    // contiguous (first prefill) mode
    const int* offsets;
    const int* kv_offsets;
    const int* num_tokens;
    const int* token_cumsum;
    int N, Hq, Hkv, D, causal;
    float scale_log2;
};

__device__ inline int find_entry(const int* cum, int n, int g) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (cum[mid] <= g) lo = mid; else hi = mid - 1;
    }
    return lo;
}

template <typename T, bool PAGED>
__global__ __launch_bounds__(64) void rows_generic_kernel(RowArgs a) {
    __shared__ float q_s[256];
    __shared__ float p_s[64];
    __shared__ int64_t row_s[64];
    const int lane = threadIdx.x;
    const int r = blockIdx.x;      // global query row
    const int hq = blockIdx.y;
    const int D = a.D;
    const int G = a.Hq / a.Hkv;
    const int kvh = hq / G;

    int nkeys;
    int64_t q_off, o_off;          // element offsets of the q / out row
    const int* bt = nullptr;
    int64_t kv_base = 0;           // contiguous mode: element offset of key 0
    if (PAGED) {
        const int n = find_entry(a.cu_q, a.N, r);
        const int P = a.cu_q[n + 1] - a.cu_q[n];
        const int i = r - a.cu_q[n];
        int L = a.lens[n];
        const int cap = a.max_blocks * a.bs;
        L = L < 0 ? 0 : (L > cap ? cap : L);
        nkeys = a.causal ? L - P + i + 1 : L;
        nkeys = nkeys < 0 ? 0 : (nkeys > L ? L : nkeys);
        q_off = ((int64_t)r * a.Hq + hq) * D;
        o_off = q_off;
        bt = a.bt + (int64_t)n * a.max_blocks;
    } else {
        const int e = find_entry(a.token_cumsum, a.N, r);
        const int local = r - a.token_cumsum[e];
        nkeys = min(a.num_tokens[e], local + 1);
        q_off = (int64_t)a.offsets[e] + (int64_t)local * a.Hq * D + (int64_t)hq * D;
        const int64_t out_row = a.offsets[e] / (a.Hq * D) + local;
        o_off = (out_row * a.Hq + hq) * D;
        kv_base = a.kv_offsets[e];
    }

    const T* qp = reinterpret_cast<const T*>(a.q) + q_off;
    for (int d = lane; d < D; d += 64) q_s[d] = Elem<T>::to_f32(qp[d]) * a.scale_log2;
    __syncthreads();

    const T* kp = reinterpret_cast<const T*>(a.k);
    const T* vp = reinterpret_cast<const T*>(a.v);
    const int64_t row_elems = (int64_t)a.Hkv * D;
    float m = kNegBig, l = 0.0f, acc[4] = {0.f, 0.f, 0.f, 0.f};

    for (int t0 = 0; t0 < nkeys; t0 += 64) {
        const int t = t0 + lane;
        const bool valid = t < nkeys;
        int64_t row = 0;
        float s = -INFINITY;
        if (valid) {
            if (PAGED)
                row = ((int64_t)max(bt[t / a.bs], 0) * a.bs + t % a.bs) * row_elems + (int64_t)kvh * D;
            else
                row = kv_base + (int64_t)t * row_elems + (int64_t)kvh * D;
            // four interleaved running sums, added pairwise (as the generic decode)
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
        const int n = min(64, nkeys - t0);
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
    // A row with no visible key (possible only for inconsistent lengths) gives zeros.
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    T* op = reinterpret_cast<T*>(a.out) + o_off;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = lane + 64 * i;
        if (d < D) op[d] = Elem<T>::from_f32(acc[i] * inv);
    }
}

template <bool PAGED>
int launch_rows(const RowArgs& a, int rows, int dtype, hipStream_t st) {
    dim3 grid(rows, a.Hq);
    if (dtype == LLKV_DTYPE_F32) rows_generic_kernel<float, PAGED><<<grid, 64, 0, st>>>(a);
    else if (dtype == LLKV_DTYPE_F16) rows_generic_kernel<_Float16, PAGED><<<grid, 64, 0, st>>>(a);
    else rows_generic_kernel<bf16_t, PAGED><<<grid, 64, 0, st>>>(a);
    return check_launch(PAGED ? "llkv_paged_prefill" : "llkv_first_prefill_batched");
}

}  // namespace
}  // namespace llkv

using namespace llkv;

extern "C" size_t llkv_paged_prefill_workspace_size(int num_seqs, int total_q, int max_q_len,
                                                    int max_seq_len, int num_q_heads,
                                                    int head_dim, int block_size, int dtype) {
    return prefill_mfma_workspace(num_seqs, num_q_heads, head_dim, block_size, dtype, total_q,
                                  max_q_len, max_seq_len);
}

extern "C" int llkv_paged_prefill(void* out, const void* q, const void* k_pool,
                                  const void* v_pool, const int* block_table,
                                  int max_blocks_per_seq, const int* cu_q,
                                  const int* seq_lens, int num_seqs, int total_q,
                                  int max_q_len, int max_seq_len, int num_q_heads,
                                  int num_kv_heads, int head_dim, int block_size,
                                  int causal, float scale, int dtype, void* workspace,
                                  size_t workspace_bytes, void* stream) {
    const char* fn = "llkv_paged_prefill";
    if (num_seqs == 0 || total_q == 0) return LLKV_OK;
    if (num_seqs < 0 || total_q < 0 || num_q_heads <= 0 || num_kv_heads <= 0 ||
        head_dim <= 0 || block_size <= 0 || max_blocks_per_seq <= 0)
        return set_error(LLKV_ERR_INVALID, "%s: bad shape arguments", fn);
    if (head_dim > 256)
        return set_error(LLKV_ERR_UNSUPPORTED, "%s: head_dim too large (%d > 256)", fn, head_dim);
    if (num_q_heads % num_kv_heads != 0)
        return set_error(LLKV_ERR_INVALID, "%s: num_q_heads %d not a multiple of num_kv_heads %d",
                         fn, num_q_heads, num_kv_heads);
    if (dtype_bytes(dtype) == 0) return set_error(LLKV_ERR_INVALID, "%s: unsupported dtype %d", fn, dtype);
    if (!out || !q || !k_pool || !v_pool || !block_table || !cu_q || !seq_lens)
        return set_error(LLKV_ERR_INVALID, "%s: null pointer", fn);
    // token positions (max_blocks_per_seq * block_size) and table offsets are int on the device
    if ((int64_t)max_blocks_per_seq * block_size > INT32_MAX ||
        (int64_t)num_seqs * max_blocks_per_seq > INT32_MAX)
        return set_error(LLKV_ERR_UNSUPPORTED, "%s: block table too large", fn);
    hipStream_t st = (hipStream_t)stream;

    MfmaPrefillArgs m = {};
    m.out = out;
    m.q = q;
    m.k = k_pool;
    m.v = v_pool;
    m.bt = block_table;
    m.cu_q = cu_q;
    m.lens = seq_lens;
    m.max_blocks = max_blocks_per_seq;
    m.N = num_seqs;
    m.Hq = num_q_heads;
    m.Hkv = num_kv_heads;
    m.causal = causal;
    m.scale_log2 = scale * kLog2e;
    int r = launch_prefill_mfma(m, head_dim, block_size, dtype, total_q, max_q_len,
                                max_seq_len, workspace, workspace_bytes, st);
    if (r != -1) return r;   // -1: shape not covered by the MFMA kernel

    RowArgs a = {};
    a.out = out;
    a.q = q;
    a.k = k_pool;
    a.v = v_pool;
    a.bt = block_table;
    a.cu_q = cu_q;
    a.lens = seq_lens;
    a.max_blocks = max_blocks_per_seq;
    a.bs = block_size;
    a.N = num_seqs;
    a.Hq = num_q_heads;
    a.Hkv = num_kv_heads;
    a.D = head_dim;
    a.causal = causal;
    a.scale_log2 = scale * kLog2e;
    return launch_rows<true>(a, total_q, dtype, st);
}

extern "C" int llkv_first_prefill_batched(void* out, const void* q, const void* k,
                                          const void* v, int num_q_heads, int num_kv_heads,
                                          int head_dim, const int* offsets,
                                          const int* kv_offsets, const int* num_tokens,
                                          const int* token_cumsum, const int* start_poss,
                                          int N, int P_total, int max_tokens, float scale,
                                          int dtype, void* stream) {
    (void)start_poss;   // causal test start+pos <= start+local reduces to pos <= local
    const char* fn = "llkv_first_prefill_batched";
    if (N == 0 || P_total == 0) return LLKV_OK;
    if (N < 0 || P_total < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0)
        return set_error(LLKV_ERR_INVALID, "%s: bad shape arguments", fn);
    if (head_dim > 256)
        return set_error(LLKV_ERR_UNSUPPORTED, "%s: head_dim too large (%d > 256)", fn, head_dim);
    if (num_q_heads % num_kv_heads != 0)
        return set_error(LLKV_ERR_INVALID, "%s: num_q_heads not a multiple of num_kv_heads", fn);
    if (dtype_bytes(dtype) == 0) return set_error(LLKV_ERR_INVALID, "%s: unsupported dtype %d", fn, dtype);
    if (!out || !q || !k || !v || !offsets || !kv_offsets || !num_tokens || !token_cumsum)
        return set_error(LLKV_ERR_INVALID, "%s: null pointer", fn);
    const int bound = (max_tokens > 0 && max_tokens < P_total) ? max_tokens : P_total;
    MfmaPrefillArgs m = {};
    m.out = out;
    m.q = q;
    m.k = k;
    m.v = v;
    m.N = N;
    m.Hq = num_q_heads;
    m.Hkv = num_kv_heads;
    m.causal = 1;
    m.scale_log2 = scale * kLog2e;
    m.contig = 1;
    m.q_off = offsets;
    m.kv_off = kv_offsets;
    m.ntok = num_tokens;
    m.tcum = token_cumsum;
    m.q_row = num_q_heads * head_dim;
    const int r = launch_prefill_mfma(m, head_dim, kPage, dtype, P_total, bound, bound, nullptr, 0,
                                      (hipStream_t)stream);
    if (r != -1) return r;   // -1: shape not covered by the MFMA kernels

    RowArgs a = {};
    a.out = out;
    a.q = q;
    a.k = k;
    a.v = v;
    a.offsets = offsets;
    a.kv_offsets = kv_offsets;
    a.num_tokens = num_tokens;
    a.token_cumsum = token_cumsum;
    a.N = N;
    a.Hq = num_q_heads;
    a.Hkv = num_kv_heads;
    a.D = head_dim;
    a.scale_log2 = scale * kLog2e;
    return launch_rows<false>(a, P_total, dtype, (hipStream_t)stream);
}
