// KV append (slot mapping), chunk scatter, batched scatter and block-table
// gather for gfx950.
//
// All four are pure row copies between a contiguous [rows, Hkv, D] buffer and
// the paged pool [num_blocks, block_size, Hkv, D]; only the row mapping
// differs.  Copies move the widest naturally aligned unit (16 B when the row
// size allows it, i.e. global_load/store_dwordx4), one unit per lane, with a
// flat grid-stride loop, so a wave reads/writes 1 KiB contiguous runs and the
// bits are moved unchanged (bit-exact for every dtype).
#include <hip/hip_runtime.h>

#include "common.h"

namespace llkv {
namespace {

// Row maps: given a row index, produce source/destination byte offsets.
struct SlotMap {  // append: src row i -> pool row slot[i]
    const int64_t* slots;
    int64_t row_bytes;
    __device__ bool operator()(int64_t i, int64_t& s, int64_t& d) const {
        int64_t slot = slots[i];
        s = i * row_bytes;
        d = slot * row_bytes;
        return slot >= 0;
    }
};

struct ChunkMap {  // scatter_prefill: chunk token t -> position start + t
    const int* table;
    int start_pos, block_size;
    int64_t row_bytes;
    __device__ bool operator()(int64_t t, int64_t& s, int64_t& d) const {
        int pos = start_pos + (int)t;
        int64_t phys = table[pos / block_size];
        s = t * row_bytes;
        d = (phys * block_size + pos % block_size) * row_bytes;
        return phys >= 0;
    }
};

__device__ inline int find_entry(const int* cum, int n, int g) {
    // largest e in [0, n) with cum[e] <= g
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (cum[mid] <= g) lo = mid; else hi = mid - 1;
    }
    return lo;
}

struct BatchedMap {  // scatter_prefill_batched
    const int* kv_offsets;
    const int* start_poss;
    const int* token_cumsum;
    const int* flat_bt;
    int N, max_blocks, block_size, esize;
    int64_t row_bytes;
    __device__ bool operator()(int64_t g, int64_t& s, int64_t& d) const {
        int e = find_entry(token_cumsum, N, (int)g);
        int local = (int)g - token_cumsum[e];
        int pos = start_poss[e] + local;
        if (pos < 0 || pos / block_size >= max_blocks) return false;   // outside the table
        int64_t phys = flat_bt[(int64_t)e * max_blocks + pos / block_size];
        s = (int64_t)kv_offsets[e] * esize + (int64_t)local * row_bytes;
        d = (phys * block_size + pos % block_size) * row_bytes;
        return phys >= 0;
    }
};

struct GatherMap {  // gather: output row g -> pool row of its (seq, pos)
    const int* table;
    const int* cu_seqlens;
    int B, max_blocks, block_size;
    int64_t row_bytes;
    __device__ bool operator()(int64_t g, int64_t& s, int64_t& d) const {
        int b = find_entry(cu_seqlens, B, (int)g);
        int pos = (int)g - cu_seqlens[b];
        if (pos < 0 || pos / block_size >= max_blocks) return false;   // outside the table
        int64_t phys = table[(int64_t)b * max_blocks + pos / block_size];
        s = (phys * block_size + pos % block_size) * row_bytes;
        d = g * row_bytes;
        return phys >= 0;
    }
};

template <typename U, typename Map>
__global__ __launch_bounds__(256) void copy_rows_kernel(
    Map map, char* __restrict__ k_dst, char* __restrict__ v_dst,
    const char* __restrict__ k_src, const char* __restrict__ v_src,
    int64_t n_rows, int units_per_row) {
    const int64_t total = n_rows * units_per_row;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += stride) {
        int64_t row = i / units_per_row;
        int c = (int)(i - row * units_per_row);
        int64_t s, d;
        if (!map(row, s, d)) continue;
        const int64_t off = (int64_t)c * sizeof(U);
        U kv = *reinterpret_cast<const U*>(k_src + s + off);
        U vv = *reinterpret_cast<const U*>(v_src + s + off);
        *reinterpret_cast<U*>(k_dst + d + off) = kv;
        *reinterpret_cast<U*>(v_dst + d + off) = vv;
    }
}

int unit_for(int64_t row_bytes, const void* a, const void* b, const void* c,
             const void* d) {
    uintptr_t m = (uintptr_t)a | (uintptr_t)b | (uintptr_t)c | (uintptr_t)d |
                  (uintptr_t)row_bytes;
    if ((m & 15) == 0) return 16;
    if ((m & 7) == 0) return 8;
    if ((m & 3) == 0) return 4;
    return 2;
}

template <typename Map>
int launch_copy(const char* what, Map map, void* kd, void* vd, const void* ks,
                const void* vs, int64_t n_rows, int64_t row_bytes, int unit,
                hipStream_t st) {
    if (n_rows <= 0) return LLKV_OK;
    int upr = (int)(row_bytes / unit);
    int64_t total = n_rows * upr;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 256 * 64) blocks = 256 * 64;   // grid-stride beyond ~64 WG/CU
    dim3 grid((unsigned)blocks), block(256);
    char* k_d = (char*)kd;
    char* v_d = (char*)vd;
    const char* k_s = (const char*)ks;
    const char* v_s = (const char*)vs;
    switch (unit) {
        case 16: copy_rows_kernel<uint4><<<grid, block, 0, st>>>(map, k_d, v_d, k_s, v_s, n_rows, upr); break;
        case 8: copy_rows_kernel<uint2><<<grid, block, 0, st>>>(map, k_d, v_d, k_s, v_s, n_rows, upr); break;
        case 4: copy_rows_kernel<uint32_t><<<grid, block, 0, st>>>(map, k_d, v_d, k_s, v_s, n_rows, upr); break;
        default: copy_rows_kernel<uint16_t><<<grid, block, 0, st>>>(map, k_d, v_d, k_s, v_s, n_rows, upr); break;
    }
    return check_launch(what);
}

int check_common(const char* what, int Hkv, int D, int dtype) {
    if (Hkv <= 0 || D <= 0)
        return set_error(LLKV_ERR_INVALID, "%s: num_kv_heads and head_dim must be positive", what);
    if (dtype_bytes(dtype) == 0)
        return set_error(LLKV_ERR_INVALID, "%s: unsupported dtype %d", what, dtype);
    return LLKV_OK;
}

}  // namespace
}  // namespace llkv

using namespace llkv;

extern "C" int llkv_append(void* k_pool, void* v_pool, const void* k_src,
                           const void* v_src, const int64_t* slot_mapping,
                           int64_t n_tokens, int num_kv_heads, int head_dim,
                           int dtype, void* stream) {
    if (int st = check_common("llkv_append", num_kv_heads, head_dim, dtype)) return st;
    if (n_tokens < 0) return set_error(LLKV_ERR_INVALID, "llkv_append: n_tokens < 0");
    if (n_tokens == 0) return LLKV_OK;
    if (!k_pool || !v_pool || !k_src || !v_src || !slot_mapping)
        return set_error(LLKV_ERR_INVALID, "llkv_append: null pointer");
    int64_t rb = (int64_t)num_kv_heads * head_dim * dtype_bytes(dtype);
    SlotMap m{slot_mapping, rb};
    return launch_copy("llkv_append", m, k_pool, v_pool, k_src, v_src, n_tokens, rb,
                       unit_for(rb, k_pool, v_pool, k_src, v_src), (hipStream_t)stream);
}

extern "C" int llkv_scatter_prefill(void* k_pool, void* v_pool, const void* k_src,
                                    const void* v_src, int start_pos, int n_tokens,
                                    const int* block_table, int max_blocks,
                                    int num_kv_heads, int head_dim, int block_size,
                                    int dtype, void* stream) {
    if (int st = check_common("llkv_scatter_prefill", num_kv_heads, head_dim, dtype)) return st;
    if (n_tokens <= 0) return LLKV_OK;
    if (start_pos < 0 || block_size <= 0)
        return set_error(LLKV_ERR_INVALID, "llkv_scatter_prefill: bad start_pos/block_size");
    if (max_blocks > 0 && (int64_t)(start_pos + n_tokens - 1) / block_size >= max_blocks)
        return set_error(LLKV_ERR_INVALID,
                         "llkv_scatter_prefill: positions [%d, %d) exceed max_blocks %d x %d",
                         start_pos, start_pos + n_tokens, max_blocks, block_size);
    if (!k_pool || !v_pool || !k_src || !v_src || !block_table)
        return set_error(LLKV_ERR_INVALID, "llkv_scatter_prefill: null pointer");
    int64_t rb = (int64_t)num_kv_heads * head_dim * dtype_bytes(dtype);
    ChunkMap m{block_table, start_pos, block_size, rb};
    return launch_copy("llkv_scatter_prefill", m, k_pool, v_pool, k_src, v_src, n_tokens,
                       rb, unit_for(rb, k_pool, v_pool, k_src, v_src), (hipStream_t)stream);
}

extern "C" int llkv_scatter_prefill_batched(void* k_pool, void* v_pool,
                                            const void* k_flat, const void* v_flat,
                                            int num_kv_heads, int head_dim,
                                            const int* kv_offsets, const int* num_tokens,
                                            const int* start_poss, const int* token_cumsum,
                                            const int* flat_bt, int max_blocks, int N,
                                            int P_total, int block_size, int dtype,
                                            void* stream) {
    (void)num_tokens;
    if (int st = check_common("llkv_scatter_prefill_batched", num_kv_heads, head_dim, dtype)) return st;
    if (P_total <= 0 || N <= 0) return LLKV_OK;
    if (block_size <= 0 || max_blocks <= 0)
        return set_error(LLKV_ERR_INVALID, "llkv_scatter_prefill_batched: bad block_size/max_blocks");
    if (!k_pool || !v_pool || !k_flat || !v_flat || !kv_offsets || !start_poss ||
        !token_cumsum || !flat_bt)
        return set_error(LLKV_ERR_INVALID, "llkv_scatter_prefill_batched: null pointer");
    int es = (int)dtype_bytes(dtype);
    int64_t rb = (int64_t)num_kv_heads * head_dim * es;
    BatchedMap m{kv_offsets, start_poss, token_cumsum, flat_bt, N, max_blocks, block_size, es, rb};
    // kv_offsets are element offsets; the copy unit never exceeds one element
    // multiple of the row, which kv_offsets that are multiples of Hkv*D satisfy.
    return launch_copy("llkv_scatter_prefill_batched", m, k_pool, v_pool, k_flat, v_flat,
                       P_total, rb, unit_for(rb, k_pool, v_pool, k_flat, v_flat),
                       (hipStream_t)stream);
}

extern "C" int llkv_gather(void* k_dst, void* v_dst, const void* k_pool,
                           const void* v_pool, const int* block_table, int max_blocks,
                           const int* cu_seqlens, int num_seqs, int64_t total_tokens,
                           int num_kv_heads, int head_dim, int block_size, int dtype,
                           void* stream) {
    if (int st = check_common("llkv_gather", num_kv_heads, head_dim, dtype)) return st;
    if (total_tokens <= 0 || num_seqs <= 0) return LLKV_OK;
    if (block_size <= 0 || max_blocks <= 0)
        return set_error(LLKV_ERR_INVALID, "llkv_gather: bad block_size/max_blocks");
    if (!k_dst || !v_dst || !k_pool || !v_pool || !block_table || !cu_seqlens)
        return set_error(LLKV_ERR_INVALID, "llkv_gather: null pointer");
    int64_t rb = (int64_t)num_kv_heads * head_dim * dtype_bytes(dtype);
    GatherMap m{block_table, cu_seqlens, num_seqs, max_blocks, block_size, rb};
    return launch_copy("llkv_gather", m, k_dst, v_dst, k_pool, v_pool, total_tokens, rb,
                       unit_for(rb, k_dst, v_dst, k_pool, v_pool), (hipStream_t)stream);
}
