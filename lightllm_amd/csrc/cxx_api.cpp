// lightllm::kv_cache operator API (reference signatures,
// include/lightllm/kv_cache/paged_attention.h:31-145) implemented over the
// C ABI.  Errors from the ABI become std::runtime_error, as the reference
// throws for unsupported head_dim / dtype.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <stdexcept>
#include <string>
#include <vector>

#include "lightllm/kv_cache/block_allocator.h"
#include "lightllm/kv_cache/paged_attention.h"
#include "lightllm_kv.h"

namespace lightllm {
namespace kv_cache {

namespace {

void throw_if(int status, const char* what) {
    if (status != LLKV_OK)
        throw std::runtime_error(std::string(what) + ": " + llkv_last_error());
}

void hip_throw(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// Per-thread device scratch, grown on demand and kept for the thread's life,
// so repeated decode calls do not allocate.
struct Scratch {
    void* ptr = nullptr;
    size_t bytes = 0;
    ~Scratch() {
        if (ptr) (void)hipFree(ptr);
    }
    void* get(size_t need) {
        if (need <= bytes) return ptr;
        if (ptr) hip_throw(hipFree(ptr), "hipFree");
        ptr = nullptr;
        bytes = 0;
        hip_throw(hipMalloc(&ptr, need), "hipMalloc(workspace)");
        bytes = need;
        return ptr;
    }
};
thread_local Scratch t_workspace;
thread_local Scratch t_meta;

void require_pool_dtype(DType d, const BlockAllocator& a, const char* what) {
    if (d != a.kv_dtype())
        throw std::runtime_error(std::string(what) + ": tensor dtype " + dtype_name(d) +
                                 " differs from the pool dtype " + dtype_name(a.kv_dtype()));
}

void require_device_pool(const BlockAllocator& a, const char* what) {
    if (a.storage() != PoolStorage::Device || a.k_storage_raw() == nullptr)
        throw std::runtime_error(std::string(what) + ": allocator has no device pools");
}

int host_max(const int* dev, int n) {
    if (n <= 0) return 0;
    std::vector<int> h(static_cast<size_t>(n));
    hip_throw(hipMemcpy(h.data(), dev, sizeof(int) * n, hipMemcpyDeviceToHost), "hipMemcpy(seq_lens)");
    return std::max(0, *std::max_element(h.begin(), h.end()));
}

}  // namespace

Tensor paged_attention(const Tensor& q, const int* block_table, int max_blocks_per_seq,
                       const int* seq_lens, BlockAllocator& allocator) {
    const int T = q.size(0), Hq = q.size(1), D = q.size(2);
    if (D > 256) throw std::runtime_error("paged_attention: head_dim too large");
    require_pool_dtype(q.dtype(), allocator, "paged_attention");
    require_device_pool(allocator, "paged_attention");
    Tensor out({T, Hq, D}, q.dtype(), Device::CUDA);
    if (T == 0) return out;
    const int Hkv = allocator.num_kv_heads();
    const int bs = allocator.block_size();
    // The reference reads seq_lens back here too (paged_attention.cu:555-560).
    const int max_len = host_max(seq_lens, T);
    const size_t ws = llkv_paged_decode_workspace_size(T, Hq, Hkv, D, bs, max_len, 0);
    void* w = ws ? t_workspace.get(ws) : nullptr;
    throw_if(llkv_paged_decode(out.raw(), q.raw(), allocator.k_storage_raw(), allocator.v_storage_raw(),
                               block_table, seq_lens, T, Hq, Hkv, D, bs, max_blocks_per_seq, max_len,
                               0, 1.0f / std::sqrt((float)D), static_cast<int>(q.dtype()), w, ws,
                               nullptr),
             "paged_attention");
    return out;
}

Tensor paged_attention_append(const Tensor& q, const Tensor& k_new, const Tensor& v_new,
                              const int* block_table, int max_blocks_per_seq, const int* seq_lens,
                              BlockAllocator& allocator) {
    const int T = q.size(0), Hq = q.size(1), D = q.size(2);
    if (D > 256) throw std::runtime_error("paged_attention_append: head_dim too large");
    require_pool_dtype(q.dtype(), allocator, "paged_attention_append");
    require_pool_dtype(k_new.dtype(), allocator, "paged_attention_append");
    require_pool_dtype(v_new.dtype(), allocator, "paged_attention_append");
    require_device_pool(allocator, "paged_attention_append");
    Tensor out({T, Hq, D}, q.dtype(), Device::CUDA);
    if (T == 0) return out;
    const int Hkv = allocator.num_kv_heads();
    const int bs = allocator.block_size();
    const int max_len = host_max(seq_lens, T);
    const size_t ws = llkv_paged_decode_workspace_size(T, Hq, Hkv, D, bs, max_len, 0);
    void* w = ws ? t_workspace.get(ws) : nullptr;
    throw_if(llkv_paged_decode_append(out.raw(), q.raw(), k_new.raw(), v_new.raw(),
                                      const_cast<void*>(allocator.k_storage_raw()),
                                      const_cast<void*>(allocator.v_storage_raw()), block_table,
                                      seq_lens, T, Hq, Hkv, D, bs, max_blocks_per_seq, max_len, 0,
                                      1.0f / std::sqrt((float)D), static_cast<int>(q.dtype()), w, ws,
                                      nullptr),
             "paged_attention_append");
    return out;
}

Tensor paged_prefill_varlen(const Tensor& q, const int* block_table, int max_blocks,
                            const int* cu_q, const int* seq_lens, int num_seqs, int max_q_len,
                            int max_seq_len, BlockAllocator& allocator, bool causal) {
    const int Ptot = q.size(0), Hq = q.size(1), D = q.size(2);
    if (D > 256) throw std::runtime_error("prefill_paged_attention: head_dim too large");
    require_pool_dtype(q.dtype(), allocator, "prefill_paged_attention");
    require_device_pool(allocator, "prefill_paged_attention");
    Tensor out({Ptot, Hq, D}, q.dtype(), Device::CUDA);
    if (Ptot == 0) return out;
    const size_t ws_bytes = llkv_paged_prefill_workspace_size(num_seqs, Ptot, max_q_len, max_seq_len, Hq,
                                                              D, allocator.block_size(),
                                                              static_cast<int>(q.dtype()));
    void* ws = ws_bytes ? t_workspace.get(ws_bytes) : nullptr;
    throw_if(llkv_paged_prefill(out.raw(), q.raw(), allocator.k_storage_raw(), allocator.v_storage_raw(),
                                block_table, max_blocks, cu_q, seq_lens, num_seqs, Ptot, max_q_len,
                                max_seq_len, Hq, allocator.num_kv_heads(), D, allocator.block_size(),
                                causal ? 1 : 0, 1.0f / std::sqrt((float)D),
                                static_cast<int>(q.dtype()), ws, ws_bytes, nullptr),
             "prefill_paged_attention");
    return out;
}

Tensor prefill_paged_attention(const Tensor& q, const int* block_table, int max_blocks,
                               const int* seq_len_ptr, BlockAllocator& allocator, bool causal) {
    const int P = q.size(0);
    // The reference reads total_seq back here too (paged_attention.cu:1036-1037).
    const int total = host_max(seq_len_ptr, 1);
    int* cu = static_cast<int*>(t_meta.get(2 * sizeof(int)));
    const int h_cu[2] = {0, P};
    hip_throw(hipMemcpy(cu, h_cu, sizeof(h_cu), hipMemcpyHostToDevice), "hipMemcpy(cu_q)");
    return paged_prefill_varlen(q, block_table, max_blocks, cu, seq_len_ptr, 1, P, total, allocator,
                                causal);
}

void scatter_prefill_kv_gpu(const Tensor& k_contig, const Tensor& v_contig, int start_pos,
                            int n_tokens, const int* block_table, int max_blocks,
                            BlockAllocator& allocator) {
    require_pool_dtype(k_contig.dtype(), allocator, "scatter_prefill_kv");
    require_pool_dtype(v_contig.dtype(), allocator, "scatter_prefill_kv");
    require_device_pool(allocator, "scatter_prefill_kv");
    throw_if(llkv_scatter_prefill(const_cast<void*>(allocator.k_storage_raw()),
                                  const_cast<void*>(allocator.v_storage_raw()), k_contig.raw(),
                                  v_contig.raw(), start_pos, n_tokens, block_table, max_blocks,
                                  allocator.num_kv_heads(), allocator.head_dim(),
                                  allocator.block_size(), static_cast<int>(k_contig.dtype()), nullptr),
             "scatter_prefill_kv");
}

void scatter_prefill_kv_batched_gpu_dispatch(DType dtype, const void* k_flat_ptr,
                                             const void* v_flat_ptr, int Hkv, int D,
                                             const int* kv_offsets, const int* num_tokens,
                                             const int* start_poss, const int* token_cumsum,
                                             const int* flat_bt, int max_blocks, int N,
                                             int P_total, BlockAllocator& allocator) {
    require_pool_dtype(dtype, allocator, "scatter_prefill_kv_batched");
    require_device_pool(allocator, "scatter_prefill_kv_batched");
    throw_if(llkv_scatter_prefill_batched(const_cast<void*>(allocator.k_storage_raw()),
                                          const_cast<void*>(allocator.v_storage_raw()), k_flat_ptr,
                                          v_flat_ptr, Hkv, D, kv_offsets, num_tokens, start_poss,
                                          token_cumsum, flat_bt, max_blocks, N, P_total,
                                          allocator.block_size(), static_cast<int>(dtype), nullptr),
             "scatter_prefill_kv_batched");
    // The reference synchronises the device after this launch (:1188, :1218).
    hip_throw(hipDeviceSynchronize(), "scatter_prefill_kv_batched");
}

void scatter_prefill_kv_batched_gpu(const float* k_flat_ptr, const float* v_flat_ptr, int Hkv,
                                    int D, const int* kv_offsets, const int* num_tokens,
                                    const int* start_poss, const int* token_cumsum,
                                    const int* flat_bt, int max_blocks, int N, int P_total,
                                    BlockAllocator& allocator) {
    scatter_prefill_kv_batched_gpu_dispatch(DType::F32, k_flat_ptr, v_flat_ptr, Hkv, D, kv_offsets,
                                            num_tokens, start_poss, token_cumsum, flat_bt,
                                            max_blocks, N, P_total, allocator);
}

void first_prefill_attn_batched_gpu_dispatch(DType dtype, void* out_ptr, const void* q_ptr,
                                             const void* k_ptr, const void* v_ptr, int Hq,
                                             int Hkv, int D, const int* offsets,
                                             const int* kv_offsets, const int* num_tokens,
                                             const int* token_cumsum, const int* start_poss,
                                             int N, int P_total, float scale) {
    if (D > 256) throw std::runtime_error("first_prefill_attn_batched: head_dim too large");
    // The longest entry (query rows token_cumsum[e + 1] - token_cumsum[e])
    // bounds the query blocks of the launch; P_total would launch mostly empty
    // work-groups.  One device-to-host read of N + 1 ints before the launch,
    // which the reference does not make; its call synchronises at the end.
    int max_tokens = 0;
    if (N > 0 && token_cumsum != nullptr) {
        std::vector<int> tc(N + 1);
        hip_throw(hipMemcpy(tc.data(), token_cumsum, (N + 1) * sizeof(int), hipMemcpyDeviceToHost),
                  "first_prefill_attn_batched");
        for (int e = 0; e < N; ++e) max_tokens = std::max(max_tokens, tc[e + 1] - tc[e]);
        if (max_tokens <= 0) max_tokens = P_total;
    }
    throw_if(llkv_first_prefill_batched(out_ptr, q_ptr, k_ptr, v_ptr, Hq, Hkv, D, offsets, kv_offsets,
                                        num_tokens, token_cumsum, start_poss, N, P_total, max_tokens,
                                        scale, static_cast<int>(dtype), nullptr),
             "first_prefill_attn_batched");
    // The reference synchronises the device after this launch (:1349, :1382).
    hip_throw(hipDeviceSynchronize(), "first_prefill_attn_batched");
}

void first_prefill_attn_batched_gpu(float* out_ptr, const float* q_ptr, const float* k_ptr,
                                    const float* v_ptr, int Hq, int Hkv, int D,
                                    const int* offsets, const int* kv_offsets,
                                    const int* num_tokens, const int* token_cumsum,
                                    const int* start_poss, int N, int P_total, float scale) {
    first_prefill_attn_batched_gpu_dispatch(DType::F32, out_ptr, q_ptr, k_ptr, v_ptr, Hq, Hkv, D,
                                            offsets, kv_offsets, num_tokens, token_cumsum,
                                            start_poss, N, P_total, scale);
}

void append_kv_slots(const Tensor& k, const Tensor& v, const int64_t* slot_mapping,
                     BlockAllocator& allocator) {
    require_pool_dtype(k.dtype(), allocator, "append_kv_slots");
    require_pool_dtype(v.dtype(), allocator, "append_kv_slots");
    require_device_pool(allocator, "append_kv_slots");
    throw_if(llkv_append(const_cast<void*>(allocator.k_storage_raw()),
                         const_cast<void*>(allocator.v_storage_raw()), k.raw(), v.raw(), slot_mapping,
                         k.size(0), allocator.num_kv_heads(), allocator.head_dim(),
                         static_cast<int>(k.dtype()), nullptr),
             "append_kv_slots");
}

void build_slots(int64_t* slots, const int* block_table, int max_blocks, const int* cu_tokens,
                 const int* start_pos, int num_seqs, int num_tokens, const BlockAllocator& allocator) {
    throw_if(llkv_build_slots(slots, block_table, max_blocks, cu_tokens, start_pos, num_seqs,
                              num_tokens, allocator.block_size(), nullptr),
             "build_slots");
}

void rope_append_kv(Tensor* q, Tensor& k, const Tensor& v, const int64_t* slot_mapping,
                    const Tensor& cos, const Tensor& sin, BlockAllocator& allocator) {
    if (q) require_pool_dtype(q->dtype(), allocator, "rope_append_kv");
    require_pool_dtype(k.dtype(), allocator, "rope_append_kv");
    require_pool_dtype(v.dtype(), allocator, "rope_append_kv");
    require_device_pool(allocator, "rope_append_kv");
    if (cos.dtype() != DType::F32 || sin.dtype() != DType::F32)
        throw std::runtime_error("rope_append_kv: cos / sin must be fp32");
    throw_if(llkv_rope_append(q ? q->raw() : nullptr, k.raw(), v.raw(),
                              const_cast<void*>(allocator.k_storage_raw()),
                              const_cast<void*>(allocator.v_storage_raw()), slot_mapping,
                              cos.data<float>(), sin.data<float>(), k.size(0), q ? q->size(1) : 0,
                              allocator.num_kv_heads(), allocator.head_dim(),
                              2 * static_cast<int>(cos.size(1)), static_cast<int>(k.dtype()), nullptr),
             "rope_append_kv");
}

}  // namespace kv_cache
}  // namespace lightllm
