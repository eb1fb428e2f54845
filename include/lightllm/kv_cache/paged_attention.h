#pragma once
/// Paged KV-cache operators for the MI355X build -- the reference's operator
/// API (include/lightllm/kv_cache/paged_attention.h:31-145 of
/// wjb554/lightllm) with identical signatures, so EngineServer::step and the
/// reference's tests call them unchanged.  Implemented over the C ABI in
/// lightllm_kv.h (gfx950 HIP kernels).
///
/// Conventions kept from the reference:
///  * attention returns a new Tensor of q's dtype; q's dtype must equal the
///    pool dtype (checked here; the reference left it undefined);
///  * block_table / seq_lens / seq_len_ptr are caller-owned device int32;
///  * scale = 1/sqrt(head_dim) for decode and paged prefill;
///  * head_dim > 256 throws std::runtime_error;
///  * the decode and prefill dispatchers read the lengths back to the host
///    (as the reference does, :555-560, :1036-1037) to size the launch; the
///    C ABI takes host-side bounds instead and never synchronises.
/// Extensions (new, additive): append_kv_slots (slot-mapping append),
/// paged_prefill_varlen (N sequences in one launch), build_slots (device slot
/// mapping of a step), rope_append_kv (fused RoPE + KV append) and
/// paged_attention_append (fused KV append + decode).

#include <cstdint>

#include "lightllm/tensor.h"

namespace lightllm {
namespace kv_cache {

class BlockAllocator;

Tensor paged_attention(const Tensor& q, const int* block_table, int max_blocks_per_seq,
                       const int* seq_lens, BlockAllocator& allocator);

Tensor prefill_paged_attention(const Tensor& q, const int* block_table, int max_blocks,
                               const int* seq_len_ptr, BlockAllocator& allocator,
                               bool causal = false);

void scatter_prefill_kv_gpu(const Tensor& k_contig, const Tensor& v_contig, int start_pos,
                            int n_tokens, const int* block_table, int max_blocks,
                            BlockAllocator& allocator);

void scatter_prefill_kv_batched_gpu(const float* k_flat_ptr, const float* v_flat_ptr, int Hkv,
                                    int D, const int* kv_offsets, const int* num_tokens,
                                    const int* start_poss, const int* token_cumsum,
                                    const int* flat_bt, int max_blocks, int N, int P_total,
                                    BlockAllocator& allocator);

void scatter_prefill_kv_batched_gpu_dispatch(DType dtype, const void* k_flat_ptr,
                                             const void* v_flat_ptr, int Hkv, int D,
                                             const int* kv_offsets, const int* num_tokens,
                                             const int* start_poss, const int* token_cumsum,
                                             const int* flat_bt, int max_blocks, int N,
                                             int P_total, BlockAllocator& allocator);

void first_prefill_attn_batched_gpu(float* out_ptr, const float* q_ptr, const float* k_ptr,
                                    const float* v_ptr, int Hq, int Hkv, int D,
                                    const int* offsets, const int* kv_offsets,
                                    const int* num_tokens, const int* token_cumsum,
                                    const int* start_poss, int N, int P_total, float scale);

void first_prefill_attn_batched_gpu_dispatch(DType dtype, void* out_ptr, const void* q_ptr,
                                             const void* k_ptr, const void* v_ptr, int Hq,
                                             int Hkv, int D, const int* offsets,
                                             const int* kv_offsets, const int* num_tokens,
                                             const int* token_cumsum, const int* start_poss,
                                             int N, int P_total, float scale);

// ---- additive extensions -------------------------------------------------

/// KV append by slot mapping: row i of k/v ([n, Hkv, D], pool dtype) goes to
/// pool row slot_mapping[i] (device int64; negative = skip).
void append_kv_slots(const Tensor& k, const Tensor& v, const int64_t* slot_mapping,
                     BlockAllocator& allocator);

/// Fused KV append + decode: k_new / v_new ([T, Hkv, D], pool dtype) are appended at
/// position seq_lens[b] - 1 of each sequence (the lengths count the new token), then
/// decode attention as paged_attention.  Equal to the append followed by paged_attention.
Tensor paged_attention_append(const Tensor& q, const Tensor& k_new, const Tensor& v_new,
                              const int* block_table, int max_blocks_per_seq, const int* seq_lens,
                              BlockAllocator& allocator);

/// Slot mapping of a step on the device (the per-token host loops of
/// EngineServer::scatter_prefill_kv / write_decode_kv, engine_server.cpp:731-787):
/// token t of sequence n (rows cu_tokens[n]..) sits at start_pos[n] + t - cu_tokens[n];
/// slots[t] = table[n][pos / bs] * bs + pos % bs, or -1 outside the table.  All
/// pointers are device memory; bs is the allocator's block size.
void build_slots(int64_t* slots, const int* block_table, int max_blocks, const int* cu_tokens,
                 const int* start_pos, int num_seqs, int num_tokens, const BlockAllocator& allocator);

/// Fused RoPE + KV append: lightllm::ops::rope(q, &k, cos, sin) (ops/rope.h:8-13,
/// Neox halves of the first 2 * cos.size(1) dims) followed by the append of the
/// rotated k and of v at slot_mapping (device int64; negative = skip).  q may be
/// null; q, k, v have the pool dtype; cos / sin are fp32 [T, rotary_dim / 2].
void rope_append_kv(Tensor* q, Tensor& k, const Tensor& v, const int64_t* slot_mapping,
                    const Tensor& cos, const Tensor& sin, BlockAllocator& allocator);

/// Varlen paged prefill: q [total_q, Hq, D]; cu_q device int32 [N+1];
/// seq_lens device int32 [N]; block_table [N, max_blocks].  Host bounds
/// max_q_len / max_seq_len size the launch (no device read-back).
Tensor paged_prefill_varlen(const Tensor& q, const int* block_table, int max_blocks,
                            const int* cu_q, const int* seq_lens, int num_seqs, int max_q_len,
                            int max_seq_len, BlockAllocator& allocator, bool causal);

}  // namespace kv_cache
}  // namespace lightllm
