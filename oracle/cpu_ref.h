/*
 * CPU oracle for the paged KV-cache hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links or calls
 * this code; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it, and only as the checker / the CPU baseline.
 *
 * Every function restates an algorithm from the reference
 * (wjb554/lightllm) and cites the file:line it follows.  Layout of a
 * paged pool, as in the reference (include/lightllm/kv_cache/block_allocator.h:149-150):
 *     K, V : [num_blocks, block_size, Hkv, D]   row-major
 *     slot = phys * block_size + pos % block_size,  phys = table[pos / block_size]
 *
 *
 * Pinning (what each function is checked against, tests/test_oracle.py unless noted):
 *   llo_fill_random, llo_rng_randf_fill   closed-form LCG known answers
 *   llo_f32_to_f16 / llo_f16_to_f32       numpy float16 casts (RNE, subnormals, ties, overflow)
 *   llo_f32_to_bf16 / llo_bf16_to_f32     torch bfloat16 casts (RNE, ties)
 *   llo_append_slots, llo_scatter_prefill, llo_scatter_prefill_batched, llo_reconstruct_kv
 *                                         numpy fancy indexing of the pool, bit-exact;
 *                                         append-then-gather identity
 *   llo_cpu_attention[_f64], llo_paged_decode[_f64]
 *                                         numpy float64 softmax attention; closed forms
 *                                         (one key -> V[0], equal keys -> mean V, length 0
 *                                         -> zeros); convex hull; the reference's ramp
 *                                         known-answer inputs (tests/test_paged_attention.cu:69-130)
 *   llo_splitk_partials, llo_splitk_merge unsplit result for S in {1,2,4,16,40}; a hand-built
 *                                         two-split + identity-split merge
 *   llo_prefill_attention[_f64], llo_prefill_attention_test_causal
 *                                         numpy masked softmax; pure-Python brute force on
 *                                         P <= 4, L <= 48; test-file causal form equals the
 *                                         kernel form when total = hist + P
 *   llo_paged_prefill[_f64]               numpy per-sequence gather + masked softmax
 *   llo_first_prefill_batched             numpy per-entry causal softmax
 *   llo_fnv1a_tokens                      published FNV-1a 64 vectors ("", "a", "abc")
 *   llo_build_slots                       pure-Python position walk; decode form (cu = 0..B,
 *                                         start = lengths) equals table[len/16]*16 + len%16
 *   llo_rope_append                       numpy float32 rotation (separately rounded products
 *                                         and sums), bit-exact for fp32 / fp16 / bf16; the
 *                                         reference's own rope known answer (tests/test_ops.cu:51-61);
 *                                         rotation by angle 0 is the identity, cos/sin of a
 *                                         true angle preserve each pair's norm
 * No function is left unpinned.
 */
#ifndef LIGHTLLM_ORACLE_CPU_REF_H
#define LIGHTLLM_ORACLE_CPU_REF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- deterministic generators ------------------------------------------ */
void llo_fill_random(float* v, size_t n, unsigned seed);
void llo_rng_randf_fill(float* v, size_t n, uint32_t* state);

/* ---- fp16 / bf16 rounding (round-to-nearest-even) ----------------------- */
uint16_t llo_f32_to_f16(float x);
float llo_f16_to_f32(uint16_t h);
uint16_t llo_f32_to_bf16(float x);
float llo_bf16_to_f32(uint16_t h);
void llo_f32_to_f16_array(const float* src, uint16_t* dst, size_t n);
void llo_f16_to_f32_array(const uint16_t* src, float* dst, size_t n);
void llo_f32_to_bf16_array(const float* src, uint16_t* dst, size_t n);
void llo_bf16_to_f32_array(const uint16_t* src, float* dst, size_t n);

/* ---- KV append / gather (pure copies, any element size) ----------------- */
void llo_append_slots(void* k_pool, void* v_pool, const void* k_src,
                      const void* v_src, const int64_t* slot_mapping,
                      int64_t n_tokens, int Hkv, int D, int elem_size);
void llo_scatter_prefill(void* k_pool, void* v_pool, const void* k_src,
                         const void* v_src, int start_pos, int n_tokens,
                         const int* block_table, int block_size, int Hkv,
                         int D, int elem_size);
void llo_scatter_prefill_batched(void* k_pool, void* v_pool,
                                 const void* k_flat, const void* v_flat,
                                 int Hkv, int D, const int* kv_offsets,
                                 const int* start_poss,
                                 const int* token_cumsum, const int* flat_bt,
                                 int max_blocks, int N, int block_size,
                                 int elem_size);
void llo_build_slots(int64_t* slots, const int* block_table, int max_blocks,
                     const int* cu, const int* start_pos, int n, int num_tokens,
                     int block_size);
void llo_rope_append(void* q, void* k, const void* v, void* k_pool, void* v_pool,
                     const int64_t* slot_mapping, const float* cos, const float* sin,
                     int T, int Hq, int Hkv, int D, int rotary_dim, int dtype);
void llo_reconstruct_kv(void* k_out, void* v_out, const void* k_pool,
                        const void* v_pool, const int* block_table,
                        int seq_len, int block_size, int Hkv, int D,
                        int elem_size);

/* ---- decode attention over contiguous K/V ------------------------------- */
void llo_cpu_attention(const float* q, int T, int Hq, int D,
                       const float* k, int seq_len, int Hkv, const float* v,
                       float* out);
void llo_cpu_attention_f64(const float* q, int T, int Hq, int D,
                           const float* k, int seq_len, int Hkv,
                           const float* v, double* out);

/* ---- batched paged decode (gather + attention per sequence) ------------- */
void llo_paged_decode(const float* q, const float* k_pool,
                      const float* v_pool, const int* block_table,
                      const int* seq_lens, int B, int Hq, int Hkv, int D,
                      int block_size, int max_blocks, float* out,
                      int nthreads);
void llo_paged_decode_f64(const float* q, const float* k_pool,
                          const float* v_pool, const int* block_table,
                          const int* seq_lens, int B, int Hq, int Hkv, int D,
                          int block_size, int max_blocks, double* out,
                          int nthreads);

/* ---- Split-K partials and log-sum-exp merge ----------------------------- */
void llo_splitk_partials(const float* q, const float* k_pool,
                         const float* v_pool, const int* block_table,
                         const int* seq_lens, int B, int Hq, int Hkv, int D,
                         int block_size, int max_blocks, int num_splits,
                         float* partial);
void llo_splitk_merge(const float* partial, int B, int Hq, int D,
                      int num_splits, float* out);

/* ---- prefill attention over contiguous K/V ------------------------------ */
void llo_prefill_attention(const float* q, int P, int Hq, int D,
                           const float* k, int total_seq, int Hkv,
                           const float* v, int causal, float* out);
void llo_prefill_attention_f64(const float* q, int P, int Hq, int D,
                               const float* k, int total_seq, int Hkv,
                               const float* v, int causal, double* out);
void llo_prefill_attention_test_causal(const float* q, int P, int Hq, int D,
                                       const float* k, int seq_len, int Hkv,
                                       const float* v, float* out);

/* ---- paged prefill (gather + prefill attention), varlen over sequences -- */
void llo_paged_prefill(const float* q, const int* cu_q, const float* k_pool,
                       const float* v_pool, const int* block_table,
                       const int* seq_lens, int N, int Hq, int Hkv, int D,
                       int block_size, int max_blocks, int causal,
                       float* out, int nthreads);
void llo_paged_prefill_f64(const float* q, const int* cu_q,
                           const float* k_pool, const float* v_pool,
                           const int* block_table, const int* seq_lens, int N,
                           int Hq, int Hkv, int D, int block_size,
                           int max_blocks, int causal, double* out,
                           int nthreads);

/* ---- batched first-prefill over contiguous K/V -------------------------- */
void llo_first_prefill_batched(float* out, const float* q, const float* k,
                               const float* v, int Hq, int Hkv, int D,
                               const int* offsets, const int* kv_offsets,
                               const int* num_tokens,
                               const int* token_cumsum, const int* start_poss,
                               int N, int P_total, float scale);

/* ---- prefix cache hash ---------------------------------------------------- */
uint64_t llo_fnv1a_tokens(const int* tokens, int n);

int llo_omp_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
