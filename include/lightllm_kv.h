/*
 * lightllm_kv.h -- C ABI of the MI355X (gfx950) paged KV-cache hot path.
 *
 * Plain pointers and sizes only.  Device pointers are HIP device memory
 * (hipMalloc / torch on ROCm); `stream` is a hipStream_t passed as void*
 * (NULL = the null stream).  Every entry point returns 0 on success or a
 * non-zero llkv_status; llkv_last_error() gives a message for the calling
 * thread.  Entry points enqueue work on `stream` and do not synchronise,
 * except where noted.
 *
 * Pool layout (src/kv_cache/block_allocator.cpp:24-27 of the reference):
 *     K, V : [num_blocks, block_size, num_kv_heads, head_dim], row-major
 * A "slot" is the row index phys * block_size + pos % block_size, with
 * phys = block_table[pos / block_size].  Row offsets are 64-bit.
 *
 * Each function names the reference interface it replaces
 * (reference = wjb554/lightllm, paths relative to its root).
 */
#ifndef LIGHTLLM_KV_H
#define LIGHTLLM_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types; values equal lightllm::DType (include/lightllm/tensor.h:14). */
enum llkv_dtype {
    LLKV_DTYPE_F32 = 0,
    LLKV_DTYPE_F16 = 1,
    LLKV_DTYPE_BF16 = 2,
    LLKV_DTYPE_I32 = 3
};

enum llkv_status {
    LLKV_OK = 0,
    LLKV_ERR_INVALID = 1,     /* bad argument (shape, dtype, null pointer)  */
    LLKV_ERR_UNSUPPORTED = 2, /* e.g. head_dim > 256, as the reference      */
    LLKV_ERR_WORKSPACE = 3,   /* workspace too small                        */
    LLKV_ERR_HIP = 4,         /* a HIP runtime call or launch failed         */
    LLKV_ERR_EXHAUSTED = 5    /* block pool exhausted                        */
};

const char* llkv_last_error(void);
const char* llkv_status_string(int status);
/* ABI version: bumped on any signature change. */
int llkv_abi_version(void);

/* ------------------------------------------------------------------------
 * KV append by slot mapping.
 * Replaces EngineServer::write_decode_kv (src/engine/engine_server.cpp:760-787,
 * two cudaMemcpy per token per layer) and InferenceEngine::write_decode_kv
 * (src/engine/engine_paged.cpp:287-331).  Row i of k_src/v_src ([n_tokens,
 * Hkv, D], contiguous) is copied bit-exactly to pool row slot_mapping[i];
 * a negative slot is skipped.
 * ------------------------------------------------------------------------ */
int llkv_append(void* k_pool, void* v_pool, const void* k_src,
                const void* v_src, const int64_t* slot_mapping,
                int64_t n_tokens, int num_kv_heads, int head_dim, int dtype,
                void* stream);

/* Replaces scatter_prefill_kv_gpu (include/lightllm/kv_cache/paged_attention.h:95-102,
 * src/kv_cache/paged_attention.cu:1097-1124): token t of a chunk goes to
 * position start_pos + t of the sequence whose table is block_table. */
int llkv_scatter_prefill(void* k_pool, void* v_pool, const void* k_src,
                         const void* v_src, int start_pos, int n_tokens,
                         const int* block_table, int max_blocks,
                         int num_kv_heads, int head_dim, int block_size,
                         int dtype, void* stream);

/* Replaces scatter_prefill_kv_batched_gpu[_dispatch]
 * (include/lightllm/kv_cache/paged_attention.h:109-124,
 * src/kv_cache/paged_attention.cu:1134-1219).  num_tokens is accepted for
 * signature parity; token_cumsum[N+1] defines the entries.  All index arrays
 * are device int32.  Unlike the reference this does not synchronise. */
int llkv_scatter_prefill_batched(void* k_pool, void* v_pool,
                                 const void* k_flat, const void* v_flat,
                                 int num_kv_heads, int head_dim,
                                 const int* kv_offsets, const int* num_tokens,
                                 const int* start_poss,
                                 const int* token_cumsum, const int* flat_bt,
                                 int max_blocks, int N, int P_total,
                                 int block_size, int dtype, void* stream);

/* Block-table gather: the device form of reconstruct_kv
 * (tests/test_paged_attention_v2.cu:219-239) and of the tile gather inside
 * every reference kernel (load_tile_float4, src/kv_cache/paged_attention.cu:46-98).
 * Sequence b's positions [0, cu_seqlens[b+1]-cu_seqlens[b]) are written to
 * rows cu_seqlens[b].. of k_dst/v_dst ([total_tokens, Hkv, D]).
 * cu_seqlens is device int32 [B+1]; block_table is [B, max_blocks]. */
int llkv_gather(void* k_dst, void* v_dst, const void* k_pool,
                const void* v_pool, const int* block_table, int max_blocks,
                const int* cu_seqlens, int num_seqs, int64_t total_tokens,
                int num_kv_heads, int head_dim, int block_size, int dtype,
                void* stream);

/* ------------------------------------------------------------------------
 * Device-side step metadata and fused RoPE + KV append (the next rows of the
 * path: the engine's per-token host loops and memcpys, and its separate RoPE
 * pass, become two launches per layer).
 * ------------------------------------------------------------------------ */

/* Slot mapping built on the device.  Replaces the host loops of
 * EngineServer::scatter_prefill_kv (src/engine/engine_server.cpp:731-757) and
 * write_decode_kv (:760-787), which look up phys = block_table[pos / bs] and
 * offset = pos % bs per token and issue two cudaMemcpy each.  Token t of
 * sequence n (rows cu_tokens[n] .. cu_tokens[n+1]-1) sits at position
 * start_pos[n] + (t - cu_tokens[n]); slots[t] = phys * bs + pos % bs, or -1
 * when the position lies outside the table or on a -1 entry (the reference
 * skips such a write, :766-774).  A decode step is cu_tokens = 0..B,
 * start_pos = seq_lens.  block_table: device int32 [num_seqs, max_blocks];
 * cu_tokens: device int32 [num_seqs + 1]; start_pos: device int32 [num_seqs];
 * slots: device int64 [num_tokens]. */
int llkv_build_slots(int64_t* slots, const int* block_table, int max_blocks,
                     const int* cu_tokens, const int* start_pos, int num_seqs,
                     int num_tokens, int block_size, void* stream);

/* Fused RoPE + KV append.  Replaces lightllm::ops::rope
 * (include/lightllm/ops/rope.h:8-13, src/ops/rope.cu:29-92) on q and k,
 * followed by write_decode_kv / scatter_prefill_kv.  Neox rotation of the first
 * rotary_dim dims of every head, pairs (i, i + rotary_dim/2):
 *     x1' = x1 * cos[t][i] - x2 * sin[t][i]
 *     x2' = x2 * cos[t][i] + x1 * sin[t][i]
 * in fp32 with each product and the sum rounded separately (no fused
 * multiply-add), then rounded to the element type.  Dims >= rotary_dim are
 * unchanged.  q [num_tokens, Hq, D] (may be NULL) and k [num_tokens, Hkv, D]
 * are rotated in place; the rotated k row and the v row are then written to
 * pool row slot_mapping[t] (negative = no pool write).  cos, sin: device fp32
 * [num_tokens, rotary_dim / 2], as the reference builds them
 * (engine_server.cpp:1553-1585).  rotary_dim even, 2 <= rotary_dim <= D.
 * The reference kernel's indexing rotates a single pair per (token, head)
 * when its block has more than one thread (rope.cu:41-53 with the launch of
 * :69-74); this entry point applies the rotation the header documents. */
int llkv_rope_append(void* q, void* k, const void* v, void* k_pool, void* v_pool,
                     const int64_t* slot_mapping, const float* cos, const float* sin,
                     int num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                     int rotary_dim, int dtype, void* stream);

/* ------------------------------------------------------------------------
 * Paged decode attention (one new token per sequence), with Split-K.
 * Replaces lightllm::kv_cache::paged_attention
 * (include/lightllm/kv_cache/paged_attention.h:31-36,
 * src/kv_cache/paged_attention.cu:537-626) and its kernels (:104-532).
 *
 * q, out     : [num_seqs, num_q_heads, head_dim], element type `dtype`
 *              (the pool's type, as the reference requires).
 * block_table: device int32 [num_seqs, max_blocks_per_seq]
 * seq_lens   : device int32 [num_seqs]; sequence b attends positions [0, len).
 * max_seq_len: host-side upper bound of every seq_lens[b] (sizes the grid
 *              without the reference's device-to-host read).
 * num_splits : 0 = automatic, chosen from the kernel's resident work-group
 *              count: with few (sequence, kv head) units each is cut into
 *              S ~ resident / units fixed splits (when the longest sequence
 *              gives a wave more than 4 pages: 16-wave work-groups, one per
 *              CU, or 0.8 x the 4-wave count; at most one split per 4
 *              pages); with many (up to 1024
 *              sequences) the batch's pages are shared equally among one
 *              resident set of work-groups, whatever the length mix (larger
 *              batches use 8-page splits);
 *              S > 0 = the reference's fixed split (S ranges of ceil(n/S) pages).
 * scale      : softmax scale (the reference uses 1/sqrt(head_dim)).
 * workspace  : device memory of at least llkv_paged_decode_workspace_size()
 *              bytes (may be NULL when that size is 0); it holds the split
 *              partials (and the balanced schedule's page prefix sums), all
 *              written before they are read within one call, so it needs no
 *              initialisation.  Calls sharing one workspace must not overlap.
 * ------------------------------------------------------------------------ */
size_t llkv_paged_decode_workspace_size(int num_seqs, int num_q_heads,
                                        int num_kv_heads, int head_dim,
                                        int block_size, int max_seq_len,
                                        int num_splits);
int llkv_paged_decode(void* out, const void* q, const void* k_pool,
                      const void* v_pool, const int* block_table,
                      const int* seq_lens, int num_seqs, int num_q_heads,
                      int num_kv_heads, int head_dim, int block_size,
                      int max_blocks_per_seq, int max_seq_len, int num_splits,
                      float scale, int dtype, void* workspace,
                      size_t workspace_bytes, void* stream);

/* The schedule llkv_paged_decode (with_append 0) or llkv_paged_decode_append
 * (with_append 1; it takes the plain call's schedule, so that its results equal
 * append + decode bit for bit) takes for these shape arguments, for 16-byte aligned
 * pointers on the current device: *kind is one of llkv_decode_schedule and
 * *splits the key splits per (sequence, kv head) (0 for the balanced
 * schedule).  No counterpart in the reference: it lets a caller see which
 * kernels a batch shape runs (and what its workspace holds) without running it.
 * The decode calls first clamp max_seq_len to max_blocks_per_seq * block_size;
 * this query takes no table width, so it reports the call's schedule when
 * max_seq_len is already within that bound (pass the clamped value otherwise).
 * Returns LLKV_OK or LLKV_ERR_INVALID. */
enum llkv_decode_schedule {
    LLKV_SCHED_ONE_SPLIT = 0,   /* one 4-wave work-group per (sequence, kv head), no merge */
    LLKV_SCHED_UNIT = 1,        /* 16-wave work-groups: one per (sequence, kv head), no merge,
                                   or (splits > 1, long contexts) fixed splits + merge     */
    LLKV_SCHED_SPLITS = 2,      /* fixed key splits, then the log-sum-exp merge kernel      */
    LLKV_SCHED_BALANCED = 3,    /* equal page shares per work-group, then the merge kernel  */
    LLKV_SCHED_GENERIC = 4      /* shapes outside the tuned kernels (splits > 1: + merge)   */
};
int llkv_paged_decode_schedule(int num_seqs, int num_q_heads, int num_kv_heads,
                               int head_dim, int block_size, int max_seq_len,
                               int num_splits, int dtype, int with_append,
                               int* kind, int* splits);

/* Paged decode that allocates nothing and takes no workspace: llkv_paged_decode
 * with its split partials in a device array of the library
 * (llkv_paged_decode_noalloc_max_bytes() = 16 MiB per GPU, held until the
 * process ends).  No counterpart in the reference: it is for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops).
 * Shapes whose llkv_paged_decode_workspace_size() exceeds the array are
 * rejected with LLKV_ERR_WORKSPACE.  Calls that overlap on one GPU share the
 * array and race: order them on one stream.  Results are those of
 * llkv_paged_decode with the same arguments. */
size_t llkv_paged_decode_noalloc_max_bytes(void);
int llkv_paged_decode_noalloc(void* out, const void* q, const void* k_pool,
                              const void* v_pool, const int* block_table,
                              const int* seq_lens, int num_seqs, int num_q_heads,
                              int num_kv_heads, int head_dim, int block_size,
                              int max_blocks_per_seq, int max_seq_len, int num_splits,
                              float scale, int dtype, void* stream);

/* Fused KV append + paged decode: llkv_append of the step's new rows followed
 * by llkv_paged_decode, in one launch (plus the merge).  Replaces a
 * paged_attention call (src/engine/engine_server.cpp:1812-1817) together with
 * the per-sequence write_decode_kv loop (:1822-1854, two cudaMemcpy each); the
 * order is append first, so the new token attends to itself (the order of a
 * decode step in which the appended token is part of the context).
 * k_new, v_new: [num_seqs, Hkv, D] in the pool dtype.  seq_lens already count
 * the new token: sequence b's new row goes to position seq_lens[b] - 1
 * (table page (L-1)/bs, row (L-1)%bs; skipped when that table entry is -1)
 * and attention covers positions [0, seq_lens[b]).  Results equal those of
 * the two calls made in order; the work-group that owns the new token reads
 * it from k_new / v_new while storing it to the pools.  Other arguments as
 * llkv_paged_decode. */
int llkv_paged_decode_append(void* out, const void* q, const void* k_new,
                             const void* v_new, void* k_pool, void* v_pool,
                             const int* block_table, const int* seq_lens,
                             int num_seqs, int num_q_heads, int num_kv_heads,
                             int head_dim, int block_size, int max_blocks_per_seq,
                             int max_seq_len, int num_splits, float scale, int dtype,
                             void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Paged prefill attention over cached prefixes, varlen over N sequences.
 * Generalises lightllm::kv_cache::prefill_paged_attention
 * (include/lightllm/kv_cache/paged_attention.h:71-77,
 * src/kv_cache/paged_attention.cu:1018-1092, kernels :641-974) from one
 * sequence to N in one launch.
 *
 * q, out    : [total_q, num_q_heads, head_dim]; sequence n owns query rows
 *             [cu_q[n], cu_q[n+1]) (device int32 [N+1]).
 * seq_lens  : device int32 [N]: total keys of sequence n (history + chunk);
 *             its chunk's K/V must already be in the pool.
 * causal    : query row i of a chunk of P rows sits at seq_len - P + i and
 *             attends keys at positions <= its own (self included), as the
 *             reference kernel (src/kv_cache/paged_attention.cu:658,712).
 * max_q_len, max_seq_len: host-side upper bounds (grid sizing).
 * workspace : device memory of llkv_paged_prefill_workspace_size() bytes for
 *             the partials of long key ranges (fp32 rows and log-sum-exp),
 *             which are then cut into
 *             chunks run in parallel; NULL (or a size of 0) runs every key
 *             range unsplit.  Calls sharing one workspace must not overlap.
 * ------------------------------------------------------------------------ */
size_t llkv_paged_prefill_workspace_size(int num_seqs, int total_q, int max_q_len,
                                         int max_seq_len, int num_q_heads,
                                         int head_dim, int block_size, int dtype);
int llkv_paged_prefill(void* out, const void* q, const void* k_pool,
                       const void* v_pool, const int* block_table,
                       int max_blocks_per_seq, const int* cu_q,
                       const int* seq_lens, int num_seqs, int total_q,
                       int max_q_len, int max_seq_len, int num_q_heads,
                       int num_kv_heads, int head_dim, int block_size,
                       int causal, float scale, int dtype, void* workspace,
                       size_t workspace_bytes, void* stream);

/* Replaces first_prefill_attn_batched_gpu[_dispatch]
 * (include/lightllm/kv_cache/paged_attention.h:130-145,
 * src/kv_cache/paged_attention.cu:1230-1383): causal attention of first
 * prefill chunks over contiguous (un-paged) K/V.  Offsets are element
 * offsets, as in the reference, of row starts (multiples of Hq*D and
 * Hkv*D, as EngineServer::step builds them, engine_server.cpp:1635-1636).
 * max_tokens is a host upper bound of num_tokens[e] (0: P_total; a tight
 * bound avoids launching empty query blocks).  16-byte aligned buffers with
 * head_dim 64, 96, 128 or 256 run on the MFMA prefill kernels; other shapes
 * on a row kernel.  Unlike the reference
 * this does not synchronise. */
int llkv_first_prefill_batched(void* out, const void* q, const void* k,
                               const void* v, int num_q_heads,
                               int num_kv_heads, int head_dim,
                               const int* offsets, const int* kv_offsets,
                               const int* num_tokens,
                               const int* token_cumsum, const int* start_poss,
                               int N, int P_total, int max_tokens, float scale,
                               int dtype, void* stream);

/* ------------------------------------------------------------------------
 * Host-side block pool + prefix cache (BlockAllocator, BlockTable,
 * PrefixCache of include/lightllm/kv_cache/block_allocator.h:37-186 and
 * prefix_cache.h:56-325), exposed as an opaque handle for non-C++ callers.
 * policy: 0 = Hash, 1 = Radix (PrefixCachePolicy).
 * storage: 0 = device pools (hipMalloc), 1 = host pools (malloc), 2 = no
 * pools (metadata only; k/v pointers are NULL).
 * ------------------------------------------------------------------------ */
typedef struct llkv_allocator llkv_allocator;

int llkv_allocator_create(int num_blocks, int block_size, int num_kv_heads,
                          int head_dim, int policy, int dtype, int storage,
                          llkv_allocator** out);
void llkv_allocator_destroy(llkv_allocator* a);
int llkv_allocator_allocate(llkv_allocator* a, uint64_t token_hash);
int llkv_allocator_allocate_tokens(llkv_allocator* a, const int* tokens,
                                   int n_tokens, int start_pos,
                                   int* out_blocks, int out_capacity,
                                   int* out_count);
void llkv_allocator_release(llkv_allocator* a, int block_id);
int llkv_allocator_find_by_hash(llkv_allocator* a, uint64_t token_hash);
/* Longest cached prefix of tokens[start_pos..]: returns matched tokens,
 * writes up to `capacity` block ids and their count. */
int llkv_allocator_find_cached_prefix(llkv_allocator* a, const int* tokens,
                                      int n_tokens, int start_pos,
                                      int* block_ids, int capacity,
                                      int* n_ids);
void llkv_allocator_insert_cached_blocks(llkv_allocator* a, const int* tokens,
                                         int n_tokens, int start_pos,
                                         const int* block_ids, int n_ids);
int llkv_allocator_evict_lru(llkv_allocator* a);
void llkv_allocator_increment_ref(llkv_allocator* a, int block_id);
int llkv_allocator_reset(llkv_allocator* a);
int llkv_allocator_num_free(const llkv_allocator* a);
int llkv_allocator_num_blocks(const llkv_allocator* a);
int llkv_allocator_ref_count(const llkv_allocator* a, int block_id);
/* Pages of block_size tokens (K and V) that fit a byte budget in the pool's
 * element type; the C form of BlockAllocator::blocks_for_budget (additive:
 * the reference engine sizes its pools as fp32, engine_server.cpp:418-422).
 * -1 for bad arguments; capped at INT32_MAX. */
int llkv_blocks_for_budget(uint64_t budget_bytes, int block_size,
                           int num_kv_heads, int head_dim, int dtype);
uint64_t llkv_allocator_token_hash(const llkv_allocator* a, int block_id);
size_t llkv_allocator_prefix_cache_size(const llkv_allocator* a);
void* llkv_allocator_k_storage(llkv_allocator* a);
void* llkv_allocator_v_storage(llkv_allocator* a);
size_t llkv_allocator_storage_bytes(const llkv_allocator* a);
/* FNV-1a 64 of a token block (HashPrefixCache::hash_tokens). */
uint64_t llkv_hash_tokens(const int* tokens, int n);

#ifdef __cplusplus
}
#endif
#endif /* LIGHTLLM_KV_H */
