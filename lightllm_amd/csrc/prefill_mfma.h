// MFMA paged prefill attention for gfx950 (fp16 / bf16 here; fp32 pools take
// a 16x16x4 f32 variant of the same schedule; head_dim 64 / 96 / 128 / 256,
// 16-token pages).  Replaces the reference's scalar prefill kernels
// (src/kv_cache/paged_attention.cu:641-974) for these shapes.
//
// Work-group: 4 waves, 128 query rows of one q_head (32 per wave), keys in
// tiles of 64 (four pages) staged through LDS with double buffering.
//
// Per wave and key tile, with v_mfma_f32_16x16x32_{f16,bf16}:
//   S^T = K Q^T   A = K rows from LDS (16 keys x 32 dims per MFMA),
//                 B = Q^T held in registers for the whole kernel.
//                 Accumulator lane l holds 4 keys of query (l % 16).
//   online softmax per query column (row max over the lane's keys, then two
//                 cross-lane xor steps); the lane's own keys are exactly the
//                 k-slice it must feed to the second MFMA, so P never leaves
//                 registers.  The key order of the A rows is permuted so that
//                 each lane's 8 keys of a 32-key k-step are contiguous.
//   O^T = V^T P^T A = V^T from LDS (V is transposed while staging),
//                 B = P^T from registers.
// Causal masking uses the reference's rule: query i of a P-row chunk over L
// keys sits at L - P + i and sees keys <= that position.
//
// When the units alone would not fill the GPU, key ranges are cut into chunks
// of chunk_tiles tiles, one work-group each (N x qblocks x max_chunks x Hq
// work-groups, the q heads of one kv head on one XCD), so that a cached prefix of thousands of keys does not
// serialise on one work-group; their partials (normalised fp32 rows + fp32
// log2-sum-exp2) are merged by
// prefill_merge_kernel.  The host plans the split from the shape bounds and the
// kernel's resident work-group count; the kernel then drops it when the units'
// actual key lengths are even enough (no unit longer than the average load of
// a compute unit), and the merge kernel follows that decision.
#pragma once

#include "attn_common.h"

namespace llkv {

struct MfmaPrefillArgs {
    void* out;
    const void* q;
    const void* k;
    const void* v;
    const int* bt;
    const int* cu_q;
    const int* lens;
    int max_blocks, N, Hq, Hkv, causal;
    // contiguous K/V (first prefill): entry n's tcum[n + 1] - tcum[n] q rows
    // start at element q_off[n] (a multiple of q_row = Hq * D), its ntok[n]
    // keys at element kv_off[n] of k / v, and query row i sees keys j <= i
    // (paged_attention.cu:1253-1285); cu_q, lens and bt are unused.
    int contig;
    const int* q_off;
    const int* kv_off;
    const int* ntok;
    const int* tcum;
    int q_row;
    float scale_log2;
    int qblocks;      // query blocks per sequence
    int max_chunks;   // key chunks per (sequence, query block)
    int chunk_tiles;  // key tiles per chunk
    int groups;       // N * qblocks * max_chunks * Hkv (chunk slot, kv head) work items
    float* part_o;    // [N*qblocks*max_chunks*Hq][BQ][D] (max_chunks > 1)
    float* part_lse;  // [N*qblocks*max_chunks*Hq][BQ]
    // Split decision made on the device from the units' key lengths (max_chunks > 1):
    // plan_flag (workspace header) receives 1 when the launch runs unsplit after all.
    int* plan_flag;
    int n_cus;        // compute units of the device
    int resident;     // resident work-groups of the launched kernel
};

// Workspace bytes for the chunked schedule (0: the shape runs unchunked).
size_t prefill_mfma_workspace(int N, int Hq, int head_dim, int block_size, int dtype,
                              int total_q, int max_q_len, int max_seq_len);

// Returns -1 when the shape is not handled (caller falls back), else a status.
// workspace may be NULL (then no key range is split).  a.contig selects the
// contiguous-K/V form (max_q_len = max_seq_len = the token-count bound).
int launch_prefill_mfma(MfmaPrefillArgs a, int head_dim, int block_size, int dtype,
                        int total_q, int max_q_len, int max_seq_len, void* workspace,
                        size_t workspace_bytes, hipStream_t st);

}  // namespace llkv
