// Read-ceiling kernels: measurement only, built into a separate library
// (liblightllm_kv_ceiling.so) that bench.py loads; not part of the product ABI.
//
// A decode call must read every K and V row of its batch's pages at least
// once, so the time a kernel takes to do nothing but read those exact bytes,
// in the pool's layout, bounds what any decode kernel over that batch can
// reach on this GPU.  Two forms:
//
//  * llkv_rc_flat: a pure read.  The host lists the batch's (page, kv head)
//    pieces -- byte offset of row 0 and the rows that hold tokens -- in the
//    order the decode visits them; each wave reads whole pieces (K and V) in a
//    grid-stride loop, every lane 16-byte loads, with no dependence between
//    loads but the loop.  No table lookups: the piece list is the page walk
//    already resolved.
//  * llkv_rc_chain: the read with the decode's own dependences and work
//    split: grid (S, Hkv, B) of 4-wave work-groups, each reads its sequence's
//    length, then its split's block-table entries, then the pages (wave w
//    takes pages w, w + 4, ...), as the fixed-split decode kernel does
//    (src/kv_cache/paged_attention.cu:324-460 of the reference splits the
//    same way), without any arithmetic on the rows.
//
// Both fold everything they load into an XOR of 32-bit words.  With checksum
// set each wave stores its word (sink[4 * blockIdx + wave], blockIdx
// linearised), and the XOR of all the words equals the XOR of the batch's K
// and V rows, which the tests check against the host.  Timed runs pass 0: the
// loads stay (the compiler cannot know the flag) and no store round trip
// delays the kernel's end.  Algorithmic bytes are
// counted exactly as the decode's (tokens, not padded pages: the rows past a
// sequence's end are not read).
#include <hip/hip_runtime.h>

#include <cstdint>

namespace llkv {
namespace ceiling {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;

__device__ inline uint32_t fold(u32x4 v) { return v.x ^ v.y ^ v.z ^ v.w; }

// XOR of acc over the wave, stored to sink[wg * kWaves + wave] by its lane 0
// (no barrier: each wave ends on its own).
__device__ inline void store_checksum(uint32_t acc, uint32_t* sink, int64_t wg, int checksum) {
    if (!checksum) return;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, off, 64);
    if ((threadIdx.x & 63) == 0) sink[wg * kWaves + (threadIdx.x >> 6)] = acc;
}

// One piece: rows [0, nrows) of piece_bytes each, stride row_stride bytes, from
// base.  Lane c of the wave takes chunk c, c + 64, ... (row = chunk / cpr).
template <int CPR>
__device__ inline uint32_t read_piece(const char* kb, const char* vb, int64_t off, int nrows,
                                      int64_t row_stride, int lane) {
    constexpr int kMaxChunks = 16 * CPR;   // 16 rows
    constexpr int kIters = (kMaxChunks + 63) / 64;
    u32x4 k[kIters], v[kIters];
#pragma unroll
    for (int i = 0; i < kIters; ++i) {
        const int c = lane + 64 * i;
        const int row = c / CPR, col = c % CPR;
        if (row < nrows) {
            const int64_t o = off + row * row_stride + col * 16;
            k[i] = *reinterpret_cast<const u32x4*>(kb + o);
            v[i] = *reinterpret_cast<const u32x4*>(vb + o);
        } else {
            k[i] = u32x4{0, 0, 0, 0};
            v[i] = u32x4{0, 0, 0, 0};
        }
    }
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < kIters; ++i) acc ^= fold(k[i]) ^ fold(v[i]);
    return acc;
}

// items[i] = (byte offset of the piece's row 0) << 5 | rows (1..16)
template <int CPR>
__global__ __launch_bounds__(64 * kWaves) void rc_flat_kernel(const char* __restrict__ kb,
                                                              const char* __restrict__ vb,
                                                              const int64_t* __restrict__ items,
                                                              int n_items, int64_t row_stride,
                                                              uint32_t* sink, int checksum) {
    const int lane = threadIdx.x & 63;
    const int gw = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const int nw = gridDim.x * kWaves;
    uint32_t acc = 0;
    int i = gw;
    // two pieces per trip: their loads are in flight together
    for (; i + nw < n_items; i += 2 * nw) {
        const int64_t a = items[i], b = items[i + nw];
        acc ^= read_piece<CPR>(kb, vb, a >> 5, (int)(a & 31), row_stride, lane);
        acc ^= read_piece<CPR>(kb, vb, b >> 5, (int)(b & 31), row_stride, lane);
    }
    if (i < n_items) {
        const int64_t a = items[i];
        acc ^= read_piece<CPR>(kb, vb, a >> 5, (int)(a & 31), row_stride, lane);
    }
    store_checksum(acc, sink, blockIdx.x, checksum);
}

template <int CPR>
__global__ __launch_bounds__(64 * kWaves) void rc_chain_kernel(const char* __restrict__ kb,
                                                               const char* __restrict__ vb,
                                                               const int* __restrict__ table,
                                                               const int* __restrict__ lens,
                                                               int max_blocks, int hkv,
                                                               int64_t piece_stride,
                                                               uint32_t* sink, int checksum) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z, S = gridDim.x;
    const int L = lens[b];
    const int n = (L + 15) / 16;
    const int per = (n + S - 1) / S;
    const int p0 = s * per, p1 = min(n, p0 + per);
    const int* bt = table + (int64_t)b * max_blocks;
    const int64_t row_stride = piece_stride * hkv;   // bytes of one pool row (all kv heads)
    uint32_t acc = 0;
    for (int p = p0 + w; p < p1; p += kWaves) {
        const int phys = bt[p];
        const int nrows = min(16, L - 16 * p);
        const int64_t off = ((int64_t)phys * 16) * row_stride + kvh * piece_stride;
        acc ^= read_piece<CPR>(kb, vb, off, nrows, row_stride, lane);
    }
    store_checksum(acc, sink, ((int64_t)b * gridDim.y + kvh) * gridDim.x + s, checksum);
}

template <int CPR>
void launch_flat(const void* k, const void* v, const int64_t* items, int n, int64_t rs, int nwg,
                 uint32_t* sink, int cs, hipStream_t st) {
    hipLaunchKernelGGL(rc_flat_kernel<CPR>, dim3(nwg), dim3(64 * kWaves), 0, st,
                       (const char*)k, (const char*)v, items, n, rs, sink, cs);
}

template <int CPR>
void launch_chain(const void* k, const void* v, const int* table, const int* lens, int max_blocks,
                  int B, int hkv, int S, int64_t ps, uint32_t* sink, int cs, hipStream_t st) {
    hipLaunchKernelGGL(rc_chain_kernel<CPR>, dim3(S, hkv, B), dim3(64 * kWaves), 0, st,
                       (const char*)k, (const char*)v, table, lens, max_blocks, hkv, ps, sink, cs);
}

}  // namespace
}  // namespace ceiling
}  // namespace llkv

using llkv::ceiling::launch_chain;
using llkv::ceiling::launch_flat;
using llkv::ceiling::rc_flat_kernel;

extern "C" {

// Pure read of n_items pieces (items as above) of piece_bytes per row (64,
// 128, 256 or 512), row_stride bytes apart, on nwg work-groups of 4 waves;
// sink: 4 * nwg uint32 checksums (one per wave), written when checksum != 0.
// Returns 0, or 1 for an unsupported piece size, or 2 for a launch error.
int llkv_rc_flat(const void* k_pool, const void* v_pool, const int64_t* items, int n_items,
                 int piece_bytes, int64_t row_stride, int nwg, void* sink, int checksum, void* stream) {
    hipStream_t st = (hipStream_t)stream;
    uint32_t* sk = (uint32_t*)sink;
    switch (piece_bytes) {
        case 64: launch_flat<4>(k_pool, v_pool, items, n_items, row_stride, nwg, sk, checksum, st); break;
        case 128: launch_flat<8>(k_pool, v_pool, items, n_items, row_stride, nwg, sk, checksum, st); break;
        case 256: launch_flat<16>(k_pool, v_pool, items, n_items, row_stride, nwg, sk, checksum, st); break;
        case 512: launch_flat<32>(k_pool, v_pool, items, n_items, row_stride, nwg, sk, checksum, st); break;
        default: return 1;
    }
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

// The decode-structured read: grid (num_splits, num_kv_heads, num_seqs); the
// piece of (page, kv head) is piece_bytes wide per row; sink: one uint32
// checksum per wave (4 per work-group), written when checksum != 0.
int llkv_rc_chain(const void* k_pool, const void* v_pool, const int* block_table, const int* seq_lens,
                  int max_blocks, int num_seqs, int num_kv_heads, int num_splits, int piece_bytes,
                  void* sink, int checksum, void* stream) {
    hipStream_t st = (hipStream_t)stream;
    uint32_t* sk = (uint32_t*)sink;
    const int64_t ps = piece_bytes;
    switch (piece_bytes) {
        case 64: launch_chain<4>(k_pool, v_pool, block_table, seq_lens, max_blocks, num_seqs, num_kv_heads, num_splits, ps, sk, checksum, st); break;
        case 128: launch_chain<8>(k_pool, v_pool, block_table, seq_lens, max_blocks, num_seqs, num_kv_heads, num_splits, ps, sk, checksum, st); break;
        case 256: launch_chain<16>(k_pool, v_pool, block_table, seq_lens, max_blocks, num_seqs, num_kv_heads, num_splits, ps, sk, checksum, st); break;
        case 512: launch_chain<32>(k_pool, v_pool, block_table, seq_lens, max_blocks, num_seqs, num_kv_heads, num_splits, ps, sk, checksum, st); break;
        default: return 1;
    }
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

// Resident work-groups of the flat kernel for this piece size on the current
// device (one full set is the grid the bench launches), 0 on error.
int llkv_rc_flat_resident(int piece_bytes) {
    int dev = 0, cus = 0, per = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    using llkv::ceiling::kWaves;
    hipError_t e = hipErrorInvalidValue;
    switch (piece_bytes) {
        case 64: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, rc_flat_kernel<4>, 64 * kWaves, 0); break;
        case 128: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, rc_flat_kernel<8>, 64 * kWaves, 0); break;
        case 256: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, rc_flat_kernel<16>, 64 * kWaves, 0); break;
        case 512: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, rc_flat_kernel<32>, 64 * kWaves, 0); break;
        default: return 0;
    }
    return e == hipSuccess ? cus * per : 0;
}

}  // extern "C"
