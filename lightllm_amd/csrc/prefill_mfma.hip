// MFMA paged prefill attention (see prefill_mfma.h for the design).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <type_traits>

#include "prefill_mfma.h"

namespace llkv {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// Native vector for staged K/V rows (HIP's uint4 struct is copied with memcpy,
// which keeps the staging registers in scratch memory).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <typename T> struct Mfma;

template <> struct Mfma<_Float16> {
    typedef f16x8 vec;
    __device__ static inline f32x4 mma(const uint4& a, const uint4& b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                     __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
    __device__ static inline uint32_t pack2(float x, float y) { return pack_h2(x, y); }
    static constexpr uint32_t kOnes = 0x3C003C00u;   // two halves of 1.0
};

template <> struct Mfma<bf16_t> {
    typedef bf16x8 vec;
    __device__ static inline f32x4 mma(const uint4& a, const uint4& b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                      __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
    __device__ static inline uint32_t pack2(float x, float y) { return pack_b2(x, y); }
    static constexpr uint32_t kOnes = 0x3F803F80u;   // two bfloat16 1.0
};

constexpr int BQ = 128;   // query rows per work-group

// Key-chunk partial rows are fp32 for every pool type.  fp16 rows (half the
// merge's traffic, 2-3 us on configuration 4) added a rounding of each chunk's
// normalised row, which chunks of opposite sign amplify in the merged output:
// seeded ragged batches over 4k-key prefixes went past the fp16 bound.
constexpr int WQ = 32;    // query rows per wave (two 16-column MFMA tiles)
constexpr int BN = 64;    // keys per tile (four pages)

// Unit u = (sequence n, query block qb): its query rows [q_lo, q_lo + BQ) of
// the sequence's P new tokens (starting at row q0 of q) over L keys, and its
// key tiles (the causal extent of the rows).  Query blocks are numbered from
// the last, so that in a sequence the longest unit comes first.
struct UnitInfo {
    int q0, P, L, kvo, hist, tiles;
};

// Sequence n's first q row, new tokens P, keys L, and (contiguous K/V) the
// element offset of its first K/V row.  Paged: rows cu_q[n] .. cu_q[n+1],
// L = seq_lens[n] capped at the table's extent.  Contiguous (first prefill):
// q rows from offsets[n] (a row start), P = token_cumsum[n + 1] - token_cumsum[n],
// L = num_tokens[n].
// hist: keys before query row 0's own position, so that causal query row i
// sees keys j <= hist + i (L - P for a chunk on a cached prefix; 0 for a first
// prefill entry, whose query and key counts may differ).
__device__ inline void seq_geom(const MfmaPrefillArgs& a, int n, int& q0, int& P, int& L, int& kvo,
                                int& hist) {
    if (a.contig) {
        q0 = a.q_off[n] / a.q_row;
        P = max(a.tcum[n + 1] - a.tcum[n], 0);
        L = max(a.ntok[n], 0);
        kvo = a.kv_off[n];
        hist = 0;
    } else {
        q0 = a.cu_q[n];
        P = a.cu_q[n + 1] - q0;
        const int l = a.lens[n];
        const int cap = a.max_blocks * kPage;
        L = l < 0 ? 0 : (l > cap ? cap : l);
        kvo = 0;
        hist = L - P;
    }
}

__device__ inline UnitInfo unit_info(const MfmaPrefillArgs& a, int u) {
    const int n = u / a.qblocks;
    const int qb = a.qblocks - 1 - (u % a.qblocks);
    UnitInfo r;
    seq_geom(a, n, r.q0, r.P, r.L, r.kvo, r.hist);
    const int q_lo = qb * BQ;
    if (q_lo >= r.P) {
        r.tiles = 0;
        return r;
    }
    int kend = a.causal ? r.hist + min(q_lo + BQ, r.P) : r.L;
    kend = kend < 0 ? 0 : (kend > r.L ? r.L : kend);
    r.tiles = (kend + BN - 1) / BN;
    return r;
}

// Units ranked by key tiles (descending, ties by index) for up to kRankUnits
// units; larger batches keep index order.  Every thread of the work-group
// calls rank_units (it contains barriers); it leaves in LDS each unit's tiles
// and lengths (so the chosen unit costs no second global round trip) and the
// unit at each rank, and returns the split decision: true when the host's key
// split is dropped because no unit has more key tiles than a compute unit's
// share of the whole launch (sum of tiles x Hq / CUs).  Such even loads run
// best unsplit (one work-group per unit, no partials or merge); uneven ones,
// where the longest unit would set the time, keep the split.
constexpr int kRankUnits = 1024;

__device__ inline bool rank_units(const MfmaPrefillArgs& a, int* order) {
    __shared__ int s_plan[2];   // sum of the units' tiles, longest unit's tiles
    const int U = a.N * a.qblocks;
    if (U > kRankUnits) return false;
    int* tiles = order;
    int* at = order + kRankUnits;
    int* q0s = order + 2 * kRankUnits;
    int* ps = order + 3 * kRankUnits;
    int* ls = order + 4 * kRankUnits;
    int* kvos = order + 5 * kRankUnits;
    for (int u = threadIdx.x; u < U; u += blockDim.x) {
        const UnitInfo r = unit_info(a, u);
        tiles[u] = r.tiles;
        q0s[u] = r.q0;
        ps[u] = r.P;
        ls[u] = r.L;
        kvos[u] = r.kvo;
    }
    __syncthreads();
    // The rank pass reads every unit's tiles: unit 0's thread also sums them, and
    // the thread of rank 0 holds the longest.
    for (int u = threadIdx.x; u < U; u += blockDim.x) {
        const int tu = tiles[u];
        int r = 0, sum = 0;
        for (int v = 0; v < U; ++v) {
            const int tv = tiles[v];
            r += (tv > tu) | ((tv == tu) & (v < u));
            sum += tv;
        }
        at[r] = u;
        if (u == 0) s_plan[0] = sum;
        if (r == 0) s_plan[1] = tu;
    }
    __syncthreads();
    return a.max_chunks > 1 && (int64_t)s_plan[1] * a.n_cus <= (int64_t)s_plan[0] * a.Hq;
}

// The unit at `rank` (after rank_units) and its UnitInfo.
__device__ inline int ranked_unit(const MfmaPrefillArgs& a, int rank, const int* order,
                                  UnitInfo& info) {
    if (a.N * a.qblocks > kRankUnits) {
        info = unit_info(a, rank);
        return rank;
    }
    const int u = order[kRankUnits + rank];
    info.q0 = order[2 * kRankUnits + u];
    info.P = order[3 * kRankUnits + u];
    info.L = order[4 * kRankUnits + u];
    info.kvo = order[5 * kRankUnits + u];
    info.tiles = order[u];
    return u;
}

// Wave priority around the S = K Q^T cluster (s_setprio: issue arbitration
// among the waves of one SIMD, not a queue or stream priority): a wave in its
// matrix phase issues ahead of waves in their softmax.  Measured at head_dim
// 128 (configuration 5: 210 -> 201 us); neutral at head_dim 64, where it is
// off.  Raising the PV cluster as well gained nothing.
#define LLKV_PF_PRIO(on, p)                                \
    do {                                                   \
        if (on) {                                          \
            __builtin_amdgcn_sched_barrier(0);             \
            __builtin_amdgcn_s_setprio(p);                 \
            __builtin_amdgcn_sched_barrier(0);             \
        }                                                  \
    } while (0)

constexpr int kPageWindow = 256;   // page ids staged in LDS at a time

constexpr int kXcds = 8;   // XCDs of an MI355X; work-groups go to them round-robin


// One work-group's work item, from its blockIdx.
//
// Work: Y = N x qblocks x max_chunks ranked chunk slots (blockIdx-independent
// order: slot / max_chunks is a rank in the descending order of the units'
// key tiles, longest-processing-time first) times Hkv kv-head groups of G
// q heads, which read the same K/V tiles.  The dispatcher hands consecutive
// work-groups to the 8 XCDs in turn, and each XCD has its own L2, so group
// j (slot-major) goes to XCD j % 8 with its G heads as that XCD's next G
// work-groups: they run together and share their K/V reads in one L2.
struct Work {
    int hq, kvh, unit, n, ci, q0, P, q_lo, L, kvo, hist, kend, t_begin, t_end;
    bool direct;   // one chunk: write the output row itself
};

// False when the work-group has nothing to do (uniform over the work-group;
// it may return before or after the ranking barriers, never between).
__device__ inline bool take_work(const MfmaPrefillArgs& a, int* order, Work& wk) {
    const int G = a.Hq / a.Hkv;
    // Work-groups b, b + CUs, b + 2 CUs of the first resident set share a CU.
    // When a CU holds two or more, the second set takes its items in reverse,
    // so that the CU holding the longest item of the first set gets the
    // shortest of the second.
    int bid = blockIdx.x;
    if (a.resident >= 2 * a.n_cus && bid >= a.n_cus && bid < 2 * a.n_cus) {
        const int hi = min(2 * a.n_cus, (int)gridDim.x);
        bid = a.n_cus + (hi - 1 - bid);
    }
    const int xcd = bid % kXcds, r = bid / kXcds;
    const int j = (r / G) * kXcds + xcd;
    if (j >= a.groups) return false;
    wk.kvh = j % a.Hkv;
    wk.hq = wk.kvh * G + r % G;
    const int y = j / a.Hkv;
    // Every work-group takes the same decision from the same lengths.  Unsplit,
    // the first N x qblocks chunk slots are the units themselves (chunk 0) and
    // the other work-groups have nothing to do.
    const bool unsplit = rank_units(a, order);
    if (blockIdx.x == 0 && threadIdx.x == 0 && a.plan_flag != nullptr) *a.plan_flag = unsplit ? 1 : 0;
    int slot;
    if (unsplit) {
        if (y >= a.N * a.qblocks) return false;
        slot = y;
        wk.ci = 0;
    } else {
        slot = y / a.max_chunks;
        wk.ci = y - slot * a.max_chunks;   // key chunk of the unit
    }
    UnitInfo ui;
    wk.unit = ranked_unit(a, slot, order, ui);  // (sequence, query block)
    wk.n = wk.unit / a.qblocks;
    const int qb = a.qblocks - 1 - (wk.unit % a.qblocks);
    wk.q0 = ui.q0;
    wk.P = ui.P;
    wk.q_lo = qb * BQ;
    if (wk.q_lo >= wk.P) return false;
    wk.L = ui.L;
    wk.kvo = ui.kvo;
    wk.hist = a.contig ? 0 : ui.L - ui.P;   // as seq_geom (not kept with the ranked units)
    int kend = a.causal ? wk.hist + min(wk.q_lo + BQ, wk.P) : wk.L;
    wk.kend = kend < 0 ? 0 : (kend > wk.L ? wk.L : kend);
    const int ntiles = (wk.kend + BN - 1) / BN;
    // at most max_chunks chunks (a max_seq_len bound below a length): the last
    // one takes the remaining tiles
    const int nchunks = unsplit ? 1 : min((ntiles + a.chunk_tiles - 1) / a.chunk_tiles, a.max_chunks);
    if (wk.ci > 0 && wk.ci >= nchunks) return false;   // chunk 0 also covers an empty key range (zeros)
    wk.t_begin = wk.ci * a.chunk_tiles;
    wk.t_end = wk.ci == nchunks - 1 ? ntiles : min(wk.t_begin + a.chunk_tiles, ntiles);
    wk.direct = nchunks <= 1;
    return true;
}

// Query rows beyond the launch's qblocks * BQ (a max_q_len bound below a
// sequence's query count) have no work-group: the top query block's chunk-0
// work-group sets them to NaN for its head, so the broken bound shows in the
// output instead of leaving stale rows.
template <typename T, int D>
__device__ inline void poison_uncovered_rows(const MfmaPrefillArgs& a, const Work& wk) {
    const int covered = a.qblocks * BQ;
    if (wk.ci != 0 || wk.q_lo != covered - BQ || wk.P <= covered) return;
    T* og = reinterpret_cast<T*>(a.out);
    const int n = (wk.P - covered) * D;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int r = covered + i / D;
        og[((int64_t)(wk.q0 + r) * a.Hq + wk.hq) * D + i % D] = Elem<T>::from_f32(__builtin_nanf(""));
    }
}

// Direct-to-LDS load of 16 bytes per lane: lane L's bytes land at LDS address
// lds + 16 L (lds uniform over the wave).  Issued as inline assembly, so that
// the compiler, which cannot tell the two tile buffers apart, does not wait for
// it before every LDS read of the other buffer; the caller waits (vmcnt) before
// the barrier that publishes the tile.  A later load only lengthens the
// compiler's own in-order vmcnt waits.
// la: the LDS byte address (lds_addr), wave-uniform.
__device__ inline uint32_t lds_addr(const void* lds) {
    return __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds);
}

__device__ inline void dma16(const void* gptr, uint32_t la) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(gptr), "s"(la)
                 : "memory", "m0");
}

// The same with a wave-uniform base (scalar registers) and a 32-bit per-lane
// byte offset (no per-lane 64-bit address arithmetic).
__device__ inline void dma16_s(const void* sbase, uint32_t voff, uint32_t la) {
    const uint64_t b = (uint64_t)(uintptr_t)sbase;
    // (readfirstlane returns int: widen through uint32_t, not by sign extension)
    const uint64_t bs = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32)) << 32) |
                        (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(bs), "s"(la)
                 : "memory", "m0");
}

// Instruction order of the S^T = K Q^T cluster (KS k-steps of 4 K operand
// reads and 8 MFMAs): the reads of k-steps 0 and 1, then each k-step's MFMAs
// followed by the reads of the k-step after next, so that one k-step's LDS
// reads are always in flight behind the MFMAs.
template <int KS, int I = 0>
__device__ inline void qk_schedule() {
    if constexpr (I == 0) __builtin_amdgcn_sched_group_barrier(0x100, KS > 1 ? 8 : 4, 0);   // DS reads
    if constexpr (I < KS) {
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);                                 // MFMAs
        if constexpr (I + 2 < KS) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
        qk_schedule<KS, I + 1>();
    }
}

// K and V tiles are row-major (key rows of D halves, KPAD apart); V's O^T
// operand is read with transposing LDS reads.  DMA: the tiles are written by
// direct-to-LDS loads in 1 KB blocks, so rows are unpadded and their 16-byte
// chunks XOR-swizzled by row instead.
template <int D, bool DMA>
struct Smem {
    static constexpr int KPAD = DMA ? D : D + 8;   // halves per K / V row (pad: spread LDS banks)
    union {
        struct {
            alignas(16) uint16_t k[2][BN * KPAD];
            alignas(16) uint16_t v[2][BN * KPAD];
        };
        int order[6 * kRankUnits];   // prologue only: unit tiles, unit at each rank, q0, P, L, K/V offset
    };
    int pages[kPageWindow];   // page ids [tbase, tbase + kPageWindow) of the sequence
};

// CG: contiguous K/V (first prefill): key j of the sequence is row kvo + j of
// k / v; the staged rows are clamped to the sequence's last, and there is no
// page table.
// head_dim 128: two waves per SIMD (<= 256 registers).
template <typename T, int D, bool CG>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 128 ? 2 : 1)))
void prefill_mfma_kernel(MfmaPrefillArgs a) {
    // Direct-to-LDS staging (head_dim 64 / 128): wave w loads page w of the
    // tile (rows 16w .. 16w + 15) of K and of V, RPB rows per 1 KB block.
    constexpr bool kDma = D == 64 || D == 128;
    using SM = Smem<D, kDma>;
    constexpr int KPAD = SM::KPAD;
    constexpr int CPR = D / 8;            // 16-byte chunks per row
    constexpr int RPB = 64 / CPR;         // rows per 1 KB block
    constexpr int BPW = 16 / RPB;         // blocks per wave (one page) per tile
    // Chunk swizzle of tile row r: row bits 0, 1, 3, 4 (the QK^T operand reads
    // rows 8 (c16 / 4) + 4 h + c16 % 4 together, so rows 8 apart must differ).
    auto swz_row = [](int r) { return ((r & 3) | ((r >> 1) & 0xC)) & (CPR - 1); };
    constexpr int KS = D / 32;            // k-steps of the QK^T product
    constexpr int DT = D / 16;            // 16-dim tiles of the output
    constexpr int KCH = BN * D / 8;       // 16-byte K chunks per tile
    constexpr int KCH_T = KCH / 256;      // per thread
    __shared__ SM sm;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index, known uniform
    const int g = lane >> 4, c16 = lane & 15;
    Work wk;
    if (!take_work(a, sm.order, wk)) return;
    // The ranking's arrays overlay the tile buffers.  Paged launches pass an
    // LDS barrier (stage_pages) before the first tile is written; contiguous
    // K/V has no page window, so every wave's reads of its unit from the
    // ranking must complete here before any wave writes the first tile.
    if constexpr (CG) lds_barrier();
    poison_uncovered_rows<T, D>(a, wk);
    const int hq = wk.hq, kvh = wk.kvh, unit = wk.unit, n = wk.n, ci = wk.ci;
    const int q0 = wk.q0, P = wk.P, q_lo = wk.q_lo, L = wk.L, kend = wk.kend;
    const int t_begin = wk.t_begin, t_end = wk.t_end;
    const bool direct = wk.direct;
    const int last_page = L > 0 ? (L - 1) / kPage : 0;
    const int* bt = a.bt + (int64_t)n * a.max_blocks;
    const T* kg = reinterpret_cast<const T*>(a.k) + (int64_t)kvh * D + (CG ? (int64_t)wk.kvo : 0);
    const T* vg = reinterpret_cast<const T*>(a.v) + (int64_t)kvh * D + (CG ? (int64_t)wk.kvo : 0);

    // ---- Q^T operands (B of S^T = K Q^T), kept in registers; loaded after the
    // page ids so that their latency overlaps the first tile's ------------
    uint4 qop[2][KS];
    const T* qg = reinterpret_cast<const T*>(a.q);
    auto load_q = [&]() {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const int ql = q_lo + w * WQ + nt * 16 + c16;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                if (ql < P)
                    qop[nt][ks] = *reinterpret_cast<const uint4*>(
                        qg + ((int64_t)(q0 + ql) * a.Hq + hq) * D + ks * 32 + g * 8);
                else
                    qop[nt][ks] = make_uint4(0, 0, 0, 0);
            }
        }
    };

    // Absolute position of this lane's two query columns; rows >= P see nothing.
    int qpos[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int ql = q_lo + w * WQ + nt * 16 + c16;
        qpos[nt] = ql < P ? (a.causal ? wk.hist + ql : L - 1) : -1;
    }

    // Smallest query position of the wave's 32 rows (every row valid), for the
    // unmasked fast path of tiles that lie entirely below it.
    const int wq0 = q_lo + w * WQ;
    const int wave_min_pos = (wq0 + WQ <= P) ? (a.causal ? wk.hist + wq0 : L - 1) : -1;

    f32x4 o[DT][2];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) o[dt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m[2] = {kNegBig, kNegBig};
    // Row sums of P on the MFMA: O^T's extra tile with an all-ones A operand;
    // every element of osum[nt] is the running sum of query column c16.
    f32x4 osum[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    const uint4 ones = make_uint4(Mfma<T>::kOnes, Mfma<T>::kOnes, Mfma<T>::kOnes, Mfma<T>::kOnes);

    // ---- staging: global -> registers -> LDS -----------------------------
    int tbase = 0;   // first page id held in sm.pages
    // V is staged like K (row-major, the same row offsets and page addresses).
    u32x4 kr[KCH_T], vr[KCH_T];
    static_assert(KCH % 256 == 0, "K / V chunks spread evenly over the threads");
    // Per-thread byte offsets inside a page and page slot of each staged row;
    // a load is then base + phys * page_bytes + offset (one 32x32->64 multiply-add).
    // Contiguous K/V: the key within the tile and the byte offset in the row.
    const uint32_t row_bytes = (uint32_t)(a.Hkv * D * sizeof(T));
    const uint32_t page_bytes = row_bytes * kPage;
    const char* kb = reinterpret_cast<const char*>(kg);
    const char* vb = reinterpret_cast<const char*>(vg);
    uint32_t koff[KCH_T];
    int kslot[KCH_T];
#pragma unroll
    for (int j = 0; j < KCH_T; ++j) {
        const int ch = tid + 256 * j;
        const int key = ch / (D / 8), c = ch % (D / 8);
        kslot[j] = CG ? key : key >> 4;
        koff[j] = (CG ? 0u : (uint32_t)(key & 15) * row_bytes) + (uint32_t)c * 16u;
    }
    auto load_tile = [&](int t, u32x4 (&kreg)[KCH_T], u32x4 (&vreg)[KCH_T]) {
        if constexpr (CG) {   // rows past the sequence's last are staged as the last
            const int key0 = t * BN, last = L - 1;
#pragma unroll
            for (int j = 0; j < KCH_T; ++j) {
                const uint64_t off = (uint64_t)min(key0 + kslot[j], last) * row_bytes + koff[j];
                kreg[j] = *reinterpret_cast<const u32x4*>(kb + off);
                vreg[j] = *reinterpret_cast<const u32x4*>(vb + off);
            }
            return;
        }
        // pages past the sequence's last are staged as the last page (valid memory)
        const int* pg = sm.pages + (4 * t - tbase);
#pragma unroll
        for (int j = 0; j < KCH_T; ++j) {
            const uint64_t off = (uint64_t)(uint32_t)max(pg[kslot[j]], 0) * page_bytes + koff[j];
            kreg[j] = *reinterpret_cast<const u32x4*>(kb + off);
            vreg[j] = *reinterpret_cast<const u32x4*>(vb + off);
        }
    };
    auto store_tile = [&](int buf, const u32x4 (&kreg)[KCH_T], const u32x4 (&vreg)[KCH_T]) {
#pragma unroll
        for (int j = 0; j < KCH_T; ++j) {
            const int ch = tid + 256 * j;
            const int key = ch / (D / 8), c = ch % (D / 8);
            *reinterpret_cast<u32x4*>(&sm.k[buf][key * KPAD + c * 8]) = kreg[j];
            *reinterpret_cast<u32x4*>(&sm.v[buf][key * KPAD + c * 8]) = vreg[j];
        }
    };
    // Half-column hc of tile row `row` in LDS: with DMA the 16-byte chunk
    // index is XOR-ed with the row (mod the chunks per row).
    auto scol = [&](int row, int hc) {
        if constexpr (kDma) return (((hc >> 3) ^ swz_row(row)) << 3) | (hc & 7);
        return hc;
    };
    // A operand of O^T = V^T P^T for output dims dt*16 .. +15 and the 32-key
    // half ss: lane (g, c16) holds dim dt*16 + c16 of keys 32 ss + 8 g .. + 7.
    // ds_read_b64_tr_b16 within each 16-lane group: output lane 4a + e gets
    // element e of the 4 halves addressed by lanes a, a + 4, a + 8, a + 12; so
    // lane c16 addresses row (key) c16 / 4, dims 4 (c16 % 4) .. + 3, and each
    // lane receives its dim over 4 consecutive keys (two reads: 8 keys).
    auto v_operand = [&](int buf, int dt, int ss) {
        typedef short s16x4 __attribute__((ext_vector_type(4)));
        const int r0 = 32 * ss + 8 * g + (c16 >> 2), hc = dt * 16 + 4 * (c16 & 3);
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(&sm.v[buf][r0 * KPAD + scol(r0, hc)]));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(&sm.v[buf][(r0 + 4) * KPAD + scol(r0 + 4, hc)]));
        typedef unsigned u32x2v __attribute__((ext_vector_type(2)));
        const u32x2v l2 = __builtin_bit_cast(u32x2v, lo), h2 = __builtin_bit_cast(u32x2v, hi);
        return make_uint4(l2.x, l2.y, h2.x, h2.y);
    };

    // Page ids live in LDS so that no K/V load waits behind a table load.
    auto stage_pages = [&](int base) {
        if constexpr (CG) return;   // no page table
        tbase = base;
        for (int i = tid; i < kPageWindow; i += 256) sm.pages[i] = bt[min(base + i, last_page)];
        lds_barrier();   // the page ids are in LDS; no global load needs to have landed
    };
    // Direct-to-LDS: lane L of block j writes LDS chunk L of rows 16w + j RPB ..,
    // i.e. row 16w + j RPB + L / CPR, chunk position L % CPR, which holds the
    // row's global chunk (L % CPR) ^ swz_row(row).
    uint32_t dma_off[BPW];   // byte offset of the lane's chunk inside its page (paged) / row (CG)
    int dma_row[BPW];        // the lane's row within the wave's page
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
        const int r = j * RPB + lane / CPR;
        const int c = (lane % CPR) ^ swz_row(16 * w + r);
        dma_row[j] = r;
        dma_off[j] = (CG ? 0u : (uint32_t)r * row_bytes) + (uint32_t)c * 16u;
    }
    // LDS byte addresses of the wave's blocks in each buffer, computed once
    // (scalar registers; the loop then only moves them to M0).
    uint32_t lds_k[2][BPW], lds_v[2][BPW];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int j = 0; j < BPW; ++j) {
            const int lrow = 16 * w + j * RPB;
            lds_k[b][j] = lds_addr(&sm.k[b][lrow * KPAD]);
            lds_v[b][j] = lds_addr(&sm.v[b][lrow * KPAD]);
        }
    auto dma_tile = [&](int t, int buf) {
        if constexpr (kDma) {
            if constexpr (CG) {
#pragma unroll
                for (int j = 0; j < BPW; ++j) {   // rows past the sequence's last are staged as the last
                    const int key = min(t * BN + 16 * w + dma_row[j], L - 1);
                    const uint64_t off = (uint64_t)key * row_bytes + dma_off[j];
                    dma16(kb + off, lds_k[buf][j]);
                    dma16(vb + off, lds_v[buf][j]);
                }
            } else {
                // the wave's page: one scalar base per pool, 32-bit lane offsets
                const int phys = __builtin_amdgcn_readfirstlane(max(sm.pages[4 * t + w - tbase], 0));
                const uint64_t pbase = (uint64_t)(uint32_t)phys * page_bytes;
#pragma unroll
                for (int j = 0; j < BPW; ++j) {
                    dma16_s(kb + pbase, dma_off[j], lds_k[buf][j]);
                    dma16_s(vb + pbase, dma_off[j], lds_v[buf][j]);
                }
            }
        }
    };
    if (t_begin < t_end) {
        stage_pages(4 * t_begin);
        load_q();
        if constexpr (kDma) {
            dma_tile(t_begin, 0);
            __builtin_amdgcn_s_waitcnt(0x3F70);   // vmcnt(0): this wave's blocks are in LDS
        } else {
            load_tile(t_begin, kr, vr);
            store_tile(0, kr, vr);
        }
    }
    __syncthreads();

    // One key tile; buf = (t - t_begin) & 1.  The loop below runs it twice per
    // trip with buf as a compile-time constant, so the LDS addresses of both
    // buffers fold into the instructions' offsets.
    auto tile_step = [&](int t, auto bufc) {
        const int buf = static_cast<int>(bufc);
        if (t + 1 < t_end) {
            // tile t+1 covers pages [4(t+1), 4(t+1)+4); restage when they leave the window
            // (uniform branch; every earlier read of sm.pages preceded the last barrier)
            if (4 * (t + 1) + 4 > tbase + kPageWindow) stage_pages(4 * (t + 1));
            if constexpr (kDma) dma_tile(t + 1, buf ^ 1);
            else load_tile(t + 1, kr, vr);
        }
        __builtin_amdgcn_sched_barrier(0);   // next tile's loads issue before this tile's MFMAs
        LLKV_PF_PRIO(D >= 128, 1);

        // ---- S^T = K Q^T over the 64 keys: 4 key tiles x 2 query tiles ----
        // k-step outer: the 8 (key tile, query tile) chains advance together,
        // and the K operands of k-step ks + 1 are read while those of ks feed
        // the matrix core.
        f32x4 s[4][2];
        auto k_operand = [&](int kt, int ks) {
            // A row c16 of key tile kt = 2*ss + h holds key 32*ss + 8*(c16/4) + 4*h + c16%4
            const int krow = 32 * (kt >> 1) + 8 * (c16 >> 2) + 4 * (kt & 1) + (c16 & 3);
            return *reinterpret_cast<const uint4*>(&sm.k[buf][krow * KPAD + scol(krow, ks * 32 + g * 8)]);
        };
        uint4 ka[2][4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) ka[0][kt] = k_operand(kt, 0);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            if (ks + 1 < KS) {
#pragma unroll
                for (int kt = 0; kt < 4; ++kt) ka[(ks + 1) & 1][kt] = k_operand(kt, ks + 1);
            }
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
                    s[kt][nt] = Mfma<T>::mma(ka[ks & 1][kt], qop[nt][ks],
                                             ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : s[kt][nt]);
        }
        if constexpr (kDma) qk_schedule<KS>();

        LLKV_PF_PRIO(D >= 128, 0);
        // ---- mask, online softmax (per query column) ----------------------
        // Scores stay raw (unscaled) until the exponent: p = 2^(s c - m) with
        // c = scale * log2(e) > 0, so the row maximum commutes with the scaling.
        const int key0 = t * BN;
        const float c = a.scale_log2;
        // Every key of the tile visible to every row of the wave (uniform): no mask.
        const bool unmasked = key0 + BN - 1 <= wave_min_pos && key0 + BN <= kend;
        float mx[2];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            if (!unmasked) {
                // key = key0 + 8g + (32 ss + 4 h + i) is visible iff key <= min(qpos, kend - 1)
                const int r = min(qpos[nt], kend - 1) - key0 - 8 * g;
#pragma unroll
                for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (32 * (kt >> 1) + 4 * (kt & 1) + i > r) s[kt][nt][i] = -INFINITY;
            }
            float v = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) v = fmaxf(v, s[kt][nt][i]);
            mx[nt] = v * c;   // this lane's 16 keys only
        }
        // Lazy rescaling: the running max m only moves when some lane's tile
        // max exceeds it by more than 8 (so p <= 2^8 otherwise); then the wave
        // reduces the row maxima over the 4 lanes of each query column and
        // rescales its accumulators once.  Usually only the first tile does, so
        // the common path has no cross-lane traffic.
        bool grow = false;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) grow |= mx[nt] > m[nt] + 8.0f;
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                float v = mx[nt];
                v = fmaxf(v, __shfl_xor(v, 16, 64));
                v = fmaxf(v, __shfl_xor(v, 32, 64));
                const float mnew = fmaxf(m[nt], v);
                const float corr = fast_exp2(m[nt] - mnew);
                m[nt] = mnew;
                osum[nt] *= corr;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) o[dt][nt] *= corr;
            }
        }
        // ---- P = 2^(S c - m) and O^T += V^T P^T, one 32-key half after the
        // other: the second half's exponentials are interleaved with the first
        // half's MFMAs, so that the VALU and the matrix core work together.
        uint4 pop[2][2];   // P^T operands [k-step = key half][query tile]
        auto softmax_half = [&](int ss) {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                float pv[2][4];
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        pv[h][i] = fast_exp2(fmaf(s[2 * ss + h][nt][i], c, -m[nt]));
                pop[ss][nt].x = Mfma<T>::pack2(pv[0][0], pv[0][1]);
                pop[ss][nt].y = Mfma<T>::pack2(pv[0][2], pv[0][3]);
                pop[ss][nt].z = Mfma<T>::pack2(pv[1][0], pv[1][1]);
                pop[ss][nt].w = Mfma<T>::pack2(pv[1][2], pv[1][3]);
            }
        };
        // The first half's MFMAs, each followed by a share of the second half's
        // exponentials; sched_barrier keeps this order (the scheduler would
        // otherwise put all VALU work first).  V^T rows of the second half are
        // read as those of the first are consumed.
        softmax_half(0);
        {
            constexpr int kMf = 2 * DT + 2;   // MFMAs per half
            uint4 va0[DT], va1[DT];
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
                va0[dt] = v_operand(buf, dt, 0);
            float pv1[2][2][4];   // [query tile][h][i] of the second half
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int k = 0; k < kMf; ++k) {
                if (k < 2 * DT) {
                    const int dt = k >> 1, nt = k & 1;
                    o[dt][nt] = Mfma<T>::mma(va0[dt], pop[0][nt], o[dt][nt]);
                    if (nt == 1)
                        va1[dt] = v_operand(buf, dt, 1);
                } else {
                    const int nt = k - 2 * DT;
                    osum[nt] = Mfma<T>::mma(ones, pop[0][nt], osum[nt]);
                }
#pragma unroll
                for (int e = k * 16 / kMf; e < (k + 1) * 16 / kMf; ++e) {
                    const int nt = e >> 3, h = (e >> 2) & 1, i = e & 3;
                    pv1[nt][h][i] = fast_exp2(fmaf(s[2 + h][nt][i], c, -m[nt]));
                }
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                pop[1][nt].x = Mfma<T>::pack2(pv1[nt][0][0], pv1[nt][0][1]);
                pop[1][nt].y = Mfma<T>::pack2(pv1[nt][0][2], pv1[nt][0][3]);
                pop[1][nt].z = Mfma<T>::pack2(pv1[nt][1][0], pv1[nt][1][1]);
                pop[1][nt].w = Mfma<T>::pack2(pv1[nt][1][2], pv1[nt][1][3]);
            }
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) o[dt][nt] = Mfma<T>::mma(va1[dt], pop[1][nt], o[dt][nt]);
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) osum[nt] = Mfma<T>::mma(ones, pop[1][nt], osum[nt]);
        }

        if constexpr (kDma) {
            if (t + 1 < t_end) __builtin_amdgcn_s_waitcnt(0x3F70);   // vmcnt(0): tile t+1 in LDS
        } else {
            if (t + 1 < t_end) store_tile(buf ^ 1, kr, vr);
        }
        __syncthreads();
    };
    {
        int t = t_begin;
        for (; t + 1 < t_end; t += 2) {
            tile_step(t, std::integral_constant<int, 0>());
            tile_step(t + 1, std::integral_constant<int, 1>());
        }
        if (t < t_end) tile_step(t, std::integral_constant<int, 0>());
    }

    // ---- normalise and write: lane holds dims dt*16 + 4g + i of its query --
    // (one chunk: the output row; several: an fp32 partial row + log2-sum-exp2,
    // -inf for a row that saw no key of this chunk)
    T* og = reinterpret_cast<T*>(a.out);
    const int64_t pidx = ((int64_t)unit * a.max_chunks + ci) * a.Hq + hq;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const float lt = osum[nt][0];
        const int row = w * WQ + nt * 16 + c16;
        const int ql = q_lo + row;
        if (ql >= P) continue;
        const float inv = lt > 0.f ? 1.0f / lt : 0.f;
        if (direct) {
            T* orow = og + ((int64_t)(q0 + ql) * a.Hq + hq) * D;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                uint2 w2;
                w2.x = Mfma<T>::pack2(o[dt][nt][0] * inv, o[dt][nt][1] * inv);
                w2.y = Mfma<T>::pack2(o[dt][nt][2] * inv, o[dt][nt][3] * inv);
                *reinterpret_cast<uint2*>(orow + dt * 16 + 4 * g) = w2;
            }
        } else {
            float* prow = a.part_o + (pidx * BQ + row) * D;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
                *reinterpret_cast<float4*>(prow + dt * 16 + 4 * g) =
                    make_float4(o[dt][nt][0] * inv, o[dt][nt][1] * inv, o[dt][nt][2] * inv,
                                o[dt][nt][3] * inv);
            if (g == 0) a.part_lse[pidx * BQ + row] = lt > 0.f ? m[nt] + fast_log2(lt) : -INFINITY;
        }
    }
}

// fp32 pools: v_mfma_f32_16x16x4f32 for both products, same work mapping,
// chunking and merge as the 16-bit kernel.  Per wave and 64-key tile:
//   S^T = K Q^T   A = K rows from LDS, one 16-byte read feeds four k-steps:
//                 lane (g, c16) holds dims 16kb + 4g .. 16kb + 4g + 3 of key
//                 row c16, and Q^T (registers) holds the same dims of query
//                 c16, so k-step j of block kb contracts dim 16kb + 4g + j.
//                 Accumulator lane (g, c16) holds keys 4g + i of query c16.
//   O^T = V^T P^T the lane's four keys 4g + i of a 16-key tile are exactly the
//                 k-slot g of four k-steps (i = 0..3), so P^T never leaves
//                 registers; A = V^T (transposed while staging) read 16 bytes
//                 (keys 4g .. 4g + 3 of one dim) per four k-steps.
// Softmax row sums are kept per lane (its own keys) and reduced over the four
// lanes of a query column at the end.
// LDS tile buffers and occupancy.  head_dim 64: K double-buffered, V^T
// single (53 KB), three waves per SIMD (the compiler spills ~60 registers to
// reach 168; still 13 % faster than two waves without spills).  head_dim 128:
// ~300 registers, one wave per SIMD, so both tiles double-buffered (137 KB).
// The S = K Q^T cluster at raised wave priority (as in the 16-bit kernel):
// configuration 4's shape in fp32 360-380 -> 339-344 us; neutral at
// head_dim 128 (one wave per SIMD).
template <int D>
struct SmemF32 {
    static constexpr int KNB = D == 64 || D == 128 ? 2 : 1;
    static constexpr int VNB = D == 128 ? 2 : 1;   // 64, 96, 256: 1
    static constexpr int KPAD = D + 4;    // floats per K row (pad: 16-byte reads of 16 rows hit distinct banks)
    static constexpr int VPAD = BN + 4;   // floats per V^T row
    union {
        struct {
            alignas(16) float k[KNB][BN * KPAD];
            alignas(16) float vt[VNB][D * VPAD];
        };
        int order[6 * kRankUnits];
    };
    int pages[kPageWindow];
};

template <int D, bool CG>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 64 ? 3 : (D == 96 ? 2 : 1))))
void prefill_f32_kernel(MfmaPrefillArgs a) {
    typedef SmemF32<D> S;
    constexpr int KPAD = S::KPAD, VPAD = S::VPAD, KNB = S::KNB, VNB = S::VNB;
    constexpr int KB = D / 16;              // 16-dim blocks of the QK^T product
    constexpr int DT = D / 16;              // 16-dim tiles of the output
    constexpr int KCH_T = BN * D / 4 / 256;          // 16-byte K chunks per thread
    constexpr int VT_N = (BN / 4) * (D / 4);           // V tasks (4 keys x 4 dims) per tile
    constexpr int VT_T = (VT_N + 255) / 256;           // per thread (head_dim 96: the last partly idle)
    __shared__ S sm;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, c16 = lane & 15;
    Work wk;
    if (!take_work(a, sm.order, wk)) return;
    // The ranking's arrays overlay the tile buffers.  Paged launches pass an
    // LDS barrier (stage_pages) before the first tile is written; contiguous
    // K/V has no page window, so every wave's reads of its unit from the
    // ranking must complete here before any wave writes the first tile.
    if constexpr (CG) lds_barrier();
    poison_uncovered_rows<float, D>(a, wk);
    const int hq = wk.hq, kvh = wk.kvh, unit = wk.unit, n = wk.n, ci = wk.ci;
    const int q0 = wk.q0, P = wk.P, q_lo = wk.q_lo, L = wk.L, kend = wk.kend;
    const int t_begin = wk.t_begin, t_end = wk.t_end;
    const int last_page = L > 0 ? (L - 1) / kPage : 0;
    const int* bt = a.bt + (int64_t)n * a.max_blocks;

    float4 qop[2][KB];
    const float* qg = reinterpret_cast<const float*>(a.q);
    auto load_q = [&]() {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const int ql = q_lo + w * WQ + nt * 16 + c16;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
                qop[nt][kb] = ql < P ? *reinterpret_cast<const float4*>(
                                           qg + ((int64_t)(q0 + ql) * a.Hq + hq) * D + kb * 16 + g * 4)
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    int qpos[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int ql = q_lo + w * WQ + nt * 16 + c16;
        qpos[nt] = ql < P ? (a.causal ? wk.hist + ql : L - 1) : -1;
    }
    const int wq0 = q_lo + w * WQ;
    const int wave_min_pos = (wq0 + WQ <= P) ? (a.causal ? wk.hist + wq0 : L - 1) : -1;

    f32x4 o[DT][2];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) o[dt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m[2] = {kNegBig, kNegBig};
    float lsum[2] = {0.f, 0.f};   // this lane's keys only

    int tbase = 0;
    u32x4 kr[KCH_T];
    u32x4 vr[VT_T][4];
    const uint32_t row_bytes = (uint32_t)(a.Hkv * D * sizeof(float));
    const uint32_t page_bytes = row_bytes * kPage;
    const int64_t kv0 = (int64_t)kvh * D + (CG ? (int64_t)wk.kvo : 0);
    const char* kb_ = reinterpret_cast<const char*>(reinterpret_cast<const float*>(a.k) + kv0);
    const char* vb_ = reinterpret_cast<const char*>(reinterpret_cast<const float*>(a.v) + kv0);
    uint32_t koff[KCH_T], voff[VT_T];
    int kslot[KCH_T], vslot[VT_T];
#pragma unroll
    for (int j = 0; j < KCH_T; ++j) {
        const int ch = tid + 256 * j;
        const int key = ch / (D / 4), c = ch % (D / 4);
        kslot[j] = CG ? key : key >> 4;   // contiguous K/V: the key within the tile
        koff[j] = (CG ? 0u : (uint32_t)(key & 15) * row_bytes) + (uint32_t)c * 16u;
    }
#pragma unroll
    for (int j = 0; j < VT_T; ++j) {
        const int task = (VT_N % 256 == 0 || tid + 256 * j < VT_N) ? tid + 256 * j : 0;   // idle: task 0's rows
        const int kq = task % (BN / 4), c = task / (BN / 4);   // keys 4kq .. 4kq+3, dims 4c .. 4c+3
        vslot[j] = CG ? 4 * kq : (4 * kq) >> 4;
        voff[j] = (CG ? 0u : (uint32_t)((4 * kq) & 15) * row_bytes) + (uint32_t)c * 16u;
    }
    // Next-tile staging in two halves (K, then V^T), so that only one half's
    // registers are live at a time.
    auto load_k = [&](int t) {
        if constexpr (CG) {   // rows past the sequence's last are staged as the last
#pragma unroll
            for (int j = 0; j < KCH_T; ++j)
                kr[j] = *reinterpret_cast<const u32x4*>(
                    kb_ + (uint64_t)min(t * BN + kslot[j], L - 1) * row_bytes + koff[j]);
            return;
        }
        const int* pg = sm.pages + (4 * t - tbase);
#pragma unroll
        for (int j = 0; j < KCH_T; ++j) {
            const uint64_t phys = (uint32_t)max(pg[kslot[j]], 0);
            kr[j] = *reinterpret_cast<const u32x4*>(kb_ + phys * page_bytes + koff[j]);
        }
    };
    auto load_v = [&](int t) {
        if constexpr (CG) {
#pragma unroll
            for (int j = 0; j < VT_T; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    vr[j][r] = *reinterpret_cast<const u32x4*>(
                        vb_ + (uint64_t)min(t * BN + vslot[j] + r, L - 1) * row_bytes + voff[j]);
            return;
        }
        const int* pg = sm.pages + (4 * t - tbase);
#pragma unroll
        for (int j = 0; j < VT_T; ++j) {
            const uint64_t phys = (uint32_t)max(pg[vslot[j]], 0);
            const char* p = vb_ + phys * page_bytes + voff[j];
#pragma unroll
            for (int r = 0; r < 4; ++r) vr[j][r] = *reinterpret_cast<const u32x4*>(p + r * row_bytes);
        }
    };
    auto store_k = [&](int buf) {
#pragma unroll
        for (int j = 0; j < KCH_T; ++j) {
            const int ch = tid + 256 * j;
            const int key = ch / (D / 4), c = ch % (D / 4);
            *reinterpret_cast<u32x4*>(&sm.k[buf][key * KPAD + c * 4]) = kr[j];
        }
    };
    auto store_v = [&](int buf) {
#pragma unroll
        for (int j = 0; j < VT_T; ++j) {
            const int task = tid + 256 * j;
            if (VT_N % 256 != 0 && task >= VT_N) break;
            const int kq = task % (BN / 4), c = task / (BN / 4);
#pragma unroll
            for (int e = 0; e < 4; ++e)   // 4x4 transpose: V^T row 4c + e, keys 4kq .. 4kq+3
                *reinterpret_cast<u32x4*>(&sm.vt[buf][(4 * c + e) * VPAD + 4 * kq]) =
                    u32x4{vr[j][0][e], vr[j][1][e], vr[j][2][e], vr[j][3][e]};
        }
    };
    auto stage_pages = [&](int base) {
        if constexpr (CG) return;   // no page table
        tbase = base;
        for (int i = tid; i < kPageWindow; i += 256) sm.pages[i] = bt[min(base + i, last_page)];
        lds_barrier();
    };
    if (t_begin < t_end) {
        stage_pages(4 * t_begin);
        load_q();
        load_k(t_begin);
        load_v(t_begin);
        store_k(0);
        store_v(0);
    }
    __syncthreads();

    for (int t = t_begin; t < t_end; ++t) {
        const int kbuf = KNB == 2 ? (t - t_begin) & 1 : 0;
        const int vbuf = VNB == 2 ? (t - t_begin) & 1 : 0;
        const bool next = t + 1 < t_end;   // uniform
        if (next) {
            if (4 * (t + 1) + 4 > tbase + kPageWindow) stage_pages(4 * (t + 1));
            load_k(t + 1);
        }
        __builtin_amdgcn_sched_barrier(0);

        LLKV_PF_PRIO(true, 1);
        // ---- S^T = K Q^T: key tile kt holds keys 16kt .. 16kt+15 ---------
        // The two halves of the head dims accumulate apart and are added at
        // the end: half the rounding steps in each sum, which halves the
        // score's rounding error (it dominates the fp32 output's error).
        f32x4 s[4][2];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            f32x4 hi[2];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                s[kt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
                hi[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                const float4 ka = *reinterpret_cast<const float4*>(
                    &sm.k[kbuf][(16 * kt + c16) * KPAD + kb * 16 + g * 4]);
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    f32x4& acc = kb < KB / 2 ? s[kt][nt] : hi[nt];
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.x, qop[nt][kb].x, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.y, qop[nt][kb].y, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.z, qop[nt][kb].z, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.w, qop[nt][kb].w, acc, 0, 0, 0);
                }
            }
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) s[kt][nt] += hi[nt];
        }
        LLKV_PF_PRIO(true, 0);
        if (next) {
            if (KNB == 1) __syncthreads();   // every wave is done with the K buffer
            store_k(KNB == 2 ? kbuf ^ 1 : 0);
            load_v(t + 1);
        }

        // ---- mask and online softmax (scores scaled in the exponent) -----
        const int key0 = t * BN;
        const float c = a.scale_log2;
        const bool unmasked = key0 + BN - 1 <= wave_min_pos && key0 + BN <= kend;
        float mx[2];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            if (!unmasked) {
                // key = key0 + 16kt + 4g + i is visible iff key <= min(qpos, kend - 1)
                const int r = min(qpos[nt], kend - 1) - key0 - 4 * g;
#pragma unroll
                for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (16 * kt + i > r) s[kt][nt][i] = -INFINITY;
            }
            float v = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) v = fmaxf(v, s[kt][nt][i]);
            mx[nt] = v * c;
        }
        bool grow = false;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) grow |= mx[nt] > m[nt] + 8.0f;
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                float v = mx[nt];
                v = fmaxf(v, __shfl_xor(v, 16, 64));
                v = fmaxf(v, __shfl_xor(v, 32, 64));
                const float mnew = fmaxf(m[nt], v);
                const float corr = fast_exp2(m[nt] - mnew);
                m[nt] = mnew;
                lsum[nt] *= corr;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) o[dt][nt] *= corr;
            }
        }
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float p = fast_exp2(fmaf(s[kt][nt][i], c, -m[nt]));
                    s[kt][nt][i] = p;
                    lsum[nt] += p;
                }

        // ---- O^T += V^T P^T ------------------------------------------------
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const float4 va = *reinterpret_cast<const float4*>(
                    &sm.vt[vbuf][(dt * 16 + c16) * VPAD + 16 * kt + 4 * g]);
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    o[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(va.x, s[kt][nt][0], o[dt][nt], 0, 0, 0);
                    o[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(va.y, s[kt][nt][1], o[dt][nt], 0, 0, 0);
                    o[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(va.z, s[kt][nt][2], o[dt][nt], 0, 0, 0);
                    o[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(va.w, s[kt][nt][3], o[dt][nt], 0, 0, 0);
                }
            }
        }

        if (next) {
            if (VNB == 1) __syncthreads();   // every wave is done with the V^T buffer
            store_v(VNB == 2 ? vbuf ^ 1 : 0);
        }
        __syncthreads();
    }

    float* og = reinterpret_cast<float*>(a.out);
    const int64_t pidx = ((int64_t)unit * a.max_chunks + ci) * a.Hq + hq;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        float lt = lsum[nt];
        lt += __shfl_xor(lt, 16, 64);
        lt += __shfl_xor(lt, 32, 64);
        const int row = w * WQ + nt * 16 + c16;
        const int ql = q_lo + row;
        if (ql >= P) continue;
        const float inv = lt > 0.f ? 1.0f / lt : 0.f;
        float* dst = wk.direct ? og + ((int64_t)(q0 + ql) * a.Hq + hq) * D
                               : a.part_o + (pidx * BQ + row) * D;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
            *reinterpret_cast<float4*>(dst + dt * 16 + 4 * g) =
                make_float4(o[dt][nt][0] * inv, o[dt][nt][1] * inv, o[dt][nt][2] * inv, o[dt][nt][3] * inv);
        if (!wk.direct && g == 0) a.part_lse[pidx * BQ + row] = lt > 0.f ? m[nt] + fast_log2(lt) : -INFINITY;
    }
}

// Four consecutive output elements from fp32 values.
template <typename T>
__device__ inline void store4(T* p, float x, float y, float z, float w) {
    uint2 w2;
    w2.x = Mfma<T>::pack2(x, y);
    w2.y = Mfma<T>::pack2(z, w);
    *reinterpret_cast<uint2*>(p) = w2;
}
template <>
__device__ inline void store4<float>(float* p, float x, float y, float z, float w) {
    *reinterpret_cast<float4*>(p) = make_float4(x, y, z, w);
}

// Merge of a (sequence, query block, q head) unit's key chunks: grid
// (Hq, N x qblocks), 256 threads; thread (row, part) merges dims
// [part * D/TPR, (part + 1) * D/TPR) of one row over the chunks with an online
// log-sum-exp (each chunk's lse and row slice are loaded together).
template <typename T, int D>
__global__ __launch_bounds__(256) void prefill_merge_kernel(MfmaPrefillArgs a) {
    // The main kernel's split decision; loaded together with the lengths below
    // and checked before anything is read or written.
    const int unsplit = *a.plan_flag;
    constexpr int TPR = 256 / BQ;     // threads per row
    constexpr int V4 = D / TPR / 4;   // float4 per thread
    const int hq = blockIdx.x, unit = blockIdx.y;
    const int n = unit / a.qblocks;
    const int qb = a.qblocks - 1 - (unit % a.qblocks);
    int q0, P, L, kvo, hist;
    seq_geom(a, n, q0, P, L, kvo, hist);
    if (unsplit != 0) return;   // every row was written by the main kernel
    const int q_lo = qb * BQ;
    const int row = threadIdx.x / TPR, part = threadIdx.x % TPR;
    if (q_lo + row >= P) return;
    int kend = a.causal ? hist + min(q_lo + BQ, P) : L;
    kend = kend < 0 ? 0 : (kend > L ? L : kend);
    const int ntiles = (kend + BN - 1) / BN;
    const int nchunks = min((ntiles + a.chunk_tiles - 1) / a.chunk_tiles, a.max_chunks);   // as take_work
    if (nchunks <= 1) return;   // written directly
    const int64_t p0 = ((int64_t)unit * a.max_chunks) * a.Hq + hq;   // chunk c at p0 + c * Hq
    float M = -INFINITY, W = 0.0f;
    float4 acc[V4];
#pragma unroll
    for (int v = 0; v < V4; ++v) acc[v] = make_float4(0.f, 0.f, 0.f, 0.f);
    // CB chunks per memory round trip: every load of a batch is issued before
    // any of its values is used (chunks past nchunks load the last one and take
    // lse -inf), and the merge step has no branch, so the compiler cannot sink
    // the row loads behind the lse.  A chunk whose row saw no key has lse -inf
    // and a zero row: weight 0, no change.  Two chunks per batch: the plan cuts
    // most split units in two, and fp32 rows of four chunks held 128 registers
    // and loaded the last chunk three times (configuration 4 57.6 -> 56.9 us).
    constexpr int CB = 2;
    for (int c0 = 0; c0 < nchunks; c0 += CB) {
        float l[CB];
        float4 raw[CB][V4];
#pragma unroll
        for (int k = 0; k < CB; ++k) {
            const int c = min(c0 + k, nchunks - 1);
            const int64_t pc = (p0 + (int64_t)c * a.Hq) * BQ + row;
            const float lk = a.part_lse[pc];
            l[k] = c0 + k < nchunks ? lk : -INFINITY;
            const float4* src = reinterpret_cast<const float4*>(a.part_o + pc * D) + part * V4;
#pragma unroll
            for (int v = 0; v < V4; ++v) raw[k][v] = src[v];
        }
#pragma unroll
        for (int k = 0; k < CB; ++k) {
            const float4* o = raw[k];
            const float Mn = fmaxf(M, l[k]);
            const bool live = Mn != -INFINITY;   // some key seen by this row so far
            const float sc = live ? fast_exp2(M - Mn) : 1.0f;
            const float wt = live ? fast_exp2(l[k] - Mn) : 0.0f;
            W = fmaf(W, sc, wt);
#pragma unroll
            for (int v = 0; v < V4; ++v) {
                acc[v].x = fmaf(acc[v].x, sc, wt * o[v].x);
                acc[v].y = fmaf(acc[v].y, sc, wt * o[v].y);
                acc[v].z = fmaf(acc[v].z, sc, wt * o[v].z);
                acc[v].w = fmaf(acc[v].w, sc, wt * o[v].w);
            }
            M = live ? Mn : M;
        }
    }
    const float inv = W > 0.f ? 1.0f / W : 0.f;
    T* orow = reinterpret_cast<T*>(a.out) + ((int64_t)(q0 + q_lo + row) * a.Hq + hq) * D + part * V4 * 4;
#pragma unroll
    for (int v = 0; v < V4; ++v)
        store4(orow + 4 * v, acc[v].x * inv, acc[v].y * inv, acc[v].z * inv, acc[v].w * inv);
}

bool prefill_mfma_handles(int head_dim, int block_size, int dtype) {
    // head_dim 256: one work-group per CU (fp32: single-buffered tiles, 134 KB)
    return block_size == kPage && (head_dim == 64 || head_dim == 96 || head_dim == 128 || head_dim == 256);
}

// Key-range split.  When the (sequence, query block, q head) units alone
// would leave the GPU idle, a unit's key tiles are cut into chunks of
// ceil(max_tiles / k) tiles, k chosen so that the launch offers about kFill
// work-groups per resident slot (counted as if every unit had the longest key
// range), with chunks of at least kMinChunkTiles tiles.  With enough units
// (k = 1) nothing is split: no partials and no merge.  The workspace is sized
// from the shape alone, for kSizingSlots resident slots (256 CUs x 4
// work-groups, above what this kernel reaches); a launch takes the smaller of
// that k and the one of its device's actual resident count.  About one
// work-group per slot: with fp32 partials, configuration 4 runs two chunks
// per long unit at 58.1 us against 59.8 us for three (1.5 per slot) and
// 80 us for two per slot; the fewer chunks, the less partial traffic.
constexpr double kFill = 1.0;
constexpr int kMinChunkTiles = 8;
constexpr int kSizingSlots = 1024;

typedef void (*PrefillFn)(MfmaPrefillArgs);

template <typename T, bool CG>
PrefillFn kernel16(int head_dim) {
    switch (head_dim) {
        case 64: return prefill_mfma_kernel<T, 64, CG>;
        case 96: return prefill_mfma_kernel<T, 96, CG>;
        case 128: return prefill_mfma_kernel<T, 128, CG>;
        default: return prefill_mfma_kernel<T, 256, CG>;
    }
}

template <bool CG>
PrefillFn kernel32(int head_dim) {
    switch (head_dim) {
        case 64: return prefill_f32_kernel<64, CG>;
        case 96: return prefill_f32_kernel<96, CG>;
        case 128: return prefill_f32_kernel<128, CG>;
        default: return prefill_f32_kernel<256, CG>;
    }
}

template <bool CG>
PrefillFn prefill_kernel_cg(int dtype, int head_dim) {
    if (dtype == LLKV_DTYPE_F32) return kernel32<CG>(head_dim);
    if (dtype == LLKV_DTYPE_F16) return kernel16<_Float16, CG>(head_dim);
    return kernel16<bf16_t, CG>(head_dim);
}

PrefillFn prefill_kernel(int dtype, int head_dim, bool contig) {
    return contig ? prefill_kernel_cg<true>(dtype, head_dim) : prefill_kernel_cg<false>(dtype, head_dim);
}

template <typename T>
PrefillFn merge_for(int head_dim) {
    switch (head_dim) {
        case 64: return prefill_merge_kernel<T, 64>;
        case 96: return prefill_merge_kernel<T, 96>;
        case 128: return prefill_merge_kernel<T, 128>;
        default: return prefill_merge_kernel<T, 256>;
    }
}

PrefillFn merge_kernel(int dtype, int head_dim) {
    if (dtype == LLKV_DTYPE_F32) return merge_for<float>(head_dim);
    if (dtype == LLKV_DTYPE_F16) return merge_for<_Float16>(head_dim);
    return merge_for<bf16_t>(head_dim);
}

// Workspace header: the main kernel's split decision (one int), read by the
// merge kernel.
constexpr size_t kPlanHeaderBytes = 256;

struct ChunkPlan {
    int qblocks, max_chunks, chunk_tiles;
};

// slots <= 0: size for kSizingSlots; otherwise the launch plan for that many
// resident slots (never more chunks than the sizing plan).
ChunkPlan chunk_plan(int N, int Hq, int total_q, int max_q_len, int max_seq_len, int slots) {
    ChunkPlan c;
    const int qmax = (max_q_len > 0 && max_q_len < total_q) ? max_q_len : total_q;
    c.qblocks = (qmax + BQ - 1) / BQ;
    const int max_tiles = (std::max(max_seq_len, 1) + BN - 1) / BN;
    const double unit_heads = (double)N * c.qblocks * Hq;
    auto splits = [&](int s) {
        int k = (int)std::ceil(kFill * s / unit_heads);
        k = std::min(k, std::max(1, max_tiles / kMinChunkTiles));
        return std::max(k, 1);
    };
    int k = splits(kSizingSlots);
    if (slots > 0) k = std::min(k, splits(slots));
    c.chunk_tiles = (max_tiles + k - 1) / k;
    c.max_chunks = (max_tiles + c.chunk_tiles - 1) / c.chunk_tiles;
    return c;
}

}  // namespace

size_t prefill_mfma_workspace(int N, int Hq, int head_dim, int block_size, int dtype, int total_q,
                              int max_q_len, int max_seq_len) {
    if (!prefill_mfma_handles(head_dim, block_size, dtype) || N <= 0 || total_q <= 0) return 0;
    const ChunkPlan c = chunk_plan(N, Hq, total_q, max_q_len, max_seq_len, 0);
    if (c.max_chunks <= 1) return 0;
    const size_t parts = (size_t)N * c.qblocks * c.max_chunks * Hq;
    return kPlanHeaderBytes + parts * BQ * sizeof(float) + parts * BQ * head_dim * sizeof(float);
}

int launch_prefill_mfma(MfmaPrefillArgs a, int head_dim, int block_size, int dtype,
                        int total_q, int max_q_len, int max_seq_len, void* workspace,
                        size_t workspace_bytes, hipStream_t st) {
    if (!prefill_mfma_handles(head_dim, block_size, dtype)) return -1;
    if (((uintptr_t)a.q | (uintptr_t)a.out | (uintptr_t)a.k | (uintptr_t)a.v) & 15) return -1;
    const int slots = resident_workgroups(reinterpret_cast<const void*>(prefill_kernel(dtype, head_dim, false)), 256);
    const ChunkPlan c = chunk_plan(a.N, a.Hq, total_q, max_q_len, max_seq_len, slots);
    a.qblocks = c.qblocks;
    const size_t need = prefill_mfma_workspace(a.N, a.Hq, head_dim, block_size, dtype, total_q,
                                               max_q_len, max_seq_len);
    if (c.max_chunks > 1 && workspace != nullptr && workspace_bytes >= need) {
        // partials laid out for the sizing plan's chunk count (>= this plan's)
        const ChunkPlan z = chunk_plan(a.N, a.Hq, total_q, max_q_len, max_seq_len, 0);
        const size_t parts = (size_t)a.N * z.qblocks * z.max_chunks * a.Hq;
        a.max_chunks = c.max_chunks;
        a.chunk_tiles = c.chunk_tiles;
        char* base = reinterpret_cast<char*>(workspace);
        a.plan_flag = reinterpret_cast<int*>(base);
        a.part_lse = reinterpret_cast<float*>(base + kPlanHeaderBytes);
        a.part_o = reinterpret_cast<float*>(base + kPlanHeaderBytes + parts * BQ * sizeof(float));
    } else {   // no split, or no (or too small a) workspace: one chunk per unit
        a.max_chunks = 1;
        a.chunk_tiles = 1 << 30;
        a.part_lse = nullptr;
        a.part_o = nullptr;
        a.plan_flag = nullptr;
    }
    a.n_cus = device_cus();
    a.resident = a.contig ? resident_workgroups(reinterpret_cast<const void*>(prefill_kernel(dtype, head_dim, true)), 256)
                          : slots;
    a.groups = a.N * a.qblocks * a.max_chunks * a.Hkv;
    const int G = a.Hq / a.Hkv;
    dim3 grid((unsigned)(((a.groups + kXcds - 1) / kXcds) * kXcds * G));
    dim3 mgrid(a.Hq, a.N * a.qblocks);
    prefill_kernel(dtype, head_dim, a.contig != 0)<<<grid, 256, 0, st>>>(a);
    if (a.max_chunks > 1) merge_kernel(dtype, head_dim)<<<mgrid, 256, 0, st>>>(a);
    return check_launch(a.contig ? "llkv_first_prefill_batched" : "llkv_paged_prefill");
}

}  // namespace llkv
