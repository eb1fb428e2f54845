// Device-side slot mapping and fused RoPE + KV append for gfx950.
//
// llkv_build_slots turns (block table, token ranges, start positions) into the
// int64 slot mapping on the device: one lane per token, a binary search over
// the token ranges, one table load.
//
// llkv_rope_append is one HBM-bound pass over the step's new rows: q rows are
// rotated in place, k rows are rotated in place and written to their pool
// slot, the rest of each k row and the v rows are copied to the pool.  Work
// items are 16-byte units (4 fp32 or 8 fp16/bf16 elements; pairs (i, i+half)
// of a rotation are one item), in one flat grid-stride index space:
//     [q pairs | k pairs | k tail | v row units]
// so every lane issues 16-byte loads and stores whatever the head layout.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.h"

namespace llkv {
namespace {

// Neox rotation of one pair in fp32, each product and each sum rounded on
// its own (the form of rope.cu:54-57 without fused multiply-adds, so the
// result does not depend on the compiler's contraction choices).
__device__ inline void rotate(float x1, float x2, float c, float s, float& o1, float& o2) {
#pragma clang fp contract(off)
    const float a = x1 * c;
    const float b = x2 * s;
    const float d = x2 * c;
    const float e = x1 * s;
    o1 = a - b;
    o2 = d + e;
}

struct RopeArgs {
    void* q;
    void* k;
    const void* v;
    void* kp;
    void* vp;
    const int64_t* slots;
    const float* cos;
    const float* sin;
    int T, Hq, Hkv, D, half;
};

// One 16-byte unit of element type T: VEC elements as fp32.
template <typename T>
struct Unit {
    static constexpr int VEC = Chunk<T>::VEC;
    __device__ static void load(const T* p, float* f) {
        Chunk<T>::unpack(*reinterpret_cast<const uint4*>(p), f);
    }
    __device__ static void store(T* p, const float* f) {
        *reinterpret_cast<uint4*>(p) = Chunk<T>::pack(f);
    }
    __device__ static void copy(T* dst, const T* src) {
        *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
    }
};

// Scalar fallback (rows or pointers not 16-byte aligned, or half not a
// multiple of the vector width).
template <typename T>
struct Unit1 {
    static constexpr int VEC = 1;
    __device__ static void load(const T* p, float* f) { f[0] = Elem<T>::to_f32(*p); }
    __device__ static void store(T* p, const float* f) { *p = Elem<T>::from_f32(f[0]); }
    __device__ static void copy(T* dst, const T* src) { *dst = *src; }
};

template <typename T, class U>
__global__ __launch_bounds__(256) void rope_append_kernel(RopeArgs a) {
    constexpr int W = U::VEC;
    // Unit indices fit 32 bits (checked on the host), so the index arithmetic
    // below is 32-bit; row offsets are 64-bit.
    const uint32_t hu = a.half / W;                 // rotation units per head row
    const uint32_t tu = (a.D - 2 * a.half) / W;     // unrotated tail units per head row
    const uint32_t du = a.D / W;                    // units per head row
    const uint32_t nA = a.q ? (uint32_t)a.T * a.Hq * hu : 0u;
    const uint32_t nB = (uint32_t)a.T * a.Hkv * hu;
    const uint32_t nC = (uint32_t)a.T * a.Hkv * tu;
    const uint32_t nD = (uint32_t)a.T * a.Hkv * du;
    const uint32_t total = nA + nB + nC + nD;
    T* q = reinterpret_cast<T*>(a.q);
    T* k = reinterpret_cast<T*>(a.k);
    const T* v = reinterpret_cast<const T*>(a.v);
    T* kp = reinterpret_cast<T*>(a.kp);
    T* vp = reinterpret_cast<T*>(a.vp);

    for (uint32_t u = blockIdx.x * blockDim.x + threadIdx.x; u < total; u += gridDim.x * blockDim.x) {
        if (u < nA + nB) {   // rotate a q or k pair unit
            const bool isq = u < nA;
            const uint32_t r = isq ? u : u - nA;
            const uint32_t H = isq ? a.Hq : a.Hkv;
            const uint32_t th = r / hu;   // token * H + head
            const int i0 = (int)(r - th * hu) * W;
            const uint32_t t = th / H;
            T* row = (isq ? q : k) + (int64_t)th * a.D;
            float x1[W], x2[W], c[W], s[W], o1[W], o2[W];
            U::load(row + i0, x1);
            U::load(row + a.half + i0, x2);
            const float* cp = a.cos + (int64_t)t * a.half + i0;
            const float* sp = a.sin + (int64_t)t * a.half + i0;
#pragma unroll
            for (int e = 0; e < W; ++e) {
                c[e] = cp[e];
                s[e] = sp[e];
            }
#pragma unroll
            for (int e = 0; e < W; ++e) rotate(x1[e], x2[e], c[e], s[e], o1[e], o2[e]);
            U::store(row + i0, o1);
            U::store(row + a.half + i0, o2);
            if (!isq) {
                const int64_t slot = a.slots[t];
                if (slot >= 0) {
                    T* prow = kp + (slot * a.Hkv + (th - t * a.Hkv)) * a.D;
                    U::store(prow + i0, o1);
                    U::store(prow + a.half + i0, o2);
                }
            }
        } else {   // copy a k tail unit or a v unit to the pool
            const bool isk = u < nA + nB + nC;
            const uint32_t r = isk ? u - nA - nB : u - nA - nB - nC;
            const uint32_t per = isk ? tu : du;
            const uint32_t th = r / per;
            const int j = (int)(r - th * per);
            const uint32_t t = th / a.Hkv;
            const int64_t slot = a.slots[t];
            if (slot < 0) continue;
            const int off = (isk ? 2 * a.half : 0) + j * W;
            const int64_t dst = (slot * a.Hkv + (th - t * a.Hkv)) * a.D + off;
            if (isk) U::copy(kp + dst, k + (int64_t)th * a.D + off);
            else U::copy(vp + dst, v + (int64_t)th * a.D + off);
        }
    }
}

__device__ inline int find_range(const int* cum, int n, int g) {
    // largest e in [0, n) with cum[e] <= g
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (cum[mid] <= g) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

__global__ __launch_bounds__(256) void build_slots_kernel(int64_t* slots, const int* bt, int max_blocks,
                                                          const int* cu, const int* start, int n,
                                                          int T, int bs) {
    for (int t = blockIdx.x * blockDim.x + threadIdx.x; t < T; t += gridDim.x * blockDim.x) {
        const int e = find_range(cu, n, t);
        const int pos = start[e] + (t - cu[e]);
        int64_t slot = -1;
        if (pos >= 0 && pos / bs < max_blocks) {
            const int phys = bt[(int64_t)e * max_blocks + pos / bs];
            if (phys >= 0) slot = (int64_t)phys * bs + pos % bs;
        }
        slots[t] = slot;
    }
}

int grid_for(int64_t items) {
    return (int)std::max<int64_t>(1, std::min<int64_t>((items + 255) / 256, 16384));
}

template <typename T>
int launch_rope(const RopeArgs& a, bool vec, hipStream_t st) {
    const int W = vec ? Chunk<T>::VEC : 1;
    const int64_t items = (int64_t)a.T * ((a.q ? a.Hq : 0) + 2 * a.Hkv) * (a.D / W);
    if (vec) rope_append_kernel<T, Unit<T>><<<grid_for(items), 256, 0, st>>>(a);
    else rope_append_kernel<T, Unit1<T>><<<grid_for(items), 256, 0, st>>>(a);
    return check_launch("llkv_rope_append");
}

}  // namespace
}  // namespace llkv

using namespace llkv;

extern "C" int llkv_build_slots(int64_t* slots, const int* block_table, int max_blocks,
                                const int* cu_tokens, const int* start_pos, int num_seqs,
                                int num_tokens, int block_size, void* stream) {
    const char* fn = "llkv_build_slots";
    if (num_tokens == 0) return LLKV_OK;
    if (num_tokens < 0 || num_seqs <= 0 || max_blocks <= 0 || block_size <= 0)
        return set_error(LLKV_ERR_INVALID, "%s: bad shape arguments", fn);
    if (!slots || !block_table || !cu_tokens || !start_pos)
        return set_error(LLKV_ERR_INVALID, "%s: null pointer", fn);
    build_slots_kernel<<<grid_for(num_tokens), 256, 0, (hipStream_t)stream>>>(
        slots, block_table, max_blocks, cu_tokens, start_pos, num_seqs, num_tokens, block_size);
    return check_launch(fn);
}

extern "C" int llkv_rope_append(void* q, void* k, const void* v, void* k_pool, void* v_pool,
                                const int64_t* slot_mapping, const float* cos, const float* sin,
                                int num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                                int rotary_dim, int dtype, void* stream) {
    const char* fn = "llkv_rope_append";
    if (num_tokens == 0) return LLKV_OK;
    if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || (q && num_q_heads <= 0))
        return set_error(LLKV_ERR_INVALID, "%s: bad shape arguments", fn);
    if (rotary_dim < 2 || rotary_dim > head_dim || rotary_dim % 2 != 0)
        return set_error(LLKV_ERR_INVALID, "%s: rotary_dim %d must be even and in [2, %d]", fn,
                         rotary_dim, head_dim);
    const size_t es = dtype_bytes(dtype);
    if (es == 0) return set_error(LLKV_ERR_INVALID, "%s: unsupported dtype %d", fn, dtype);
    if (!k || !v || !k_pool || !v_pool || !slot_mapping || !cos || !sin)
        return set_error(LLKV_ERR_INVALID, "%s: null pointer", fn);
    RopeArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.kp = k_pool;
    a.vp = v_pool;
    a.slots = slot_mapping;
    a.cos = cos;
    a.sin = sin;
    a.T = num_tokens;
    a.Hq = num_q_heads;
    a.Hkv = num_kv_heads;
    a.D = head_dim;
    a.half = rotary_dim / 2;
    const int W = (int)(16 / es);
    if ((uint64_t)num_tokens * ((q ? (uint64_t)num_q_heads : 0) + 2ull * num_kv_heads) * head_dim >= (1ull << 31))
        return set_error(LLKV_ERR_UNSUPPORTED, "%s: 2^31 or more elements in one call", fn);
    const bool vec = a.half % W == 0 && head_dim % W == 0 &&
                     (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)k_pool |
                       (uintptr_t)v_pool | (uintptr_t)cos | (uintptr_t)sin) & 15) == 0;
    hipStream_t st = (hipStream_t)stream;
    if (dtype == LLKV_DTYPE_F32) return launch_rope<float>(a, vec, st);
    if (dtype == LLKV_DTYPE_F16) return launch_rope<_Float16>(a, vec, st);
    return launch_rope<bf16_t>(a, vec, st);
}
