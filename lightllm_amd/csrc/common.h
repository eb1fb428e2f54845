// Shared device/host helpers for the gfx950 paged KV-cache kernels.
//
// Element types: F32 (float), F16 (_Float16), BF16 (bit pattern in uint16_t).
// All arithmetic is carried in fp32; conversions happen on load/store.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lightllm_kv.h"

namespace llkv {

// ---------------------------------------------------------------------------
// Element traits
// ---------------------------------------------------------------------------
struct bf16_t {
    uint16_t bits;
};

template <typename T> struct Elem;

template <> struct Elem<float> {
    static constexpr int kDtype = LLKV_DTYPE_F32;
    __device__ static inline float to_f32(float x) { return x; }
    __device__ static inline float from_f32(float x) { return x; }
};

template <> struct Elem<_Float16> {
    static constexpr int kDtype = LLKV_DTYPE_F16;
    __device__ static inline float to_f32(_Float16 x) { return (float)x; }
    __device__ static inline _Float16 from_f32(float x) { return (_Float16)x; }
};

template <> struct Elem<bf16_t> {
    static constexpr int kDtype = LLKV_DTYPE_BF16;
    __device__ static inline float to_f32(bf16_t x) {
        return __uint_as_float((uint32_t)x.bits << 16);
    }
    // Round to nearest even; NaN stays NaN (quiet bit set).
    __device__ static inline bf16_t from_f32(float x) {
        uint32_t u = __float_as_uint(x);
        bf16_t r;
        if ((u & 0x7FFFFFFFu) > 0x7F800000u) {
            r.bits = (uint16_t)((u >> 16) | 0x40u);
        } else {
            u += 0x7FFFu + ((u >> 16) & 1u);
            r.bits = (uint16_t)(u >> 16);
        }
        return r;
    }
};

// Unpack a 16-byte chunk (uint4) into VEC fp32 values.
template <typename T> struct Chunk;

template <> struct Chunk<float> {
    static constexpr int VEC = 4;
    __device__ static inline void unpack(const uint4& c, float* f) {
        f[0] = __uint_as_float(c.x);
        f[1] = __uint_as_float(c.y);
        f[2] = __uint_as_float(c.z);
        f[3] = __uint_as_float(c.w);
    }
    __device__ static inline uint4 pack(const float* f) {
        return make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]),
                          __float_as_uint(f[2]), __float_as_uint(f[3]));
    }
};

typedef _Float16 half2_v __attribute__((ext_vector_type(2)));

__device__ inline void unpack_h2(uint32_t w, float* f) {
    half2_v h = __builtin_bit_cast(half2_v, w);
    f[0] = (float)h.x;
    f[1] = (float)h.y;
}
__device__ inline uint32_t pack_h2(float a, float b) {
    half2_v h;
    h.x = (_Float16)a;
    h.y = (_Float16)b;
    return __builtin_bit_cast(uint32_t, h);
}

template <> struct Chunk<_Float16> {
    static constexpr int VEC = 8;
    __device__ static inline void unpack(const uint4& c, float* f) {
        unpack_h2(c.x, f + 0);
        unpack_h2(c.y, f + 2);
        unpack_h2(c.z, f + 4);
        unpack_h2(c.w, f + 6);
    }
    __device__ static inline uint4 pack(const float* f) {
        return make_uint4(pack_h2(f[0], f[1]), pack_h2(f[2], f[3]),
                          pack_h2(f[4], f[5]), pack_h2(f[6], f[7]));
    }
};

__device__ inline void unpack_b2(uint32_t w, float* f) {
    f[0] = __uint_as_float(w << 16);
    f[1] = __uint_as_float(w & 0xFFFF0000u);
}
__device__ inline uint32_t pack_b2(float a, float b) {
    uint32_t lo = Elem<bf16_t>::from_f32(a).bits;
    uint32_t hi = Elem<bf16_t>::from_f32(b).bits;
    return lo | (hi << 16);
}

template <> struct Chunk<bf16_t> {
    static constexpr int VEC = 8;
    __device__ static inline void unpack(const uint4& c, float* f) {
        unpack_b2(c.x, f + 0);
        unpack_b2(c.y, f + 2);
        unpack_b2(c.z, f + 4);
        unpack_b2(c.w, f + 6);
    }
    __device__ static inline uint4 pack(const float* f) {
        return make_uint4(pack_b2(f[0], f[1]), pack_b2(f[2], f[3]),
                          pack_b2(f[4], f[5]), pack_b2(f[6], f[7]));
    }
};

// ---------------------------------------------------------------------------
// Wave64 cross-lane helpers (DPP within 16-lane rows, swizzle/bpermute above)
// ---------------------------------------------------------------------------
enum : int {
    kDppQuadXor1 = 0xB1,       // quad_perm [1,0,3,2]
    kDppQuadXor2 = 0x4E,       // quad_perm [2,3,0,1]
    kDppRowHalfMirror = 0x141, // lane i <-> 7-i inside each 8-lane half-row
    kDppRowMirror = 0x140,     // lane i <-> 15-i inside each 16-lane row
};

template <int CTRL>
__device__ inline float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(
        0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of W lanes (W in 1,2,4,8,16,32,64); every lane of a
// group receives the group total.
template <int W>
__device__ inline float group_sum(float v) {
    if constexpr (W >= 2) v += dpp_f<kDppQuadXor1>(v);
    if constexpr (W >= 4) v += dpp_f<kDppQuadXor2>(v);
    if constexpr (W >= 8) v += dpp_f<kDppRowHalfMirror>(v);
    if constexpr (W >= 16) v += dpp_f<kDppRowMirror>(v);
    if constexpr (W >= 32) v += __shfl_xor(v, 16, 64);
    if constexpr (W >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

template <int W>
__device__ inline float group_max(float v) {
    if constexpr (W >= 2) v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
    if constexpr (W >= 4) v = fmaxf(v, dpp_f<kDppQuadXor2>(v));
    if constexpr (W >= 8) v = fmaxf(v, dpp_f<kDppRowHalfMirror>(v));
    if constexpr (W >= 16) v = fmaxf(v, dpp_f<kDppRowMirror>(v));
    if constexpr (W >= 32) v = fmaxf(v, __shfl_xor(v, 16, 64));
    if constexpr (W >= 64) v = fmaxf(v, __shfl_xor(v, 32, 64));
    return v;
}

__device__ inline float wave_sum(float v) { return group_sum<64>(v); }
__device__ inline float wave_max(float v) { return group_max<64>(v); }

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ inline float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kPage = 16;   // tokens per KV page (BLOCK of the reference)

}  // namespace llkv

// ---------------------------------------------------------------------------
// Host-side status plumbing shared by the C-ABI entry points.
// ---------------------------------------------------------------------------
namespace llkv {
int set_error(int status, const char* fmt, ...);
int check_launch(const char* what);
// Work-groups of `threads` threads of kernel `fn` the current device holds at
// once (compute units x resident work-groups per unit), cached per device.
int resident_workgroups(const void* fn, int threads);
// Compute units of the current device (cached per device).
int device_cus();
inline size_t dtype_bytes(int dtype) {
    return dtype == LLKV_DTYPE_F32 ? 4 : (dtype == LLKV_DTYPE_F16 || dtype == LLKV_DTYPE_BF16) ? 2 : 0;
}
}  // namespace llkv
