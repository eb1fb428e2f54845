// MFMA paged prefill attention (see prefill_mfma.h for the design).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "prefill_mfma.h"

namespace llkv {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T> struct Mfma;

template <> struct Mfma<_Float16> {
    typedef f16x8 vec;
    __device__ static inline f32x4 mma(const uint4& a, const uint4& b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                     __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
    __device__ static inline uint32_t pack2(float x, float y) { return pack_h2(x, y); }
};

template <> struct Mfma<bf16_t> {
    typedef bf16x8 vec;
    __device__ static inline f32x4 mma(const uint4& a, const uint4& b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                      __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
    __device__ static inline uint32_t pack2(float x, float y) { return pack_b2(x, y); }
};

constexpr int BQ = 128;   // query rows per work-group
constexpr int WQ = 32;    // query rows per wave (two 16-column MFMA tiles)
constexpr int BN = 64;    // keys per tile (four pages)

template <int D>
struct Smem {
    static constexpr int KPAD = D + 8;    // halves per K row (pad: spread LDS banks)
    static constexpr int VPAD = BN + 8;   // halves per V^T row
    uint16_t k[2][BN * KPAD];
    uint16_t vt[2][D * VPAD];
    int pages[1024];   // page ids [tbase, tbase + 1024) of the sequence
};

template <typename T, int D>
__global__ __launch_bounds__(256) void prefill_mfma_kernel(MfmaPrefillArgs a) {
    constexpr int KPAD = Smem<D>::KPAD, VPAD = Smem<D>::VPAD;
    constexpr int KS = D / 32;            // k-steps of the QK^T product
    constexpr int DT = D / 16;            // 16-dim tiles of the output
    constexpr int KCH = BN * D / 8;       // 16-byte K chunks per tile
    constexpr int KCH_T = KCH / 256;      // per thread
    constexpr int VT_T = (BN / 2) * (D / 8) / 256;   // V tasks (2 keys x 8 dims) per thread
    __shared__ Smem<D> sm;

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int hq = blockIdx.y;
    const int kvh = hq / (a.Hq / a.Hkv);
    const int n = blockIdx.x / a.qblocks;
    const int qb = a.qblocks - 1 - (blockIdx.x % a.qblocks);   // heavy (late) blocks first

    const int q0 = a.cu_q[n];
    const int P = a.cu_q[n + 1] - q0;
    const int q_lo = qb * BQ;
    if (q_lo >= P) return;
    int L = a.lens[n];
    const int cap = a.max_blocks * kPage;
    L = L < 0 ? 0 : (L > cap ? cap : L);
    int kend = a.causal ? L - P + min(q_lo + BQ, P) : L;
    kend = kend < 0 ? 0 : (kend > L ? L : kend);
    const int ntiles = (kend + BN - 1) / BN;
    const int last_page = L > 0 ? (L - 1) / kPage : 0;
    const int* bt = a.bt + (int64_t)n * a.max_blocks;
    const int64_t row_elems = (int64_t)a.Hkv * D;
    const T* kg = reinterpret_cast<const T*>(a.k) + (int64_t)kvh * D;
    const T* vg = reinterpret_cast<const T*>(a.v) + (int64_t)kvh * D;

    // ---- Q^T operands (B of S^T = K Q^T), kept in registers -------------
    uint4 qop[2][KS];
    const T* qg = reinterpret_cast<const T*>(a.q);
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

    // Absolute position of this lane's two query columns; rows >= P see nothing.
    int qpos[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int ql = q_lo + w * WQ + nt * 16 + c16;
        qpos[nt] = ql < P ? (a.causal ? L - P + ql : L - 1) : -1;
    }

    f32x4 o[DT][2];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) o[dt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m[2] = {kNegBig, kNegBig};
    float lsum[2] = {0.f, 0.f};

    // ---- staging: global -> registers -> LDS -----------------------------
    int tbase = 0;   // first page id held in sm.pages
    uint4 kreg[KCH_T];
    uint4 vreg[VT_T][2];
    auto load_tile = [&](int t) {
        const int key0 = t * BN;
#pragma unroll
        for (int j = 0; j < KCH_T; ++j) {
            const int ch = tid + 256 * j;
            const int key = ch / (D / 8), c = ch % (D / 8);
            const int page = min((key0 + key) >> 4, last_page);
            const int64_t row = (int64_t)max(sm.pages[page - tbase], 0) * kPage + ((key0 + key) & 15);
            kreg[j] = *reinterpret_cast<const uint4*>(kg + row * row_elems + c * 8);
        }
#pragma unroll
        for (int j = 0; j < VT_T; ++j) {
            const int task = tid + 256 * j;
            const int kp = task % (BN / 2), c = task / (BN / 2);
            const int key = key0 + 2 * kp;
            const int page = min(key >> 4, last_page);
            const int64_t row = (int64_t)max(sm.pages[page - tbase], 0) * kPage + (key & 15);
            vreg[j][0] = *reinterpret_cast<const uint4*>(vg + row * row_elems + c * 8);
            vreg[j][1] = *reinterpret_cast<const uint4*>(vg + (row + 1) * row_elems + c * 8);
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int j = 0; j < KCH_T; ++j) {
            const int ch = tid + 256 * j;
            const int key = ch / (D / 8), c = ch % (D / 8);
            *reinterpret_cast<uint4*>(&sm.k[buf][key * KPAD + c * 8]) = kreg[j];
        }
#pragma unroll
        for (int j = 0; j < VT_T; ++j) {
            const int task = tid + 256 * j;
            const int kp = task % (BN / 2), c = task / (BN / 2);
            const uint32_t* v0 = reinterpret_cast<const uint32_t*>(&vreg[j][0]);
            const uint32_t* v1 = reinterpret_cast<const uint32_t*>(&vreg[j][1]);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t lo = (v0[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
                const uint32_t hi = (v1[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
                *reinterpret_cast<uint32_t*>(&sm.vt[buf][(c * 8 + e) * VPAD + 2 * kp]) =
                    lo | (hi << 16);
            }
        }
    };

    // Page ids live in LDS so that no K/V load waits behind a table load.
    auto stage_pages = [&](int base) {
        tbase = base;
        for (int i = tid; i < 1024; i += 256) sm.pages[i] = bt[min(base + i, last_page)];
        __syncthreads();
    };
    if (ntiles > 0) {
        stage_pages(0);
        load_tile(0);
        store_tile(0);
    }
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        if (t + 1 < ntiles) {
            // tile t+1 covers pages [4(t+1), 4(t+1)+4); restage when they leave the window
            // (uniform branch; every earlier read of sm.pages preceded the last barrier)
            if (4 * (t + 1) + 4 > tbase + 1024) stage_pages(4 * (t + 1));
            load_tile(t + 1);
        }
        __builtin_amdgcn_sched_barrier(0);   // next tile's loads issue before this tile's MFMAs

        // ---- S^T = K Q^T over the 64 keys: 4 key tiles x 2 query tiles ----
        f32x4 s[4][2];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            // A row c16 of key tile kt = 2*ss + h holds key 32*ss + 8*(c16/4) + 4*h + c16%4
            const int ss = kt >> 1, h = kt & 1;
            const int krow = 32 * ss + 8 * (c16 >> 2) + 4 * h + (c16 & 3);
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) s[kt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const uint4 ka =
                    *reinterpret_cast<const uint4*>(&sm.k[buf][krow * KPAD + ks * 32 + g * 8]);
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) s[kt][nt] = Mfma<T>::mma(ka, qop[nt][ks], s[kt][nt]);
            }
        }

        // ---- scale, mask, online softmax (per query column) ---------------
        const int key0 = t * BN;
        uint4 pop[2][2];   // P^T operands [k-step][query tile]
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            float mx = kNegBig;
            float sv[4][4];
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
                const int ss = kt >> 1, h = kt & 1;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int key = key0 + 32 * ss + 8 * g + 4 * h + i;
                    const float x = s[kt][nt][i] * a.scale_log2;
                    sv[kt][i] = (key <= qpos[nt] && key < kend) ? x : -INFINITY;
                    mx = fmaxf(mx, sv[kt][i]);
                }
            }
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mnew = fmaxf(m[nt], mx);
            const float corr = fast_exp2(m[nt] - mnew);
            m[nt] = mnew;
            float ps = 0.f;
            float pv[4][4];
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    pv[kt][i] = fast_exp2(sv[kt][i] - mnew);
                    ps += pv[kt][i];
                }
            lsum[nt] = lsum[nt] * corr + ps;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[dt][nt] *= corr;
#pragma unroll
            for (int ss = 0; ss < 2; ++ss) {
                pop[ss][nt].x = Mfma<T>::pack2(pv[2 * ss][0], pv[2 * ss][1]);
                pop[ss][nt].y = Mfma<T>::pack2(pv[2 * ss][2], pv[2 * ss][3]);
                pop[ss][nt].z = Mfma<T>::pack2(pv[2 * ss + 1][0], pv[2 * ss + 1][1]);
                pop[ss][nt].w = Mfma<T>::pack2(pv[2 * ss + 1][2], pv[2 * ss + 1][3]);
            }
        }

        // ---- O^T += V^T P^T ------------------------------------------------
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
            for (int ss = 0; ss < 2; ++ss) {
                const uint4 va = *reinterpret_cast<const uint4*>(
                    &sm.vt[buf][(dt * 16 + c16) * VPAD + 32 * ss + 8 * g]);
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) o[dt][nt] = Mfma<T>::mma(va, pop[ss][nt], o[dt][nt]);
            }
        }

        if (t + 1 < ntiles) store_tile(buf ^ 1);
        __syncthreads();
    }

    // ---- normalise and write: lane holds dims dt*16 + 4g + i of its query --
    T* og = reinterpret_cast<T*>(a.out);
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        float lt = lsum[nt];
        lt += __shfl_xor(lt, 16, 64);
        lt += __shfl_xor(lt, 32, 64);
        const int ql = q_lo + w * WQ + nt * 16 + c16;
        if (ql >= P) continue;
        const float inv = lt > 0.f ? 1.0f / lt : 0.f;
        T* orow = og + ((int64_t)(q0 + ql) * a.Hq + hq) * D;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            uint2 w2;
            w2.x = Mfma<T>::pack2(o[dt][nt][0] * inv, o[dt][nt][1] * inv);
            w2.y = Mfma<T>::pack2(o[dt][nt][2] * inv, o[dt][nt][3] * inv);
            *reinterpret_cast<uint2*>(orow + dt * 16 + 4 * g) = w2;
        }
    }
}

}  // namespace

int launch_prefill_mfma(MfmaPrefillArgs a, int head_dim, int block_size, int dtype,
                        int total_q, int max_q_len, int max_seq_len, hipStream_t st) {
    (void)max_seq_len;
    if (block_size != kPage) return -1;
    if (dtype != LLKV_DTYPE_F16 && dtype != LLKV_DTYPE_BF16) return -1;
    if (head_dim != 64 && head_dim != 128) return -1;
    if (((uintptr_t)a.q | (uintptr_t)a.out | (uintptr_t)a.k | (uintptr_t)a.v) & 15) return -1;
    int qmax = (max_q_len > 0 && max_q_len < total_q) ? max_q_len : total_q;
    a.qblocks = (qmax + BQ - 1) / BQ;
    dim3 grid(a.N * a.qblocks, a.Hq);
    if (dtype == LLKV_DTYPE_F16) {
        if (head_dim == 64) prefill_mfma_kernel<_Float16, 64><<<grid, 256, 0, st>>>(a);
        else prefill_mfma_kernel<_Float16, 128><<<grid, 256, 0, st>>>(a);
    } else {
        if (head_dim == 64) prefill_mfma_kernel<bf16_t, 64><<<grid, 256, 0, st>>>(a);
        else prefill_mfma_kernel<bf16_t, 128><<<grid, 256, 0, st>>>(a);
    }
    return check_launch("llkv_paged_prefill");
}

}  // namespace llkv
