// MFMA paged decode body for fp32 / fp16 / bf16 K/V on gfx950 (16-token
// pages, head_dim 64 / 128, up to 16 query heads per KV head).  Included by
// decode.hip, which instantiates it under the fixed-split and the balanced
// schedules.
//
// Per KV head the decode step is two small matrix products:
//     S^T [tokens x G] = K [tokens x D] . Q^T [D x G]
//     O^T [D x G]      = V^T [D x tokens] . P^T [tokens x G]
// with the G query heads as the 16-wide N dimension.  The second product runs
// on v_mfma_f32_16x16x4_f32 (full fp32 products and sums; 16-bit V is widened
// exactly), the first on v_mfma_f32_16x16x4_f32 for fp32 pools and on
// v_mfma_f32_16x16x32_{f16,bf16} (exact products, fp32 sums) for 16-bit pools.
// Operand layouts are chosen so that nothing goes through LDS:
//   * K (fp32): lane (g = lane/16, c = lane%16) holds token c of the page and,
//     for k-step ks, dim 16*(ks/4) + 4*g + ks%4 -- four 16-byte loads per page;
//     (16-bit): token c, dims 32*ks + 8*g .. + 7, one 16-byte load per k-step;
//   * S^T lands in lane (g, c) as tokens 4g+i (i < 4) of query c, which is
//     exactly the B operand P^T of the second product for k-step i;
//   * V^T: lane (g, c) loads V[token 4g+i][dims 64h + 4c .. 64h + 4c+3] as one
//     16-byte (fp32) or 8-byte (16-bit) load, 16 lanes of a group reading one
//     contiguous row segment; element
//     j of that vector is the A operand of output tile dt = 4h + j, so tile dt
//     row r holds dim 64h + 4r + j (a permutation undone when the tiles are
//     written to LDS).
// Softmax state (max, sum) is per query column, kept in every lane of the
// column; the running max needs two cross-row shuffles per page.
// A work-group runs a round of up to kSegMax segments (page ranges of
// different (sequence, kv head) units) at once: the 4 waves take interleaved
// pages of the round's concatenated page list, so every wave issues its first
// loads at the start whatever the segment boundaries; a wave that crosses into
// the next segment parks its softmax state in LDS and loads the next query
// rows.  Afterwards the waves merge each segment's states through LDS, the
// query heads spread over the waves.
#pragma once

#include "attn_common.h"

namespace llkv {

typedef float mf32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int mu32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int mu32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 mf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 mf16x4 __attribute__((ext_vector_type(4)));
typedef short ms16x4 __attribute__((ext_vector_type(4)));

typedef __bf16 mbf16x8 __attribute__((ext_vector_type(8)));

// Score operands S^T = K Q^T per element type.  load_q fills the Q^T operand
// of query column c (zero beyond G), load_k the K operand of token row c of a
// page, scores returns the lane's 4 scores scaled into the exp2 domain.
template <typename T, int D> struct ScoreOps;

template <int D> struct ScoreOps<float, D> {
    static constexpr int NQ = D / 4;    // one fp32 per k-step
    static constexpr int NK = D / 16;   // float4 per page row
    typedef float QReg;
    typedef float4 KReg;
    __device__ static void load_q(const float* qrow, bool valid, int g, float scale, QReg (&q)[NQ]) {
#pragma unroll
        for (int cc = 0; cc < NK; ++cc) {
            float4 v = valid ? *reinterpret_cast<const float4*>(qrow + 16 * cc + 4 * g)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
            q[4 * cc + 0] = v.x * scale;
            q[4 * cc + 1] = v.y * scale;
            q[4 * cc + 2] = v.z * scale;
            q[4 * cc + 3] = v.w * scale;
        }
    }
    // krow: K row of the lane's token, at this kv head's dims
    __device__ static void load_k(const float* krow, int g, KReg (&k)[NK]) {
#pragma unroll
        for (int cc = 0; cc < NK; ++cc) k[cc] = *reinterpret_cast<const float4*>(krow + 16 * cc + 4 * g);
    }
    // From head_dim 128 on, the four quarters of the head dims accumulate
    // apart and are added pairwise at the end: a quarter of the rounding steps
    // in each sum (the score's rounding dominates the fp32 output's error
    // there; one running sum reached the bound on seeded shapes, two sums
    // 1.007 of it on one of ~600).  At head_dim 64 more accumulators would
    // spill registers in the fused-append variant.
    __device__ static mf32x4 scores(const KReg (&k)[NK], const QReg (&q)[NQ], float) {
        constexpr int kParts = D >= 128 ? 4 : 1;   // running sums over consecutive dim blocks
        constexpr int kPer = NK / kParts;
        mf32x4 acc[kParts];
#pragma unroll
        for (int j = 0; j < kParts; ++j) acc[j] = mf32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int cc = 0; cc < NK; ++cc) {
            mf32x4& a = acc[cc / kPer];
            a = __builtin_amdgcn_mfma_f32_16x16x4f32(k[cc].x, q[4 * cc + 0], a, 0, 0, 0);
            a = __builtin_amdgcn_mfma_f32_16x16x4f32(k[cc].y, q[4 * cc + 1], a, 0, 0, 0);
            a = __builtin_amdgcn_mfma_f32_16x16x4f32(k[cc].z, q[4 * cc + 2], a, 0, 0, 0);
            a = __builtin_amdgcn_mfma_f32_16x16x4f32(k[cc].w, q[4 * cc + 3], a, 0, 0, 0);
        }
        if constexpr (kParts == 1) return acc[0];   // Q was pre-scaled
        else return (acc[0] + acc[1]) + (acc[2] + acc[3]);
    }
    // V[row][dims 4c .. 4c+3] widened to fp32
    __device__ static float4 load_v4(const float* p) { return *reinterpret_cast<const float4*>(p); }
};

template <typename T16, int D> struct ScoreOps16 {
    static constexpr int NQ = D / 32;   // 8 halves per k-step of 32 dims
    static constexpr int NK = D / 32;
    typedef mu32x4 QReg;
    typedef mu32x4 KReg;
    __device__ static void load_q(const T16* qrow, bool valid, int g, float, QReg (&q)[NQ]) {
#pragma unroll
        for (int ks = 0; ks < NQ; ++ks)
            q[ks] = valid ? *reinterpret_cast<const mu32x4*>(qrow + 32 * ks + 8 * g) : mu32x4{0u, 0u, 0u, 0u};
    }
    __device__ static void load_k(const T16* krow, int g, KReg (&k)[NK]) {
#pragma unroll
        for (int ks = 0; ks < NK; ++ks) k[ks] = *reinterpret_cast<const mu32x4*>(krow + 32 * ks + 8 * g);
    }
    __device__ static mf32x4 mma(const mu32x4& a, const mu32x4& b, mf32x4 c) {
        if constexpr (Elem<T16>::kDtype == LLKV_DTYPE_F16)
            return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(mf16x8, a), __builtin_bit_cast(mf16x8, b), c, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(mbf16x8, a), __builtin_bit_cast(mbf16x8, b), c, 0, 0, 0);
    }
    __device__ static mf32x4 scores(const KReg (&k)[NK], const QReg (&q)[NQ], float scale) {
        mf32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < NK; ++ks) s = mma(k[ks], q[ks], s);
        return s * scale;
    }
    __device__ static float4 load_v4(const T16* p) {
        const mu32x2 w = *reinterpret_cast<const mu32x2*>(p);
        float f[4];
        if constexpr (sizeof(T16) == 2 && Elem<T16>::kDtype == LLKV_DTYPE_F16) {
            unpack_h2(w.x, f);
            unpack_h2(w.y, f + 2);
        } else {
            unpack_b2(w.x, f);
            unpack_b2(w.y, f + 2);
        }
        return make_float4(f[0], f[1], f[2], f[3]);
    }
};

template <int D> struct ScoreOps<_Float16, D> : ScoreOps16<_Float16, D> {};
template <int D> struct ScoreOps<bf16_t, D> : ScoreOps16<bf16_t, D> {};

// A = true: the fused-append variant (llkv_paged_decode_append), which reads
// the segment's new token from the caller's buffers; the plain variant's page
// loop has no trace of it.
// WV: waves per work-group (kDecodeWaves; kUnitWaves for the one-work-group-
// per-unit schedule of small batches).
template <typename TT, int D, int G, bool A = false, int WV = kDecodeWaves>
struct MfmaDecode {
    static_assert(G >= 1 && G <= 16, "up to 16 query heads per KV head");
    static_assert(D % 32 == 0, "head_dim multiple of 32");
    using T = TT;
    using Ops = ScoreOps<T, D>;
    static constexpr int W = WV;              // waves per work-group
    static constexpr int kThreads = 64 * W;
    // V is loaded in 64-dim groups (h), lane c holding dims 64h + 4c .. + 3;
    // with head_dim 96 the last group is half empty (lanes c >= 8 load none).
    static constexpr int VH = (D + 63) / 64;  // V vectors per lane per token
    static constexpr int DT = 4 * VH;         // O^T tiles (tile 4h + j: dims 64h + 4r + j)
    static constexpr int MD = (D + 63) / 64;
    static constexpr int GQ = G, HD = D;
    // 16-bit pools at head_dim 256: O^T = V^T P^T on the 16x16x16 f16 / bf16
    // MFMA (P rounded to the pool type, as in the prefill): 127.8 -> 113.1 us
    // on a B = 64 Gemma-2 shape in fp16.  At head_dim 64 / 128 the page loop is
    // not bound by its MFMAs and this form measured 1-2 % slower, so those, and
    // fp32 pools, keep v_mfma_f32_16x16x4f32 with V widened and P in fp32.
    static constexpr bool kHalfPV = Elem<T>::kDtype != LLKV_DTYPE_F32 && D == 256;
    // Resident waves per SIMD the register budget is held to: 5 (<= 96
    // registers) for head_dim 64; head_dim 128 needs more and gets 4.
    // head_dim 256: ~200 VGPRs (two waves per SIMD, no spills; three spill 33-49).
    // The unit schedule's 16-wave work-group puts four waves on each SIMD.
    // The fused-append variant of fp32 pools holds one wave per SIMD fewer:
    // its new-row pointers took it past the register budget (2-9 registers
    // spilled at head_dim 64, ~50 at 128); configuration 2 fused 25.9 ->
    // 24.5 us at four waves.
    static constexpr bool kA32 = A && Elem<T>::kDtype == LLKV_DTYPE_F32;
    static constexpr int kWavesPerEU =
        W > kDecodeWaves ? 4
                         : (D == 64 ? (kA32 ? 4 : 5) : (D == 96 ? 3 : (D == 128 ? (kA32 ? 3 : 4) : 2)));
    // Segments per round: two where the LDS for the parked states stays small.
    // (The unit schedule runs one segment per work-group.)
    static constexpr int kSegMax = (W == kDecodeWaves && G * D <= 512) ? 2 : 1;

    struct Smem {
        float acc[kSegMax][W][G][D];
        float ml[kSegMax][W][G][2];   // (max, sum); sum 0: the wave had no page
    };

    __device__ static void round(const DecodeArgs& a, Smem& sm, const SegDesc* segs, int nseg,
                                 int64_t po_stride, int64_t pl_stride) {
        const int tid = threadIdx.x, lane = tid & 63;
        const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index, known uniform
        const int g = lane >> 4, c = lane & 15;
        const int np_total = segs[nseg - 1].cum + segs[nseg - 1].npages;
        const int64_t row_elems = (int64_t)a.Hkv * D;

        // Empty states for this wave's slots (a wave may own no page of a segment).
        for (int s = 0; s < nseg; ++s) {
            for (int i = lane; i < G * D; i += 64) (&sm.acc[s][w][0][0])[i] = 0.0f;
            if (lane < G) {
                sm.ml[s][w][lane][0] = kNegBig;
                sm.ml[s][w][lane][1] = 0.0f;
            }
        }

        // Physical page of this wave's k-th page (k = lane + tbl_k0), j = w + 4k.
        int tbl = 0, tbl_k0 = 0;
        auto load_tbl = [&](int k0) {
            const int j = w + W * (k0 + lane);
            int v = 0;
            if (j < np_total) {
                int s = 0;
                while (s + 1 < nseg && j >= segs[s + 1].cum) ++s;
                const SegDesc& d = segs[s];
                v = a.bt[(int64_t)d.b * a.max_blocks + d.pg_begin + (j - d.cum)];
            }
            tbl = v;
        };
        load_tbl(0);

        // State of the current segment.
        int cur = -1, sb = 0, skvh = 0, spg = 0, scum = 0, stok = 0;
        // Fused append: page and row of the segment's new token (-1: none).
        int snew_pg = -1, snew_r = 0;
        int next_cum = 0;   // first page of the next segment (register copy)
        typename Ops::QReg qop[Ops::NQ];
        mf32x4 o[DT];
        float m = kNegBig, lsum = 0.0f;

        auto flush = [&](int s) {
            float ls = lsum;
            ls += __shfl_xor(ls, 16, 64);
            ls += __shfl_xor(ls, 32, 64);
            if (c < G) {
                // tile 4h + j, row 4g + i  ->  dim 64h + 16g + 4i + j
#pragma unroll
                for (int h = 0; h < VH; ++h)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (D % 64 == 0 || 64 * h + 16 * g + 4 * i < D)
                            *reinterpret_cast<float4*>(&sm.acc[s][w][c][64 * h + 16 * g + 4 * i]) =
                                make_float4(o[4 * h][i], o[4 * h + 1][i], o[4 * h + 2][i], o[4 * h + 3][i]);
                if (g == 0) {
                    sm.ml[s][w][c][0] = m;
                    sm.ml[s][w][c][1] = ls;
                }
            }
        };

        typename Ops::KReg kr[Ops::NK];
        float4 vr[VH][4];    // fp32 V (fp32 / bf16 pools)
        mu32x2 vh[VH][4];    // raw fp16 V (fp16 pools)
        for (int k = 0;; ++k) {
            const int j = w + W * k;
            if (j >= np_total) break;
            if (k - tbl_k0 >= 64) {
                tbl_k0 = k;
                load_tbl(k);
            }
            if (j >= next_cum) {   // uniform: park the previous state, start the next segment
                int s = cur < 0 ? 0 : cur;
                while (s + 1 < nseg && j >= segs[s + 1].cum) ++s;
                if (cur >= 0) flush(cur);
                cur = s;
                next_cum = s + 1 < nseg ? segs[s + 1].cum : INT_MAX;
                sb = segs[s].b;
                skvh = segs[s].kvh;
                spg = segs[s].pg_begin;
                scum = segs[s].cum;
                stok = segs[s].tok_end;
                if constexpr (A) {
                    const int nt = __builtin_amdgcn_readfirstlane(segs[s].new_tok);
                    snew_pg = nt >= 0 ? nt / kPage : -1;
                    snew_r = nt % kPage;
                }
                // Q^T operand: column c is query head kvh*G + c (zero beyond G).
                const T* qrow = reinterpret_cast<const T*>(a.q) + ((int64_t)sb * a.Hq + skvh * G + c) * D;
                Ops::load_q(qrow, c < G, g, a.scale_log2, qop);
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) o[dt] = mf32x4{0.f, 0.f, 0.f, 0.f};
                m = kNegBig;
                lsum = 0.0f;
            }
            const int pg = spg + (j - scum);
            const int64_t phys = max(__builtin_amdgcn_readlane(tbl, k - tbl_k0), 0);

            // K row of the lane's token c; V rows 4g + i, dims 64h + 4c .. + 3.
            // The new token of a fused append is read from the caller's buffers
            // (its pool row is being written by this work-group).
            const bool newpage = A && pg == snew_pg;   // uniform
            const int64_t nrow = ((int64_t)sb * a.Hkv + skvh) * D;   // the new rows' offset
            const T* kp = reinterpret_cast<const T*>(a.k) + (int64_t)skvh * D + (phys * kPage + c) * row_elems;
            if (newpage && c == snew_r) kp = reinterpret_cast<const T*>(a.knew) + nrow;
            Ops::load_k(kp, g, kr);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const T* vp = reinterpret_cast<const T*>(a.v) + (int64_t)skvh * D +
                              (phys * kPage + 4 * g + i) * row_elems + 4 * c;
                if (newpage && 4 * g + i == snew_r) vp = reinterpret_cast<const T*>(a.vnew) + nrow + 4 * c;
#pragma unroll
                for (int h = 0; h < VH; ++h) {
                    if (D % 64 != 0 && 64 * h + 4 * c >= D) {   // past the head's last dim
                        vh[h][i] = mu32x2{0u, 0u};
                        vr[h][i] = make_float4(0.f, 0.f, 0.f, 0.f);
                    } else if constexpr (kHalfPV) {
                        vh[h][i] = *reinterpret_cast<const mu32x2*>(vp + 64 * h);
                    } else {
                        vr[h][i] = Ops::load_v4(vp + 64 * h);
                    }
                }
            }
            // The fused variant's pointer selects make the scheduler sink the V
            // loads next to their MFMAs; keep all of the page's loads first.
            if constexpr (A) __builtin_amdgcn_sched_barrier(0);

            const mf32x4 sacc = Ops::scores(kr, qop, a.scale_log2);
            const int t0 = pg * kPage + 4 * g;
            float x[4];
            float mt = kNegBig;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[i] = (t0 + i < stok) ? sacc[i] : -INFINITY;
                mt = fmaxf(mt, x[i]);
            }
            mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
            mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
            const float mnew = fmaxf(m, mt);
            const float corr = fast_exp2(m - mnew);
            m = mnew;
            float p[4];
            float ps = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                p[i] = fast_exp2(x[i] - mnew);
                ps += p[i];
            }
            lsum = fmaf(lsum, corr, ps);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[dt] *= corr;
            if constexpr (kHalfPV) {
                // One v_mfma_f32_16x16x16_f16 per output tile: the lane's 4x4
                // block (tokens 4g + i, dims 4c + j) gives tile (h, j) its A
                // operand (tokens 4g .. 4g + 3 of dim 64h + 4c + j) with two
                // v_perm_b32, and its own scores p[0..3] are the B operand.
                constexpr bool kF16 = Elem<T>::kDtype == LLKV_DTYPE_F16;
                const mu32x2 pb = kF16 ? mu32x2{pack_h2(p[0], p[1]), pack_h2(p[2], p[3])}
                                       : mu32x2{pack_b2(p[0], p[1]), pack_b2(p[2], p[3])};
#pragma unroll
                for (int h = 0; h < VH; ++h)
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        const unsigned sel = (jj & 1) ? 0x07060302u : 0x05040100u;
                        const int wd = jj >> 1;
                        const mu32x2 av = {__builtin_amdgcn_perm(vh[h][1][wd], vh[h][0][wd], sel),
                                           __builtin_amdgcn_perm(vh[h][3][wd], vh[h][2][wd], sel)};
                        if constexpr (kF16)
                            o[4 * h + jj] = __builtin_amdgcn_mfma_f32_16x16x16f16(
                                __builtin_bit_cast(mf16x4, av), __builtin_bit_cast(mf16x4, pb), o[4 * h + jj], 0, 0, 0);
                        else
                            o[4 * h + jj] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                                __builtin_bit_cast(ms16x4, av), __builtin_bit_cast(ms16x4, pb), o[4 * h + jj], 0, 0, 0);
                    }
            } else
#pragma unroll
            for (int h = 0; h < VH; ++h)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    o[4 * h + 0] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[h][i].x, p[i], o[4 * h + 0], 0, 0, 0);
                    o[4 * h + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[h][i].y, p[i], o[4 * h + 1], 0, 0, 0);
                    o[4 * h + 2] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[h][i].z, p[i], o[4 * h + 2], 0, 0, 0);
                    o[4 * h + 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[h][i].w, p[i], o[4 * h + 3], 0, 0, 0);
                }
        }
        if (cur >= 0) flush(cur);
        LLKV_TRACE_POINT(1);
        __syncthreads();

        // Merge the 4 waves' states of each segment; heads spread over the waves.
        for (int s = 0; s < nseg; ++s) {
            const SegDesc& d = segs[s];
            for (int h = w; h < G; h += W) {
                float M = sm.ml[s][0][h][0];
#pragma unroll
                for (int ww = 1; ww < W; ++ww) M = fmaxf(M, sm.ml[s][ww][h][0]);
                float f[W], L = 0.0f;
#pragma unroll
                for (int ww = 0; ww < W; ++ww) {
                    f[ww] = fast_exp2(sm.ml[s][ww][h][0] - M);
                    L = fmaf(f[ww], sm.ml[s][ww][h][1], L);
                }
                const float inv = 1.0f / L;
#pragma unroll
                for (int i = 0; i < MD; ++i) {
                    const int dd = lane + 64 * i;
                    if (D % 64 != 0 && dd >= D) break;
                    float ov = 0.0f;
#pragma unroll
                    for (int ww = 0; ww < W; ++ww) ov = fmaf(f[ww], sm.acc[s][ww][h][dd], ov);
                    ov *= inv;
                    if (d.direct)
                        reinterpret_cast<T*>(a.out)[((int64_t)d.b * a.Hq + d.kvh * G + h) * D + dd] =
                            Elem<T>::from_f32(ov);
                    else
                        a.part_o[d.po_off + h * po_stride + dd] = ov;
                }
                if (!d.direct && lane == 0) a.part_lse[d.pl_off + h * pl_stride] = M + fast_log2(L);
            }
        }
        lds_barrier();   // the partial / output stores need not complete here
        LLKV_TRACE_POINT(2);
    }
};

}  // namespace llkv
