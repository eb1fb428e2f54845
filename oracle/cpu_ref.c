/*
 * CPU oracle for the paged KV-cache hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * Restates, in plain C, the CPU reference code held by wjb554/lightllm's own
 * tests and the arithmetic of its kernels.  Each function cites the
 * reference file:line it follows.  It is the checker for the HIP kernels and
 * the CPU baseline of bench.py; it is never part of the product path.
 */
#include "cpu_ref.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int llo_omp_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* Generators                                                                */
/* ------------------------------------------------------------------------ */

/* tests/test_paged_attention_v2.cu:58-64 (same LCG in tests/test_paged_prefill.cu:59-65):
 * s = s*1664525 + 1013904223; v = (s & 0x7FFF)/16384 - 1 */
void llo_fill_random(float* v, size_t n, unsigned seed) {
    unsigned s = seed;
    for (size_t i = 0; i < n; i++) {
        s = s * 1664525u + 1013904223u;
        v[i] = ((float)(s & 0x7FFFu) / 16384.0f) - 1.0f;
    }
}

/* tests/test_attention_fp16.cpp:31-38 and :97-102 (rand_vec):
 * state = state*1103515245 + 12345; u = (state & 0x7FFFFFFF)/2^31; v = 2u-1 */
void llo_rng_randf_fill(float* v, size_t n, uint32_t* state) {
    uint32_t s = *state;
    for (size_t i = 0; i < n; i++) {
        s = s * 1103515245u + 12345u;
        float u = (float)(s & 0x7FFFFFFFu) / 2147483648.0f;
        v[i] = u * 2.0f - 1.0f;
    }
    *state = s;
}

/* ------------------------------------------------------------------------ */
/* fp16 / bf16 conversions (IEEE round-to-nearest-even), as __float2half /    */
/* __half2float used by tests/test_attention_fp16.cpp:105-119.               */
/* ------------------------------------------------------------------------ */
static uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

uint16_t llo_f32_to_f16(float x) {
    uint32_t u = f2u(x);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t absu = u & 0x7FFFFFFFu;
    if (absu >= 0x7F800000u) {                 /* inf or nan */
        if (absu > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((absu >> 13) & 0x3FFu));
        return (uint16_t)(sign | 0x7C00u);
    }
    if (absu >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520 -> inf */
    if (absu < 0x38800000u) {                  /* below 2^-14: subnormal half */
        /* value = absu as float; subnormal half unit = 2^-24 */
        float a = u2f(absu);
        /* scale to units of 2^-24 and round to nearest even */
        float scaled = a * 16777216.0f;        /* exact: power-of-two scaling */
        float r = nearbyintf(scaled);          /* default rounding mode: nearest-even */
        return (uint16_t)(sign | (uint32_t)r);
    }
    uint32_t exp = ((absu >> 23) - 127 + 15);
    uint32_t mant = absu & 0x7FFFFFu;
    uint32_t h = (exp << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1;  /* carry may bump exponent: correct */
    return (uint16_t)(sign | h);
}

float llo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    if (exp == 0) {
        float v = (float)mant * (1.0f / 16777216.0f);   /* mant * 2^-24, exact */
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7F800000u | (mant << 13));
    return u2f(sign | ((exp - 15 + 127) << 23) | (mant << 13));
}

uint16_t llo_f32_to_bf16(float x) {
    uint32_t u = f2u(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);  /* quiet nan */
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7FFFu + lsb;
    return (uint16_t)(u >> 16);
}

float llo_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

void llo_f32_to_f16_array(const float* s, uint16_t* d, size_t n) { for (size_t i = 0; i < n; i++) d[i] = llo_f32_to_f16(s[i]); }
void llo_f16_to_f32_array(const uint16_t* s, float* d, size_t n) { for (size_t i = 0; i < n; i++) d[i] = llo_f16_to_f32(s[i]); }
void llo_f32_to_bf16_array(const float* s, uint16_t* d, size_t n) { for (size_t i = 0; i < n; i++) d[i] = llo_f32_to_bf16(s[i]); }
void llo_bf16_to_f32_array(const uint16_t* s, float* d, size_t n) { for (size_t i = 0; i < n; i++) d[i] = llo_bf16_to_f32(s[i]); }

/* ------------------------------------------------------------------------ */
/* KV append / scatter / gather                                              */
/* ------------------------------------------------------------------------ */

/* Slot-mapping append.  Slot arithmetic of tests/test_attention_divergence.cpp:147-168
 * (write_kv_to_cache) and src/kv_cache/paged_attention.cu:996-1008:
 * destination row = slot = phys*bs + pos%bs; the row holds Hkv*D elements.
 * A negative slot is skipped (padding entries). */
void llo_append_slots(void* k_pool, void* v_pool, const void* k_src,
                      const void* v_src, const int64_t* slot_mapping,
                      int64_t n_tokens, int Hkv, int D, int elem_size) {
    size_t row = (size_t)Hkv * D * elem_size;
    for (int64_t i = 0; i < n_tokens; i++) {
        int64_t slot = slot_mapping[i];
        if (slot < 0) continue;
        memcpy((char*)k_pool + (size_t)slot * row, (const char*)k_src + (size_t)i * row, row);
        memcpy((char*)v_pool + (size_t)slot * row, (const char*)v_src + (size_t)i * row, row);
    }
}

/* Slot mapping of a step.  Restates the host loops of
 * EngineServer::scatter_prefill_kv (src/engine/engine_server.cpp:731-757) and
 * write_decode_kv (:760-787): pos = start + i, phys = table[pos / bs],
 * row = phys*bs + pos%bs; a position outside the table is skipped
 * (:766-774), here slot -1.  Token t belongs to the sequence n with
 * cu[n] <= t < cu[n+1]. */
void llo_build_slots(int64_t* slots, const int* block_table, int max_blocks,
                     const int* cu, const int* start_pos, int n, int num_tokens,
                     int block_size) {
    for (int e = 0; e < n; e++) {
        for (int t = cu[e]; t < cu[e + 1] && t < num_tokens; t++) {
            int pos = start_pos[e] + (t - cu[e]);
            int64_t slot = -1;
            if (pos >= 0 && pos / block_size < max_blocks) {
                int phys = block_table[(size_t)e * max_blocks + pos / block_size];
                if (phys >= 0) slot = (int64_t)phys * block_size + pos % block_size;
            }
            slots[t] = slot;
        }
    }
}

static float load_elem(const void* p, size_t i, int dtype) {
    if (dtype == 0) return ((const float*)p)[i];
    if (dtype == 1) return llo_f16_to_f32(((const uint16_t*)p)[i]);
    return llo_bf16_to_f32(((const uint16_t*)p)[i]);
}

static void store_elem(void* p, size_t i, int dtype, float x) {
    if (dtype == 0) ((float*)p)[i] = x;
    else if (dtype == 1) ((uint16_t*)p)[i] = llo_f32_to_f16(x);
    else ((uint16_t*)p)[i] = llo_f32_to_bf16(x);
}

/* One Neox pair: the arithmetic of src/ops/rope.cu:54-57 with every product
 * and sum rounded to fp32 on its own (no contraction into fused
 * multiply-adds, which -march=x86-64-v3 would otherwise allow). */
__attribute__((optimize("fp-contract=off"), noinline))
static void rope_pair(float x1, float x2, float c, float s, float* o1, float* o2) {
    float a = x1 * c, b = x2 * s, d = x2 * c, e = x1 * s;
    *o1 = a - b;
    *o2 = d + e;
}

static void rope_rows(void* x, int T, int H, int D, int half, const float* cos,
                      const float* sin, int dtype) {
    for (int t = 0; t < T; t++)
        for (int h = 0; h < H; h++) {
            size_t row = ((size_t)t * H + h) * D;
            for (int i = 0; i < half; i++) {
                float o1, o2;
                rope_pair(load_elem(x, row + i, dtype), load_elem(x, row + half + i, dtype),
                          cos[(size_t)t * half + i], sin[(size_t)t * half + i], &o1, &o2);
                store_elem(x, row + i, dtype, o1);
                store_elem(x, row + half + i, dtype, o2);
            }
        }
}

/* RoPE on q and k (the documented contract of include/lightllm/ops/rope.h:8-13:
 * Neox halves of the first rotary_dim dims, cos/sin [T, rotary_dim/2]), then the
 * rotated k rows and the v rows appended at slot_mapping (llo_append_slots).
 * q may be NULL.  dtype: 0 fp32, 1 fp16, 2 bf16. */
void llo_rope_append(void* q, void* k, const void* v, void* k_pool, void* v_pool,
                     const int64_t* slot_mapping, const float* cos, const float* sin,
                     int T, int Hq, int Hkv, int D, int rotary_dim, int dtype) {
    int half = rotary_dim / 2;
    if (q) rope_rows(q, T, Hq, D, half, cos, sin, dtype);
    rope_rows(k, T, Hkv, D, half, cos, sin, dtype);
    llo_append_slots(k_pool, v_pool, k, v, slot_mapping, T, Hkv, D, dtype == 0 ? 4 : 2);
}

/* src/kv_cache/paged_attention.cu:986-1010 (scatter_prefill_kv_kernel):
 * token t of the chunk goes to pos = start_pos + t, phys = bt[pos/bs], offset pos%bs. */
void llo_scatter_prefill(void* k_pool, void* v_pool, const void* k_src,
                         const void* v_src, int start_pos, int n_tokens,
                         const int* block_table, int block_size, int Hkv,
                         int D, int elem_size) {
    size_t row = (size_t)Hkv * D * elem_size;
    for (int t = 0; t < n_tokens; t++) {
        int pos = start_pos + t;
        int64_t phys = block_table[pos / block_size];
        int64_t slot = phys * block_size + pos % block_size;
        memcpy((char*)k_pool + (size_t)slot * row, (const char*)k_src + (size_t)t * row, row);
        memcpy((char*)v_pool + (size_t)slot * row, (const char*)v_src + (size_t)t * row, row);
    }
}

/* src/kv_cache/paged_attention.cu:1134-1164 (scatter_prefill_kv_batched_kernel):
 * global token g -> entry e with token_cumsum[e] <= g < token_cumsum[e+1];
 * source element offset kv_offsets[e] + local*Hkv*D; destination from flat_bt[e*max_blocks + pos/bs]. */
void llo_scatter_prefill_batched(void* k_pool, void* v_pool,
                                 const void* k_flat, const void* v_flat,
                                 int Hkv, int D, const int* kv_offsets,
                                 const int* start_poss,
                                 const int* token_cumsum, const int* flat_bt,
                                 int max_blocks, int N, int block_size,
                                 int elem_size) {
    size_t row_elems = (size_t)Hkv * D;
    size_t row = row_elems * elem_size;
    for (int e = 0; e < N; e++) {
        for (int g = token_cumsum[e]; g < token_cumsum[e + 1]; g++) {
            int local = g - token_cumsum[e];
            int pos = start_poss[e] + local;
            int64_t phys = flat_bt[(size_t)e * max_blocks + pos / block_size];
            int64_t slot = phys * block_size + pos % block_size;
            size_t src_elem = (size_t)kv_offsets[e] + (size_t)local * row_elems;
            memcpy((char*)k_pool + (size_t)slot * row, (const char*)k_flat + src_elem * elem_size, row);
            memcpy((char*)v_pool + (size_t)slot * row, (const char*)v_flat + src_elem * elem_size, row);
        }
    }
}

/* tests/test_paged_attention_v2.cu:219-239 / tests/test_paged_prefill.cu:216-239 (reconstruct_kv):
 * contiguous [seq_len, Hkv, D] from the paged pool. */
void llo_reconstruct_kv(void* k_out, void* v_out, const void* k_pool,
                        const void* v_pool, const int* block_table,
                        int seq_len, int block_size, int Hkv, int D,
                        int elem_size) {
    size_t row = (size_t)Hkv * D * elem_size;
    for (int pos = 0; pos < seq_len; pos++) {
        int64_t phys = block_table[pos / block_size];
        int64_t slot = phys * block_size + pos % block_size;
        memcpy((char*)k_out + (size_t)pos * row, (const char*)k_pool + (size_t)slot * row, row);
        memcpy((char*)v_out + (size_t)pos * row, (const char*)v_pool + (size_t)slot * row, row);
    }
}

/* ------------------------------------------------------------------------ */
/* Decode attention                                                          */
/* ------------------------------------------------------------------------ */

/* One (query row, head) of tests/test_paged_attention_v2.cu:111-155 (cpu_attention):
 * two-pass softmax in fp32, max init -1e38, scores = dot*scale, exp(s - max), divide
 * by the sum, then the weighted V sum.  Keys are rows of `stride` floats. */
static void attn_row_f32(const float* qr, int D, const float* k, const float* v,
                         size_t stride, int L, float scale, float* scores, float* o) {
    float mx = -1e38f;
    for (int pos = 0; pos < L; pos++) {
        const float* kr = k + (size_t)pos * stride;
        float dot = 0.0f;
        for (int d = 0; d < D; d++) dot += qr[d] * kr[d];
        scores[pos] = dot * scale;
        mx = fmaxf(mx, scores[pos]);
    }
    float sum = 0.0f;
    for (int pos = 0; pos < L; pos++) {
        scores[pos] = expf(scores[pos] - mx);
        sum += scores[pos];
    }
    for (int pos = 0; pos < L; pos++) scores[pos] /= sum;
    for (int d = 0; d < D; d++) {
        float acc = 0.0f;
        for (int pos = 0; pos < L; pos++) acc += scores[pos] * v[(size_t)pos * stride + d];
        o[d] = acc;
    }
}

/* The same algorithm carried in double (tie-breaker oracle). */
static void attn_row_f64(const float* qr, int D, const float* k, const float* v,
                         size_t stride, int L, double* scores, double* o) {
    double scale = 1.0 / sqrt((double)D);
    double mx = -1e300, sum = 0.0;
    for (int pos = 0; pos < L; pos++) {
        const float* kr = k + (size_t)pos * stride;
        double dot = 0.0;
        for (int d = 0; d < D; d++) dot += (double)qr[d] * (double)kr[d];
        scores[pos] = dot * scale;
        if (scores[pos] > mx) mx = scores[pos];
    }
    for (int pos = 0; pos < L; pos++) { scores[pos] = exp(scores[pos] - mx); sum += scores[pos]; }
    for (int d = 0; d < D; d++) {
        double acc = 0.0;
        for (int pos = 0; pos < L; pos++) acc += scores[pos] * (double)v[(size_t)pos * stride + d];
        o[d] = L > 0 ? acc / sum : 0.0;
    }
}

/* tests/test_paged_attention_v2.cu:111-155 (cpu_attention): all T query rows attend the
 * same seq_len keys of contiguous [seq_len, Hkv, D]; kv_head = h / (Hq/Hkv);
 * seq_len == 0 gives zeros. */
void llo_cpu_attention(const float* q, int T, int Hq, int D, const float* k,
                       int seq_len, int Hkv, const float* v, float* out) {
    int groups = Hq / Hkv;
    float scale = 1.0f / sqrtf((float)D);
    float* scores = (float*)malloc(sizeof(float) * (seq_len > 0 ? seq_len : 1));
    for (int t = 0; t < T; t++)
        for (int h = 0; h < Hq; h++)
            attn_row_f32(q + ((size_t)t * Hq + h) * D, D, k + (size_t)(h / groups) * D,
                         v + (size_t)(h / groups) * D, (size_t)Hkv * D, seq_len, scale,
                         scores, out + ((size_t)t * Hq + h) * D);
    free(scores);
}

void llo_cpu_attention_f64(const float* q, int T, int Hq, int D,
                           const float* k, int seq_len, int Hkv,
                           const float* v, double* out) {
    int groups = Hq / Hkv;
    double* scores = (double*)malloc(sizeof(double) * (seq_len > 0 ? seq_len : 1));
    for (int t = 0; t < T; t++)
        for (int h = 0; h < Hq; h++)
            attn_row_f64(q + ((size_t)t * Hq + h) * D, D, k + (size_t)(h / groups) * D,
                         v + (size_t)(h / groups) * D, (size_t)Hkv * D, seq_len, scores,
                         out + ((size_t)t * Hq + h) * D);
    free(scores);
}

/* Batched decode the way the reference's tests check paged_attention:
 * reconstruct_kv per sequence (tests/test_paged_attention_v2.cu:219-239), then
 * cpu_attention with T=1 (:111-155).  nthreads > 1 runs OpenMP over (seq, q_head). */
static void decode_impl(const float* q, const float* k_pool, const float* v_pool,
                        const int* block_table, const int* seq_lens, int B, int Hq,
                        int Hkv, int D, int block_size, int max_blocks,
                        float* out32, double* out64, int nthreads) {
    size_t row = (size_t)Hkv * D;
    size_t* off = (size_t*)malloc(sizeof(size_t) * (B + 1));
    int maxL = 1;
    off[0] = 0;
    for (int b = 0; b < B; b++) {
        int L = seq_lens[b] > 0 ? seq_lens[b] : 0;
        off[b + 1] = off[b] + (size_t)L;
        if (L > maxL) maxL = L;
    }
    float* kc = (float*)malloc(sizeof(float) * (off[B] * row + 1));
    float* vc = (float*)malloc(sizeof(float) * (off[B] * row + 1));
    if (nthreads < 1) nthreads = 1;
    int groups = Hq / Hkv;
    float scale = 1.0f / sqrtf((float)D);
#pragma omp parallel num_threads(nthreads)
    {
        float* s32 = (float*)malloc(sizeof(float) * maxL);
        double* s64 = (double*)malloc(sizeof(double) * maxL);
#pragma omp for schedule(dynamic)
        for (int b = 0; b < B; b++)
            llo_reconstruct_kv(kc + off[b] * row, vc + off[b] * row, k_pool, v_pool,
                               block_table + (size_t)b * max_blocks, seq_lens[b],
                               block_size, Hkv, D, (int)sizeof(float));
#pragma omp for schedule(dynamic) collapse(2)
        for (int b = 0; b < B; b++) {
            for (int h = 0; h < Hq; h++) {
                int L = seq_lens[b] > 0 ? seq_lens[b] : 0;
                const float* kb = kc + off[b] * row + (size_t)(h / groups) * D;
                const float* vb = vc + off[b] * row + (size_t)(h / groups) * D;
                const float* qr = q + ((size_t)b * Hq + h) * D;
                if (out32) attn_row_f32(qr, D, kb, vb, row, L, scale, s32, out32 + ((size_t)b * Hq + h) * D);
                if (out64) attn_row_f64(qr, D, kb, vb, row, L, s64, out64 + ((size_t)b * Hq + h) * D);
            }
        }
        free(s32);
        free(s64);
    }
    free(kc);
    free(vc);
    free(off);
}

void llo_paged_decode(const float* q, const float* k_pool, const float* v_pool,
                      const int* block_table, const int* seq_lens, int B, int Hq,
                      int Hkv, int D, int block_size, int max_blocks, float* out,
                      int nthreads) {
    decode_impl(q, k_pool, v_pool, block_table, seq_lens, B, Hq, Hkv, D,
                block_size, max_blocks, out, NULL, nthreads);
}

void llo_paged_decode_f64(const float* q, const float* k_pool,
                          const float* v_pool, const int* block_table,
                          const int* seq_lens, int B, int Hq, int Hkv, int D,
                          int block_size, int max_blocks, double* out,
                          int nthreads) {
    decode_impl(q, k_pool, v_pool, block_table, seq_lens, B, Hq, Hkv, D,
                block_size, max_blocks, NULL, out, nthreads);
}

/* ------------------------------------------------------------------------ */
/* Split-K                                                                   */
/* ------------------------------------------------------------------------ */

/* src/kv_cache/paged_attention.cu:324-460 (paged_attention_kernel_splitk), restated:
 * split s covers blocks [s*ceil(n/S), min(+ceil(n/S), n)); online softmax (m0 = -1e38,
 * corr = exp(m_old - m), l = l*corr + e, acc = acc*corr + e*v); partial layout
 * [B, Hq, S, D+2] = (acc[D], l, m); a split with no blocks writes (0.., 0, -1e38). */
void llo_splitk_partials(const float* q, const float* k_pool,
                         const float* v_pool, const int* block_table,
                         const int* seq_lens, int B, int Hq, int Hkv, int D,
                         int block_size, int max_blocks, int S, float* partial) {
    int groups = Hq / Hkv;
    float scale = 1.0f / sqrtf((float)D);
    for (int b = 0; b < B; b++) {
        int L = seq_lens[b];
        int nb = (L + block_size - 1) / block_size;
        int bps = (nb + S - 1) / S;
        for (int h = 0; h < Hq; h++) {
            int kvh = h / groups;
            const float* qr = q + ((size_t)b * Hq + h) * D;
            for (int s = 0; s < S; s++) {
                float* p = partial + (((size_t)b * Hq + h) * S + s) * (D + 2);
                int b0 = s * bps, b1 = b0 + bps < nb ? b0 + bps : nb;
                float m = -1e38f, l = 0.0f;
                for (int d = 0; d < D; d++) p[d] = 0.0f;
                if (b0 >= nb) { p[D] = 0.0f; p[D + 1] = -1e38f; continue; }
                for (int pos = b0 * block_size; pos < b1 * block_size && pos < L; pos++) {
                    int64_t phys = block_table[(size_t)b * max_blocks + pos / block_size];
                    size_t rowoff = (((size_t)phys * block_size + pos % block_size) * Hkv + kvh) * D;
                    float dot = 0.0f;
                    for (int d = 0; d < D; d++) dot += qr[d] * k_pool[rowoff + d];
                    dot *= scale;
                    float m_old = m;
                    m = fmaxf(m_old, dot);
                    float corr = expf(m_old - m);
                    float e = expf(dot - m);
                    l = l * corr + e;
                    for (int d = 0; d < D; d++) p[d] = p[d] * corr + e * v_pool[rowoff + d];
                }
                p[D] = l;
                p[D + 1] = m;
            }
        }
    }
}

/* src/kv_cache/paged_attention.cu:477-532 (paged_attention_reduce_kernel), restated:
 * skip l_s == 0; first live split initialises; then branch on m < m_s;
 * out = (l == 0) ? 0 : acc/(l + 1e-8). */
void llo_splitk_merge(const float* partial, int B, int Hq, int D, int S, float* out) {
    for (int b = 0; b < B; b++) {
        for (int h = 0; h < Hq; h++) {
            const float* base = partial + ((size_t)b * Hq + h) * S * (D + 2);
            float* o = out + ((size_t)b * Hq + h) * D;
            float m = -1e38f, l = 0.0f;
            for (int d = 0; d < D; d++) o[d] = 0.0f;
            for (int s = 0; s < S; s++) {
                const float* p = base + (size_t)s * (D + 2);
                float l_s = p[D];
                if (l_s == 0.0f) continue;
                float m_s = p[D + 1];
                if (l == 0.0f) {
                    m = m_s; l = l_s;
                    for (int d = 0; d < D; d++) o[d] = p[d];
                    continue;
                }
                float m_max = fmaxf(m, m_s);
                if (m < m_s) {
                    float so = expf(m - m_max);
                    l = l * so + l_s;
                    for (int d = 0; d < D; d++) o[d] = o[d] * so + p[d];
                } else {
                    float sn = expf(m_s - m_max);
                    l = l + l_s * sn;
                    for (int d = 0; d < D; d++) o[d] += p[d] * sn;
                }
                m = m_max;
            }
            for (int d = 0; d < D; d++) o[d] = (l == 0.0f) ? 0.0f : o[d] / (l + 1e-8f);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Prefill                                                                   */
/* ------------------------------------------------------------------------ */

/* One (query row, head) of tests/test_paged_prefill.cu:113-158 (cpu_prefill_attention):
 * online softmax (m0 = -1e38, corr = exp(m_old - m), l = l*corr + e, acc = acc*corr + e*v),
 * output acc * 1/(l + 1e-8), over the first `att` keys (rows of `stride` floats). */
static void prefill_row_f32(const float* qr, int D, const float* k, const float* v,
                            size_t stride, int att, float scale, float* acc, float* o) {
    float mx = -1e38f, l = 0.0f;
    for (int d = 0; d < D; d++) acc[d] = 0.0f;
    for (int pos = 0; pos < att; pos++) {
        const float* kr = k + (size_t)pos * stride;
        const float* vr = v + (size_t)pos * stride;
        float dot = 0.0f;
        for (int d = 0; d < D; d++) dot += qr[d] * kr[d];
        dot *= scale;
        float m_old = mx;
        mx = fmaxf(mx, dot);
        float corr = expf(m_old - mx);
        float e = expf(dot - mx);
        l = l * corr + e;
        for (int d = 0; d < D; d++) acc[d] = acc[d] * corr + e * vr[d];
    }
    float inv = 1.0f / (l + 1e-8f);
    for (int d = 0; d < D; d++) o[d] = acc[d] * inv;
}

/* Keys visible to query t of a P-row chunk over total_seq keys.  The causal rule follows
 * the kernel, src/kv_cache/paged_attention.cu:658,712: query t sits at
 * abs = total_seq - P + t and attends keys pos <= abs (self included). */
static int visible_keys(int causal, int total_seq, int P, int t) {
    int att = causal ? total_seq - P + t + 1 : total_seq;
    if (att > total_seq) att = total_seq;
    return att < 0 ? 0 : att;
}

void llo_prefill_attention(const float* q, int P, int Hq, int D, const float* k,
                           int total_seq, int Hkv, const float* v, int causal,
                           float* out) {
    int groups = Hq / Hkv;
    float scale = 1.0f / sqrtf((float)D);
    float* acc = (float*)malloc(sizeof(float) * D);
    for (int t = 0; t < P; t++)
        for (int h = 0; h < Hq; h++)
            prefill_row_f32(q + ((size_t)t * Hq + h) * D, D, k + (size_t)(h / groups) * D,
                            v + (size_t)(h / groups) * D, (size_t)Hkv * D,
                            visible_keys(causal, total_seq, P, t), scale, acc,
                            out + ((size_t)t * Hq + h) * D);
    free(acc);
}

/* Exact softmax in double (tie-breaker), same masking rule. */
void llo_prefill_attention_f64(const float* q, int P, int Hq, int D,
                               const float* k, int total_seq, int Hkv,
                               const float* v, int causal, double* out) {
    int groups = Hq / Hkv;
    double* sc = (double*)malloc(sizeof(double) * (total_seq > 0 ? total_seq : 1));
    for (int t = 0; t < P; t++)
        for (int h = 0; h < Hq; h++)
            attn_row_f64(q + ((size_t)t * Hq + h) * D, D, k + (size_t)(h / groups) * D,
                         v + (size_t)(h / groups) * D, (size_t)Hkv * D,
                         visible_keys(causal, total_seq, P, t), sc,
                         out + ((size_t)t * Hq + h) * D);
    free(sc);
}

/* tests/test_paged_prefill.cu:164-210 (cpu_prefill_attention_causal) verbatim in rule:
 * att_len = seq_len - (P-1-t); rows with att_len <= 0 stay zero. */
void llo_prefill_attention_test_causal(const float* q, int P, int Hq, int D,
                                       const float* k, int seq_len, int Hkv,
                                       const float* v, float* out) {
    int groups = Hq / Hkv;
    float scale = 1.0f / sqrtf((float)D);
    float* acc = (float*)malloc(sizeof(float) * D);
    memset(out, 0, sizeof(float) * (size_t)P * Hq * D);
    for (int t = 0; t < P; t++) {
        int att_len = seq_len - (P - 1 - t);
        if (att_len <= 0) continue;
        for (int h = 0; h < Hq; h++) {
            int kvh = h / groups;
            const float* qr = q + ((size_t)t * Hq + h) * D;
            float mx = -1e38f, l = 0.0f;
            for (int d = 0; d < D; d++) acc[d] = 0.0f;
            for (int pos = 0; pos < att_len; pos++) {
                const float* kr = k + ((size_t)pos * Hkv + kvh) * D;
                float dot = 0.0f;
                for (int d = 0; d < D; d++) dot += qr[d] * kr[d];
                dot *= scale;
                float m_old = mx;
                mx = fmaxf(mx, dot);
                float corr = expf(m_old - mx);
                float e = expf(dot - mx);
                l = l * corr + e;
                for (int d = 0; d < D; d++)
                    acc[d] = acc[d] * corr + e * v[((size_t)pos * Hkv + kvh) * D + d];
            }
            float inv = 1.0f / (l + 1e-8f);
            float* o = out + ((size_t)t * Hq + h) * D;
            for (int d = 0; d < D; d++) o[d] = acc[d] * inv;
        }
    }
    free(acc);
}

/* Paged prefill for N sequences (varlen): sequence n has q rows [cu_q[n], cu_q[n+1])
 * and seq_lens[n] total keys (history + chunk).  Per sequence: reconstruct_kv
 * (tests/test_paged_prefill.cu:216-239) then the prefill attention above -- the
 * "old reconstruction" path of tests/test_paged_prefill.cu:244-256. */
static void prefill_impl(const float* q, const int* cu_q, const float* k_pool,
                         const float* v_pool, const int* block_table,
                         const int* seq_lens, int N, int Hq, int Hkv, int D,
                         int block_size, int max_blocks, int causal, float* out32,
                         double* out64, int nthreads) {
    size_t row = (size_t)Hkv * D;
    if (nthreads < 1) nthreads = 1;
    int groups = Hq / Hkv;
    float scale = 1.0f / sqrtf((float)D);
    for (int n = 0; n < N; n++) {
        int L = seq_lens[n];
        int P = cu_q[n + 1] - cu_q[n];
        float* kc = (float*)malloc(sizeof(float) * ((size_t)L * row + 1));
        float* vc = (float*)malloc(sizeof(float) * ((size_t)L * row + 1));
        llo_reconstruct_kv(kc, vc, k_pool, v_pool, block_table + (size_t)n * max_blocks,
                           L, block_size, Hkv, D, (int)sizeof(float));
        /* OpenMP over (query row, q_head) */
#pragma omp parallel num_threads(nthreads)
        {
            float* acc = (float*)malloc(sizeof(float) * D);
            double* sc = (double*)malloc(sizeof(double) * (L > 0 ? L : 1));
#pragma omp for schedule(dynamic) collapse(2)
            for (int t = 0; t < P; t++) {
                for (int h = 0; h < Hq; h++) {
                    int att = visible_keys(causal, L, P, t);
                    const float* kb = kc + (size_t)(h / groups) * D;
                    const float* vb = vc + (size_t)(h / groups) * D;
                    const float* qr = q + ((size_t)(cu_q[n] + t) * Hq + h) * D;
                    size_t o = ((size_t)(cu_q[n] + t) * Hq + h) * D;
                    if (out32) prefill_row_f32(qr, D, kb, vb, row, att, scale, acc, out32 + o);
                    if (out64) attn_row_f64(qr, D, kb, vb, row, att, sc, out64 + o);
                }
            }
            free(acc);
            free(sc);
        }
        free(kc);
        free(vc);
    }
}

void llo_paged_prefill(const float* q, const int* cu_q, const float* k_pool,
                       const float* v_pool, const int* block_table,
                       const int* seq_lens, int N, int Hq, int Hkv, int D,
                       int block_size, int max_blocks, int causal, float* out,
                       int nthreads) {
    prefill_impl(q, cu_q, k_pool, v_pool, block_table, seq_lens, N, Hq, Hkv, D,
                 block_size, max_blocks, causal, out, NULL, nthreads);
}

void llo_paged_prefill_f64(const float* q, const int* cu_q, const float* k_pool,
                           const float* v_pool, const int* block_table,
                           const int* seq_lens, int N, int Hq, int Hkv, int D,
                           int block_size, int max_blocks, int causal,
                           double* out, int nthreads) {
    prefill_impl(q, cu_q, k_pool, v_pool, block_table, seq_lens, N, Hq, Hkv, D,
                 block_size, max_blocks, causal, NULL, out, nthreads);
}

/* src/kv_cache/paged_attention.cu:1230-1325 (first_prefill_attn_batched_kernel), restated:
 * row g of entry e (local r): keys pos in [0, num_tokens[e]) with start+pos <= start+r,
 * K/V element offset kv_offsets[e] + pos*Hkv*D + kvh*D, Q offset offsets[e] + r*Hq*D + h*D,
 * output row offsets[e]/(Hq*D) + r; online softmax with +1e-8. */
void llo_first_prefill_batched(float* out, const float* q, const float* k,
                               const float* v, int Hq, int Hkv, int D,
                               const int* offsets, const int* kv_offsets,
                               const int* num_tokens, const int* token_cumsum,
                               const int* start_poss, int N, int P_total,
                               float scale) {
    int groups = Hq / Hkv;
    float* acc = (float*)malloc(sizeof(float) * D);
    for (int g = 0; g < P_total; g++) {
        int e = 0;
        while (e < N && g >= token_cumsum[e + 1]) e++;
        int r = g - token_cumsum[e];
        int abs_q = start_poss[e] + r;
        for (int h = 0; h < Hq; h++) {
            int kvh = h / groups;
            const float* qr = q + (size_t)offsets[e] + (size_t)r * Hq * D + (size_t)h * D;
            float mx = -1e38f, l = 0.0f;
            for (int d = 0; d < D; d++) acc[d] = 0.0f;
            for (int pos = 0; pos < num_tokens[e]; pos++) {
                if (start_poss[e] + pos > abs_q) break;
                const float* kr = k + (size_t)kv_offsets[e] + (size_t)pos * Hkv * D + (size_t)kvh * D;
                const float* vr = v + (size_t)kv_offsets[e] + (size_t)pos * Hkv * D + (size_t)kvh * D;
                float dot = 0.0f;
                for (int d = 0; d < D; d++) dot += qr[d] * kr[d];
                dot *= scale;
                float m_old = mx;
                mx = fmaxf(mx, dot);
                float corr = expf(m_old - mx);
                float ee = expf(dot - mx);
                l = l * corr + ee;
                for (int d = 0; d < D; d++) acc[d] = acc[d] * corr + ee * vr[d];
            }
            int out_row = offsets[e] / (Hq * D) + r;
            float* o = out + ((size_t)out_row * Hq + h) * D;
            for (int d = 0; d < D; d++) o[d] = acc[d] / (l + 1e-8f);
        }
    }
    free(acc);
}

/* src/kv_cache/hash_prefix_cache.cpp:23-30 (FNV-1a 64 over (uint32)token). */
uint64_t llo_fnv1a_tokens(const int* tokens, int n) {
    uint64_t h = 14695981039346656037ULL;
    for (int i = 0; i < n; i++) {
        h ^= (uint64_t)(uint32_t)tokens[i];
        h *= 1099511628211ULL;
    }
    return h;
}
