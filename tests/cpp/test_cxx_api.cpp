// Tests of the reference-signature C++ API (lightllm::kv_cache), written the
// way the reference's own tests are (standalone main, CHECK counter).
//
//   test_cxx_api cpu   BlockAllocator / BlockTable semantics, no GPU
//                      (restating tests/test_paged_attention.cu:48-66 and
//                      tests/test_paged_attention_v2.cu:610-650, plus the
//                      FIFO / hash-probe / eviction / reset rules of
//                      src/kv_cache/block_allocator.cpp)
//   test_cxx_api gpu   paged_attention, prefill_paged_attention,
//                      scatter_prefill_kv_gpu, the batched scatter and
//                      first-prefill entry points, against the CPU oracle
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <numeric>
#include <stdexcept>
#include <vector>

#include "cpu_ref.h"
#include "lightllm/kv_cache/block_allocator.h"
#include "lightllm/kv_cache/paged_attention.h"

using namespace lightllm;
using namespace lightllm::kv_cache;

static int passed = 0, failed = 0;
static void CHECK(const char* name, bool cond) {
    if (cond) {
        ++passed;
    } else {
        ++failed;
        std::fprintf(stderr, "  FAIL: %s\n", name);
    }
}

// ---------------------------------------------------------------------------
static void test_allocator_cpu() {
    BlockAllocator alloc(64, 16, 2, 64, PrefixCachePolicy::Hash, DType::F32, PoolStorage::None);
    CHECK("num_blocks", alloc.num_blocks() == 64);
    CHECK("num_free", alloc.num_free() == 64);
    CHECK("block_size", alloc.block_size() == 16);
    CHECK("hkv", alloc.num_kv_heads() == 2);
    CHECK("hdim", alloc.head_dim() == 64);
    // 288 GB of fp16 K+V, Llama-3-8B heads: 288e9 / (16 * 8 * 128 * 2 B * 2) pages
    CHECK("budget_288GB_fp16", BlockAllocator::blocks_for_budget(288000000000ull, 16, 8, 128, DType::F16) ==
                                   (int)(288000000000ull / 65536));
    CHECK("budget_fp32_half", BlockAllocator::blocks_for_budget(1ull << 30, 16, 2, 64, DType::F32) ==
                                  2 * BlockAllocator::blocks_for_budget(1ull << 30, 16, 2, 128, DType::F32));
    int b0 = alloc.allocate(0x123), b1 = alloc.allocate(0x456);
    CHECK("fifo_0", b0 == 0);
    CHECK("fifo_1", b1 == 1);
    CHECK("free_62", alloc.num_free() == 62);
    CHECK("hash_kept", alloc.block(b0).token_hash == 0x123);
    alloc.release(b0);
    alloc.release(b1);
    CHECK("free_64", alloc.num_free() == 64);
    // released blocks go to the back of the FIFO
    CHECK("fifo_after_release", alloc.allocate() == 2);
    alloc.release(2);
    std::vector<int> all;
    for (int i = 0; i < 64; ++i) all.push_back(alloc.allocate());
    bool ok = true;
    for (int b : all) ok = ok && b >= 0;
    CHECK("bulk", ok);
    CHECK("exhausted", alloc.num_free() == 0);
    CHECK("alloc_fail", alloc.allocate() == -1);
    for (int b : all) alloc.release(b);
    CHECK("all_free_again", alloc.num_free() == 64);
    alloc.release(5);   // ref already 0: ignored
    CHECK("double_release_ignored", alloc.num_free() == 64);

    // hash probe + prefix sharing
    std::vector<int> toks(40);
    std::iota(toks.begin(), toks.end(), 100);
    std::vector<int> blocks;
    int n_new = alloc.allocate_tokens(toks.data(), 40, 0, blocks);
    CHECK("tokens_new_3", n_new == 3 && blocks.size() == 3);
    uint64_t h0 = HashPrefixCache::hash_tokens(toks.data(), 16);
    CHECK("tokens_hash_full_block", alloc.block(blocks[0]).token_hash == h0);
    CHECK("tokens_hash_partial_zero", alloc.block(blocks[2]).token_hash == 0);
    CHECK("find_by_hash", alloc.find_by_hash(h0) == blocks[0]);
    int again = alloc.allocate(h0);
    CHECK("probe_hit_same_id", again == blocks[0]);
    CHECK("probe_hit_ref2", alloc.block(blocks[0]).ref_count == 2);
    std::vector<int> blocks2;
    int n_new2 = alloc.allocate_tokens(toks.data(), 40, 0, blocks2);
    CHECK("share_prefix_new_1", n_new2 == 1 && blocks2.size() == 3);
    CHECK("share_prefix_ids", blocks2[0] == blocks[0] && blocks2[1] == blocks[1]);
    auto hit = alloc.find_cached_prefix(toks, 0);
    CHECK("cached_prefix_32", hit.matched_tokens == 32);

    // LRU eviction on exhaustion: free every block; cached ones stay evictable
    alloc.reset();
    CHECK("reset_free", alloc.num_free() == 64);
    CHECK("reset_cache_empty", alloc.prefix_cache()->size() == 0);
    std::vector<int> held;
    std::vector<int> t16(16);
    std::iota(t16.begin(), t16.end(), 7);
    std::vector<int> cached;
    alloc.allocate_tokens(t16.data(), 16, 0, cached);
    CHECK("cached_one", cached.size() == 1 && alloc.prefix_cache()->size() == 1);
    for (int i = 0; i < 63; ++i) held.push_back(alloc.allocate());
    CHECK("pool_full", alloc.num_free() == 0 && alloc.allocate() == -1);
    alloc.release(cached[0]);   // ref 0: removed from use, freed, still cached
    CHECK("freed_cached", alloc.num_free() == 1);
    int x = alloc.allocate();
    CHECK("reuse_freed", x == cached[0]);
    // now exhausted; the cache entry of x is evictable (ref 0 in the cache)
    int y = alloc.allocate();
    CHECK("evict_then_alloc", y == cached[0]);

    // BlockTable
    BlockTable bt(8);
    bt.append(3);
    bt.append(7);
    bt.append(12);
    CHECK("bt_size", bt.size() == 3);
    CHECK("bt_0", bt[0] == 3 && bt[1] == 7 && bt[2] == 12);
    for (int i = 3; i < 8; ++i) bt.append(i * 10);
    CHECK("bt_full", bt.size() == 8 && bt[7] == 70);
    bool threw = false;
    try {
        bt.append(1);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    CHECK("bt_overflow_throws", threw);

    // policy from env
    setenv("LIGHTLLM_PREFIX_CACHE", "radix", 1);
    CHECK("env_radix", prefix_cache_policy_from_env() == PrefixCachePolicy::Radix);
    setenv("LIGHTLLM_PREFIX_CACHE", "bogus", 1);
    CHECK("env_default_hash", prefix_cache_policy_from_env() == PrefixCachePolicy::Hash);
    unsetenv("LIGHTLLM_PREFIX_CACHE");

    // pools sized past 2^32 elements use 64-bit offsets (no device memory touched)
    BlockAllocator big(262144, 16, 8, 128, PrefixCachePolicy::Hash, DType::F16, PoolStorage::None);
    CHECK("block_bytes_llama", big.block_bytes() == 16u * 8 * 128 * 2);
}

// ---------------------------------------------------------------------------
static std::vector<float> rnd(size_t n, unsigned seed) {
    std::vector<float> v(n);
    llo_fill_random(v.data(), n, seed);
    return v;
}

static bool close(const std::vector<float>& got, const std::vector<double>& ref, double rtol,
                  double atol, const char* what) {
    double worst = 0;
    bool ok = true;
    for (size_t i = 0; i < got.size(); ++i) {
        double e = std::fabs((double)got[i] - ref[i]);
        if (e > atol + rtol * std::fabs(ref[i])) ok = false;
        worst = std::max(worst, e);
    }
    std::printf("  %-40s max abs err %.3e\n", what, worst);
    return ok;
}

static void test_ops_gpu() {
    const int Hq = 14, Hkv = 2, D = 64, bs = 16, nb = 256;
    BlockAllocator alloc(nb, bs, Hkv, D);   // device pools, fp32, as the reference default
    const size_t row = (size_t)Hkv * D;

    // ---- scatter a 300-token sequence through scatter_prefill_kv_gpu ----
    const int L = 300, nblk = (L + bs - 1) / bs;
    std::vector<int> table;
    for (int i = 0; i < nblk; ++i) table.push_back(alloc.allocate());
    std::vector<float> kc = rnd((size_t)L * row, 11), vc = rnd((size_t)L * row, 12);
    Tensor kt({L, Hkv, D}, DType::F32, Device::CUDA), vt({L, Hkv, D}, DType::F32, Device::CUDA);
    kt.copy_from(kc.data(), kc.size() * 4);
    vt.copy_from(vc.data(), vc.size() * 4);
    Tensor bt({nblk}, DType::I32, Device::CUDA);
    bt.copy_from(table.data(), table.size() * 4);
    scatter_prefill_kv_gpu(kt, vt, 0, L, bt.data<int>(), nblk, alloc);
    (void)hipDeviceSynchronize();

    std::vector<float> kpool((size_t)nb * bs * row), vpool((size_t)nb * bs * row);
    (void)hipMemcpy(kpool.data(), alloc.k_storage_raw(), kpool.size() * 4, hipMemcpyDeviceToHost);
    (void)hipMemcpy(vpool.data(), alloc.v_storage_raw(), vpool.size() * 4, hipMemcpyDeviceToHost);
    std::vector<float> kg((size_t)L * row), vg((size_t)L * row);
    llo_reconstruct_kv(kg.data(), vg.data(), kpool.data(), vpool.data(), table.data(), L, bs, Hkv, D, 4);
    CHECK("scatter_bit_exact", std::memcmp(kg.data(), kc.data(), kc.size() * 4) == 0 &&
                                   std::memcmp(vg.data(), vc.data(), vc.size() * 4) == 0);

    // ---- paged_attention: one decode token over the 300 keys ----
    std::vector<float> q = rnd((size_t)Hq * D, 13);
    Tensor qt({1, Hq, D}, DType::F32, Device::CUDA);
    qt.copy_from(q.data(), q.size() * 4);
    Tensor sl({1}, DType::I32, Device::CUDA);
    sl.copy_from(&L, 4);
    Tensor out = paged_attention(qt, bt.data<int>(), nblk, sl.data<int>(), alloc);
    std::vector<float> got((size_t)Hq * D);
    out.copy_to(got.data(), got.size() * 4);
    std::vector<double> ref((size_t)Hq * D);
    llo_cpu_attention_f64(q.data(), 1, Hq, D, kc.data(), L, Hkv, vc.data(), ref.data());
    CHECK("paged_attention_shape", out.size(0) == 1 && out.size(1) == Hq && out.size(2) == D);
    CHECK("paged_attention_fp32", close(got, ref, 1e-5, 1e-6, "paged_attention fp32 L=300"));

    // ---- prefill_paged_attention: last 44 tokens as a chunk over 256 history ----
    const int P = 44;
    std::vector<float> qp = rnd((size_t)P * Hq * D, 14);
    Tensor qpt({P, Hq, D}, DType::F32, Device::CUDA);
    qpt.copy_from(qp.data(), qp.size() * 4);
    for (int causal = 0; causal < 2; ++causal) {
        Tensor op = prefill_paged_attention(qpt, bt.data<int>(), nblk, sl.data<int>(), alloc, causal);
        std::vector<float> g2((size_t)P * Hq * D);
        op.copy_to(g2.data(), g2.size() * 4);
        std::vector<double> r2((size_t)P * Hq * D);
        llo_prefill_attention_f64(qp.data(), P, Hq, D, kc.data(), L, Hkv, vc.data(), causal, r2.data());
        CHECK(causal ? "prefill_causal_fp32" : "prefill_noncausal_fp32",
              close(g2, r2, 1e-5, 1e-6, causal ? "prefill causal fp32" : "prefill non-causal fp32"));
    }

    // ---- dtype mismatch throws (the reference left it undefined) ----
    Tensor q16({1, Hq, D}, DType::F16, Device::CUDA);
    bool threw = false;
    try {
        paged_attention(q16, bt.data<int>(), nblk, sl.data<int>(), alloc);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    CHECK("dtype_mismatch_throws", threw);
    threw = false;
    try {
        Tensor qbig({1, Hq, 320}, DType::F32, Device::CUDA);
        paged_attention(qbig, bt.data<int>(), nblk, sl.data<int>(), alloc);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    CHECK("head_dim_too_large_throws", threw);

    // ---- batched first prefill: scatter + contiguous causal attention ----
    const int N = 3;
    int ntok[N] = {5, 17, 33};
    std::vector<int> cum(N + 1, 0), offs(N), kvoffs(N), starts(N, 0);
    for (int e = 0; e < N; ++e) cum[e + 1] = cum[e] + ntok[e];
    const int Ptot = cum[N];
    for (int e = 0; e < N; ++e) {
        offs[e] = cum[e] * Hq * D;
        kvoffs[e] = cum[e] * Hkv * D;
    }
    const int mb = 4;
    std::vector<int> flat((size_t)N * mb, -1);
    for (int e = 0; e < N; ++e)
        for (int b = 0; b < (ntok[e] + bs - 1) / bs; ++b) flat[(size_t)e * mb + b] = alloc.allocate();
    std::vector<float> qf = rnd((size_t)Ptot * Hq * D, 21), kf = rnd((size_t)Ptot * row, 22),
                       vf = rnd((size_t)Ptot * row, 23);
    auto dev_i = [](const std::vector<int>& h) {
        Tensor t({(int)h.size()}, DType::I32, Device::CUDA);
        t.copy_from(h.data(), h.size() * 4);
        return t;
    };
    Tensor d_cum = dev_i(cum), d_offs = dev_i(offs), d_kvoffs = dev_i(kvoffs), d_starts = dev_i(starts),
           d_flat = dev_i(flat), d_ntok = dev_i(std::vector<int>(ntok, ntok + N));
    Tensor d_q({Ptot, Hq, D}, DType::F32, Device::CUDA), d_k({Ptot, Hkv, D}, DType::F32, Device::CUDA),
        d_v({Ptot, Hkv, D}, DType::F32, Device::CUDA), d_o({Ptot, Hq, D}, DType::F32, Device::CUDA);
    d_q.copy_from(qf.data(), qf.size() * 4);
    d_k.copy_from(kf.data(), kf.size() * 4);
    d_v.copy_from(vf.data(), vf.size() * 4);
    scatter_prefill_kv_batched_gpu(d_k.data<float>(), d_v.data<float>(), Hkv, D, d_kvoffs.data<int>(),
                                   d_ntok.data<int>(), d_starts.data<int>(), d_cum.data<int>(),
                                   d_flat.data<int>(), mb, N, Ptot, alloc);
    (void)hipMemcpy(kpool.data(), alloc.k_storage_raw(), kpool.size() * 4, hipMemcpyDeviceToHost);
    bool exact = true;
    for (int e = 0; e < N; ++e) {
        std::vector<float> k1((size_t)ntok[e] * row), v1((size_t)ntok[e] * row);
        llo_reconstruct_kv(k1.data(), v1.data(), kpool.data(), kpool.data(), &flat[(size_t)e * mb],
                           ntok[e], bs, Hkv, D, 4);
        exact = exact && std::memcmp(k1.data(), &kf[(size_t)cum[e] * row], k1.size() * 4) == 0;
    }
    CHECK("scatter_batched_bit_exact", exact);
    first_prefill_attn_batched_gpu(d_o.data<float>(), d_q.data<float>(), d_k.data<float>(),
                                   d_v.data<float>(), Hq, Hkv, D, d_offs.data<int>(),
                                   d_kvoffs.data<int>(), d_ntok.data<int>(), d_cum.data<int>(),
                                   d_starts.data<int>(), N, Ptot, 1.0f / std::sqrt((float)D));
    std::vector<float> g3((size_t)Ptot * Hq * D), r3f((size_t)Ptot * Hq * D);
    d_o.copy_to(g3.data(), g3.size() * 4);
    llo_first_prefill_batched(r3f.data(), qf.data(), kf.data(), vf.data(), Hq, Hkv, D, offs.data(),
                              kvoffs.data(), ntok, cum.data(), starts.data(), N, Ptot,
                              1.0f / std::sqrt((float)D));
    std::vector<double> r3(r3f.begin(), r3f.end());
    CHECK("first_prefill_batched_fp32", close(g3, r3, 2e-5, 2e-6, "first_prefill_batched fp32"));
}

// Fused RoPE + append and the device slot mapping through the C++ API, bit for bit the oracle's.
static void test_rope_append_gpu() {
    const int Hq = 14, Hkv = 2, D = 64, bs = 16, nb = 32, T = 5;
    BlockAllocator alloc(nb, bs, Hkv, D);
    std::vector<int> table;
    for (int i = 0; i < 4; ++i) table.push_back(alloc.allocate());
    const int cu[2] = {0, T}, start[1] = {13};   // positions 13..17 cross a page boundary
    Tensor d_bt({4}, DType::I32, Device::CUDA), d_cu({2}, DType::I32, Device::CUDA),
        d_st({1}, DType::I32, Device::CUDA);
    d_bt.copy_from(table.data(), 16);
    d_cu.copy_from(cu, 8);
    d_st.copy_from(start, 4);
    int64_t* slots = nullptr;
    (void)hipMalloc(&slots, T * sizeof(int64_t));
    build_slots(slots, d_bt.data<int>(), 4, d_cu.data<int>(), d_st.data<int>(), 1, T, alloc);
    std::vector<int64_t> got_slots(T), want_slots(T);
    (void)hipMemcpy(got_slots.data(), slots, T * sizeof(int64_t), hipMemcpyDeviceToHost);
    llo_build_slots(want_slots.data(), table.data(), 4, cu, start, 1, T, bs);
    CHECK("build_slots", got_slots == want_slots);

    std::vector<float> q = rnd((size_t)T * Hq * D, 31), k = rnd((size_t)T * Hkv * D, 32),
                       v = rnd((size_t)T * Hkv * D, 33), cs((size_t)T * D / 2), sn((size_t)T * D / 2);
    for (int t = 0; t < T; ++t)
        for (int i = 0; i < D / 2; ++i) {
            const double ang = (start[0] + t) / std::pow(10000.0, 2.0 * i / D);
            cs[(size_t)t * D / 2 + i] = (float)std::cos(ang);
            sn[(size_t)t * D / 2 + i] = (float)std::sin(ang);
        }
    Tensor tq({T, Hq, D}, DType::F32, Device::CUDA), tk({T, Hkv, D}, DType::F32, Device::CUDA),
        tv({T, Hkv, D}, DType::F32, Device::CUDA), tc({T, D / 2}, DType::F32, Device::CUDA),
        ts({T, D / 2}, DType::F32, Device::CUDA);
    tq.copy_from(q.data(), q.size() * 4);
    tk.copy_from(k.data(), k.size() * 4);
    tv.copy_from(v.data(), v.size() * 4);
    tc.copy_from(cs.data(), cs.size() * 4);
    ts.copy_from(sn.data(), sn.size() * 4);
    std::vector<float> kp((size_t)nb * bs * Hkv * D), vp(kp.size());
    (void)hipMemcpy(kp.data(), alloc.k_storage_raw(), kp.size() * 4, hipMemcpyDeviceToHost);
    (void)hipMemcpy(vp.data(), alloc.v_storage_raw(), vp.size() * 4, hipMemcpyDeviceToHost);
    rope_append_kv(&tq, tk, tv, slots, tc, ts, alloc);
    (void)hipDeviceSynchronize();
    llo_rope_append(q.data(), k.data(), v.data(), kp.data(), vp.data(), want_slots.data(), cs.data(),
                    sn.data(), T, Hq, Hkv, D, D, 0);
    std::vector<float> gq(q.size()), gk(k.size()), gkp(kp.size()), gvp(vp.size());
    tq.copy_to(gq.data(), gq.size() * 4);
    tk.copy_to(gk.data(), gk.size() * 4);
    (void)hipMemcpy(gkp.data(), alloc.k_storage_raw(), gkp.size() * 4, hipMemcpyDeviceToHost);
    (void)hipMemcpy(gvp.data(), alloc.v_storage_raw(), gvp.size() * 4, hipMemcpyDeviceToHost);
    CHECK("rope_append_q_bit_exact", std::memcmp(gq.data(), q.data(), q.size() * 4) == 0);
    CHECK("rope_append_k_bit_exact", std::memcmp(gk.data(), k.data(), k.size() * 4) == 0);
    CHECK("rope_append_pools_bit_exact", std::memcmp(gkp.data(), kp.data(), kp.size() * 4) == 0 &&
                                             std::memcmp(gvp.data(), vp.data(), vp.size() * 4) == 0);
    (void)hipFree(slots);
}

// paged_attention_append == append_kv_slots then paged_attention, bit for bit.
static void test_decode_append_gpu() {
    const int Hq = 14, Hkv = 2, D = 64, bs = 16, nb = 64, B = 3, mb = 4;
    BlockAllocator fa(nb, bs, Hkv, D), ua(nb, bs, Hkv, D);
    const size_t pool = (size_t)nb * bs * Hkv * D;
    std::vector<float> kp = rnd(pool, 41), vp = rnd(pool, 42);
    for (BlockAllocator* a : {&fa, &ua}) {
        (void)hipMemcpy(const_cast<void*>(a->k_storage_raw()), kp.data(), pool * 4, hipMemcpyHostToDevice);
        (void)hipMemcpy(const_cast<void*>(a->v_storage_raw()), vp.data(), pool * 4, hipMemcpyHostToDevice);
    }
    const int lens[B] = {5, 16, 40};   // after the append: new tokens at 4, 15, 39
    std::vector<int> table((size_t)B * mb, -1);
    int next = 3;
    for (int b = 0; b < B; ++b)
        for (int p = 0; p < (lens[b] + bs - 1) / bs; ++p) table[(size_t)b * mb + p] = next++ * 2 % nb;
    std::vector<int64_t> slots(B);
    for (int b = 0; b < B; ++b) {
        const int pos = lens[b] - 1;
        slots[b] = (int64_t)table[(size_t)b * mb + pos / bs] * bs + pos % bs;
    }
    Tensor d_bt({B * mb}, DType::I32, Device::CUDA), d_sl({B}, DType::I32, Device::CUDA);
    d_bt.copy_from(table.data(), table.size() * 4);
    d_sl.copy_from(lens, sizeof(lens));
    std::vector<float> q = rnd((size_t)B * Hq * D, 43), kn = rnd((size_t)B * Hkv * D, 44),
                       vn = rnd((size_t)B * Hkv * D, 45);
    Tensor tq({B, Hq, D}, DType::F32, Device::CUDA), tk({B, Hkv, D}, DType::F32, Device::CUDA),
        tv({B, Hkv, D}, DType::F32, Device::CUDA);
    tq.copy_from(q.data(), q.size() * 4);
    tk.copy_from(kn.data(), kn.size() * 4);
    tv.copy_from(vn.data(), vn.size() * 4);
    int64_t* d_slots = nullptr;
    (void)hipMalloc(&d_slots, B * sizeof(int64_t));
    (void)hipMemcpy(d_slots, slots.data(), B * sizeof(int64_t), hipMemcpyHostToDevice);
    Tensor fused = paged_attention_append(tq, tk, tv, d_bt.data<int>(), mb, d_sl.data<int>(), fa);
    append_kv_slots(tk, tv, d_slots, ua);
    Tensor plain = paged_attention(tq, d_bt.data<int>(), mb, d_sl.data<int>(), ua);
    (void)hipDeviceSynchronize();
    std::vector<float> of((size_t)B * Hq * D), op(of.size()), fk(pool), uk(pool), fv(pool), uv(pool);
    fused.copy_to(of.data(), of.size() * 4);
    plain.copy_to(op.data(), op.size() * 4);
    (void)hipMemcpy(fk.data(), fa.k_storage_raw(), pool * 4, hipMemcpyDeviceToHost);
    (void)hipMemcpy(uk.data(), ua.k_storage_raw(), pool * 4, hipMemcpyDeviceToHost);
    (void)hipMemcpy(fv.data(), fa.v_storage_raw(), pool * 4, hipMemcpyDeviceToHost);
    (void)hipMemcpy(uv.data(), ua.v_storage_raw(), pool * 4, hipMemcpyDeviceToHost);
    CHECK("decode_append_output_bit_exact", std::memcmp(of.data(), op.data(), of.size() * 4) == 0);
    CHECK("decode_append_pools_bit_exact", std::memcmp(fk.data(), uk.data(), pool * 4) == 0 &&
                                               std::memcmp(fv.data(), uv.data(), pool * 4) == 0);
    (void)hipFree(d_slots);
}

int main(int argc, char** argv) {
    const bool gpu = argc > 1 && std::strcmp(argv[1], "gpu") == 0;
    if (gpu) {
        std::printf("== C++ API on the GPU\n");
        test_ops_gpu();
        test_rope_append_gpu();
        test_decode_append_gpu();
    } else {
        std::printf("== BlockAllocator / BlockTable (CPU)\n");
        test_allocator_cpu();
    }
    std::printf("%d passed, %d failed, %d total\n", passed, failed, passed + failed);
    return failed == 0 ? 0 : 1;
}
