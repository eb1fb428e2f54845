"""Pins the CPU oracle (oracle/libcpu_ref.so) before it is trusted as the checker.

Every oracle function is compared here with something that does not share its
code: numpy float64 attention written from the softmax definition, numpy fancy
indexing for the page gathers, numpy / torch for IEEE half and bfloat16
rounding, closed forms (one key, equal keys, empty sequence), brute force on
tiny inputs, the associativity of the log-sum-exp merge, and the reference's own
known-answer inputs (ramp data of tests/test_paged_attention.cu:69-130, LCGs of
tests/test_paged_attention_v2.cu:58-64 and tests/test_attention_fp16.cpp:31-38,
FNV-1a 64 test vectors).  A mistake such as a dropped scale, a transposed
head index or an off-by-one causal mask fails at least one of them.
"""
import math

import numpy as np
import pytest
import torch

import oracle

PAGE = 16


# ---------------------------------------------------------------------------
# independent numpy restatements (float64)
# ---------------------------------------------------------------------------

def np_attend(q, k, v, scale, nkeys=None):
    """q [Hq, D]; k, v [L, Hkv, D]; row h attends keys [0, nkeys[h]) (all if None)."""
    hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    out = np.zeros((hq, d))
    for h in range(hq):
        n = k.shape[0] if nkeys is None else nkeys[h]
        if n <= 0:
            continue
        kk = k[:n, h // g].astype(np.float64)
        vv = v[:n, h // g].astype(np.float64)
        s = kk @ q[h].astype(np.float64) * scale
        p = np.exp(s - s.max())
        out[h] = p @ vv / p.sum()
    return out


def np_gather(pool, table_row, n):
    pos = np.arange(n)
    rows = table_row[pos // PAGE].astype(np.int64) * PAGE + pos % PAGE
    return pool.reshape(-1, *pool.shape[2:])[rows]


def make_pools(rng, nb, hkv, d, dtype=np.float32):
    k = rng.standard_normal((nb, PAGE, hkv, d)).astype(dtype)
    v = rng.standard_normal((nb, PAGE, hkv, d)).astype(dtype)
    return k, v


def make_tables(rng, lens, nb, extra=0):
    mb = max(1, max((L + PAGE - 1) // PAGE for L in lens)) + extra
    perm = rng.permutation(nb).astype(np.int32)
    t = np.full((len(lens), mb), -1, np.int32)
    p = 0
    for i, L in enumerate(lens):
        n = (L + PAGE - 1) // PAGE
        t[i, :n] = perm[p:p + n]
        p += n
    return t


def close(a, b, rtol, atol):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    err = np.abs(a - b)
    bound = atol + rtol * np.abs(b)
    assert np.all(err <= bound), f"max excess {np.max(err - bound):.3e}"


# ---------------------------------------------------------------------------
# generators and rounding
# ---------------------------------------------------------------------------

def test_fill_random_known_answers():
    # s_{i+1} = s_i * 1664525 + 1013904223 (mod 2^32); v = (s & 0x7FFF)/16384 - 1
    out = oracle.fill_random(4, 0)
    s, exp = 0, []
    for _ in range(4):
        s = (s * 1664525 + 1013904223) % 2**32
        exp.append((s & 0x7FFF) / 16384.0 - 1.0)
    assert out.tolist() == pytest.approx(exp, abs=0)
    assert out[0] == (1013904223 & 0x7FFF) / 16384.0 - 1.0
    big = oracle.fill_random(100000, 42)
    assert big.min() >= -1.0 and big.max() < 1.0 and abs(big.mean()) < 0.01


def test_rng_randf_known_answers():
    out, st = oracle.rng_randf(3, 1)
    s, exp = 1, []
    for _ in range(3):
        s = (s * 1103515245 + 12345) % 2**32
        exp.append((s & 0x7FFFFFFF) / 2**31 * 2 - 1)
    assert st == s
    np.testing.assert_allclose(out, exp, rtol=0, atol=1e-7)


def _rounding_inputs():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10,
        rng.standard_normal(2000).astype(np.float32) * 1e-6,          # half subnormals
        (rng.standard_normal(2000) * 60000).astype(np.float32),        # near overflow
        np.array([0.0, -0.0, 65504, 65519.99, 65520, -65520, 1e-8, 2**-24, 2**-25,
                  3 * 2**-26, np.inf, -np.inf], np.float32),
    ])
    # exact ties of half: 1 + (2k+1) * 2^-11
    ties = (1.0 + (2 * np.arange(200) + 1) * 2.0**-11).astype(np.float32)
    return np.concatenate([x, ties, -ties])


def test_f16_rounding_matches_numpy():
    x = _rounding_inputs()
    ours = oracle.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(ours, ref)
    nan = oracle.f32_to_f16_bits(np.array([np.nan], np.float32))
    assert np.isnan(nan.view(np.float16)).all()
    back = oracle.f16_bits_to_f32(ref)
    np.testing.assert_array_equal(back, ref.view(np.float16).astype(np.float32))


def test_bf16_rounding_matches_torch():
    x = _rounding_inputs()
    ties = (1.0 + (2 * np.arange(100) + 1) * 2.0**-8).astype(np.float32)
    x = np.concatenate([x, ties, -ties, np.array([3.4e38], np.float32)])
    ours = oracle.f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, ref)
    back = oracle.bf16_bits_to_f32(ref)
    np.testing.assert_array_equal(back, torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16)
                                  .float().numpy())


def test_fnv1a_vectors():
    assert oracle.fnv1a_tokens([]) == 0xCBF29CE484222325
    assert oracle.fnv1a_tokens([0x61]) == 0xAF63DC4C8601EC8C   # FNV-1a 64 of "a"
    assert oracle.fnv1a_tokens([0x61, 0x62, 0x63]) == 0xE71FA2190541574B   # "abc"


# ---------------------------------------------------------------------------
# copies
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [np.float32, np.uint16])
def test_append_and_gather_bit_exact(dtype):
    rng = np.random.default_rng(1)
    nb, hkv, d = 64, 2, 64
    shape = (nb, PAGE, hkv, d)
    k = rng.integers(0, 60000, shape).astype(dtype)   # fp16 / bf16 pools are moved as raw 16-bit words
    v = rng.integers(0, 60000, shape).astype(dtype)
    n = 40
    ks = rng.integers(0, 60000, (n, hkv, d)).astype(dtype)
    vs = rng.integers(0, 60000, (n, hkv, d)).astype(dtype)
    slots = rng.choice(nb * PAGE, n, replace=False).astype(np.int64)
    slots[3] = -1   # skipped
    k2, v2 = k.copy(), v.copy()
    oracle.append_slots(k2, v2, ks, vs, slots)
    ek, ev = k.reshape(-1, hkv, d).copy(), v.reshape(-1, hkv, d).copy()
    m = slots >= 0
    ek[slots[m]] = ks[m]
    ev[slots[m]] = vs[m]
    np.testing.assert_array_equal(k2.reshape(-1, hkv, d), ek)
    np.testing.assert_array_equal(v2.reshape(-1, hkv, d), ev)
    # gather: reconstruct_kv equals numpy indexing; append then gather is the identity
    table = rng.permutation(nb)[:5].astype(np.int32)
    L = 70
    gk, gv = oracle.reconstruct_kv(k2, v2, table, L)
    np.testing.assert_array_equal(gk, np_gather(k2, table, L))
    np.testing.assert_array_equal(gv, np_gather(v2, table, L))
    pos = np.arange(L)
    rt_slots = table[pos // PAGE].astype(np.int64) * PAGE + pos % PAGE
    src = rng.integers(0, 60000, (L, hkv, d)).astype(dtype)
    oracle.append_slots(k2, v2, src, src, rt_slots)
    gk, _ = oracle.reconstruct_kv(k2, v2, table, L)
    np.testing.assert_array_equal(gk, src)


def test_scatter_prefill_matches_slot_math():
    rng = np.random.default_rng(2)
    nb, hkv, d = 32, 2, 16
    k, v = make_pools(rng, nb, hkv, d)
    table = rng.permutation(nb)[:6].astype(np.int32)
    start, n = 21, 50
    ks = rng.standard_normal((n, hkv, d)).astype(np.float32)
    vs = rng.standard_normal((n, hkv, d)).astype(np.float32)
    k2, v2 = k.copy(), v.copy()
    oracle.scatter_prefill(k2, v2, ks, vs, start, n, table)
    pos = np.arange(start, start + n)
    rows = table[pos // PAGE].astype(np.int64) * PAGE + pos % PAGE
    ek = k.reshape(-1, hkv, d).copy()
    ek[rows] = ks
    np.testing.assert_array_equal(k2.reshape(-1, hkv, d), ek)
    gk, gv = oracle.reconstruct_kv(k2, v2, table, start + n)
    np.testing.assert_array_equal(gv[start:], vs)


def test_scatter_prefill_batched_matches_per_entry():
    rng = np.random.default_rng(3)
    nb, hkv, d, mb = 64, 2, 16, 6
    k, v = make_pools(rng, nb, hkv, d)
    ntok = [17, 5, 33]
    starts = [0, 40, 3]
    perm = rng.permutation(nb).astype(np.int32)
    bt = perm[:3 * mb].reshape(3, mb)
    cum = np.concatenate([[0], np.cumsum(ntok)]).astype(np.int32)
    kv_off = (cum[:-1] * hkv * d).astype(np.int32)
    kf = rng.standard_normal((cum[-1], hkv, d)).astype(np.float32)
    vf = rng.standard_normal((cum[-1], hkv, d)).astype(np.float32)
    k1, v1 = k.copy(), v.copy()
    oracle.scatter_prefill_batched(k1, v1, kf, vf, kv_off, starts, cum, bt.reshape(-1), mb)
    k2, v2 = k.copy(), v.copy()
    for e in range(3):
        oracle.scatter_prefill(k2, v2, kf[cum[e]:cum[e + 1]], vf[cum[e]:cum[e + 1]], starts[e],
                               ntok[e], bt[e])
    np.testing.assert_array_equal(k1, k2)
    np.testing.assert_array_equal(v1, v2)


# ---------------------------------------------------------------------------
# decode attention
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("hq,hkv,d", [(14, 2, 64), (8, 8, 32), (4, 1, 128), (32, 8, 128)])
def test_decode_matches_numpy(hq, hkv, d):
    rng = np.random.default_rng(hq * 100 + d)
    lens = [1, 15, 16, 17, 100, 333]
    nb = 64
    k, v = make_pools(rng, nb, hkv, d)
    bt = make_tables(rng, lens, nb, extra=1)
    q = rng.standard_normal((len(lens), hq, d)).astype(np.float32)
    o32 = oracle.paged_decode(q, k, v, bt, lens)
    o64 = oracle.paged_decode(q, k, v, bt, lens, f64=True)
    for b, L in enumerate(lens):
        ref = np_attend(q[b], np_gather(k, bt[b], L), np_gather(v, bt[b], L), 1 / math.sqrt(d))
        close(o64[b], ref, 1e-12, 1e-13)
        close(o32[b], ref, 1e-5, 1e-6)
    # the multi-threaded form computes the same values
    np.testing.assert_array_equal(oracle.paged_decode(q, k, v, bt, lens, nthreads=4), o32)


def test_decode_closed_forms():
    rng = np.random.default_rng(5)
    hq, hkv, d, nb = 4, 2, 32, 16
    k, v = make_pools(rng, nb, hkv, d)
    # sequence 1: all keys equal -> output is the mean of V
    k[5] = k[5, 0]
    k[6] = k[5, 0]
    bt = np.array([[3, -1], [5, 6], [7, -1]], np.int32)
    lens = [1, 32, 0]
    q = rng.standard_normal((3, hq, d)).astype(np.float32)
    out = oracle.paged_decode(q, k, v, bt, lens, f64=True)
    for h in range(hq):
        np.testing.assert_allclose(out[0, h], v[3, 0, h // 2], rtol=0, atol=1e-12)   # L=1 -> V[0]
        mean = np.concatenate([v[5, :, h // 2], v[6, :, h // 2]]).astype(np.float64).mean(0)
        np.testing.assert_allclose(out[1, h], mean, rtol=0, atol=1e-12)
    assert np.all(out[2] == 0)   # seq_len 0 -> zeros (src/kv_cache/paged_attention.cu:224-227)


def test_decode_convex_hull_and_outliers():
    rng = np.random.default_rng(6)
    hq, hkv, d, nb = 14, 2, 64, 80
    k, v = make_pools(rng, nb, hkv, d)
    k[rng.random(k.shape) < 0.01] *= 8   # config 3's outliers
    lens = [1024]
    bt = make_tables(rng, lens, nb)
    q = rng.standard_normal((1, hq, d)).astype(np.float32) * 3
    out = oracle.paged_decode(q, k, v, bt, lens)
    assert np.isfinite(out).all()
    vv = np_gather(v, bt[0], 1024)
    for h in range(hq):
        assert np.all(out[0, h] <= vv[:, h // 7].max(0) + 1e-6)
        assert np.all(out[0, h] >= vv[:, h // 7].min(0) - 1e-6)


def test_reference_ramp_known_answer():
    # tests/test_paged_attention.cu:69-130: pools and q filled with (i % 100 - 50)/100,
    # tables [0, 1] and [2], lengths 24 and 8, T=2, Hq=4, Hkv=2, D=64
    nb, hkv, d, hq = 64, 2, 64, 4
    ramp = ((np.arange(nb * PAGE * hkv * d) % 100) - 50) / 100.0
    pool = ramp.astype(np.float32).reshape(nb, PAGE, hkv, d)
    q = (((np.arange(2 * hq * d) % 100) - 50) / 100.0).astype(np.float32).reshape(2, hq, d)
    bt = np.full((2, 8), -1, np.int32)
    bt[0, :2] = [0, 1]
    bt[1, 0] = 2
    out = oracle.paged_decode(q, pool, pool, bt, [24, 8])
    for b, L in enumerate([24, 8]):
        kk = np_gather(pool, bt[b], L)
        ref = np_attend(q[b], kk, kk, 1 / 8.0)
        close(out[b], ref, 1e-5, 1e-6)


@pytest.mark.parametrize("S", [1, 2, 4, 16, 40])
def test_splitk_merge_equals_unsplit(S):
    rng = np.random.default_rng(7)
    hq, hkv, d, nb = 14, 2, 64, 256
    lens = [1, 16, 200, 1024, 1500]
    k, v = make_pools(rng, nb, hkv, d)
    bt = make_tables(rng, lens, nb)
    q = rng.standard_normal((len(lens), hq, d)).astype(np.float32)
    part = oracle.splitk_partials(q, k, v, bt, lens, S)
    # splits past a sequence's pages are identities (l = 0, m = -1e38) and are skipped
    nblk = (1 + PAGE - 1) // PAGE
    assert np.all(part[0, :, nblk:, d] == 0) if S > 1 else True
    out = oracle.splitk_merge(part)
    ref = oracle.paged_decode(q, k, v, bt, lens, f64=True)
    close(out, ref, 1e-5, 1e-6)


def test_splitk_merge_hand_built():
    # two live splits and one identity: merge must equal the softmax over the union
    d = 4
    s1 = np.array([0.3, -1.2])
    s2 = np.array([2.0])
    v1 = np.arange(8, dtype=np.float64).reshape(2, 4)
    v2 = np.array([[1.0, -1.0, 0.5, 2.0]])
    part = np.zeros((1, 1, 3, d + 2), np.float32)
    for s, (sc, vv) in enumerate([(s1, v1), (s2, v2)]):
        m = sc.max()
        e = np.exp(sc - m)
        part[0, 0, s, :d] = e @ vv
        part[0, 0, s, d] = e.sum()
        part[0, 0, s, d + 1] = m
    part[0, 0, 2, d + 1] = -1e38
    out = oracle.splitk_merge(part)
    allsc = np.concatenate([s1, s2])
    p = np.exp(allsc - allsc.max())
    ref = p @ np.concatenate([v1, v2]) / p.sum()
    close(out[0, 0], ref, 1e-6, 1e-7)


# ---------------------------------------------------------------------------
# prefill attention
# ---------------------------------------------------------------------------

def _causal_counts(P, total, hq):
    hist = total - P
    return [[hist + i + 1] * hq for i in range(P)]


@pytest.mark.parametrize("causal", [False, True])
def test_prefill_matches_numpy(causal):
    rng = np.random.default_rng(8)
    P, total, hq, hkv, d = 37, 90, 6, 2, 32
    q = rng.standard_normal((P, hq, d)).astype(np.float32)
    k = rng.standard_normal((total, hkv, d)).astype(np.float32)
    v = rng.standard_normal((total, hkv, d)).astype(np.float32)
    o32 = oracle.prefill_attention(q, k, v, causal)
    o64 = oracle.prefill_attention(q, k, v, causal, f64=True)
    counts = _causal_counts(P, total, hq) if causal else [None] * P
    for i in range(P):
        ref = np_attend(q[i], k, v, 1 / math.sqrt(d), counts[i])
        close(o64[i], ref, 1e-12, 1e-13)
        close(o32[i], ref, 1e-5, 1e-6)
    if causal:
        # the test-file causal form (att_len = total - (P-1-t)) equals the kernel's
        # (keys <= hist + t) when total = hist + P
        close(oracle.prefill_attention_test_causal(q, k, v), o32, 1e-6, 1e-7)


def test_prefill_brute_force_tiny():
    rng = np.random.default_rng(9)
    for P, total in [(1, 1), (2, 5), (4, 4), (3, 48)]:
        hq, hkv, d = 2, 1, 4
        q = rng.standard_normal((P, hq, d)).astype(np.float32)
        k = rng.standard_normal((total, hkv, d)).astype(np.float32)
        v = rng.standard_normal((total, hkv, d)).astype(np.float32)
        out = oracle.prefill_attention(q, k, v, True, f64=True)
        for i in range(P):
            for h in range(hq):
                lim = total - P + i + 1
                w = [math.exp(sum(float(q[i, h, e]) * float(k[j, 0, e]) for e in range(d)) / 2.0)
                     for j in range(lim)]
                for e in range(d):
                    ref = sum(w[j] * float(v[j, 0, e]) for j in range(lim)) / sum(w)
                    assert abs(out[i, h, e] - ref) < 1e-9


def test_paged_prefill_matches_numpy():
    rng = np.random.default_rng(10)
    hq, hkv, d, nb = 14, 2, 64, 128
    prefixes, chunks = [0, 40, 256, 17], [33, 16, 70, 1]
    totals = [p + c for p, c in zip(prefixes, chunks)]
    k, v = make_pools(rng, nb, hkv, d)
    bt = make_tables(rng, totals, nb)
    bt[3, :1] = bt[2, :1]   # a shared first page (prefix-cache hit)
    cu = np.concatenate([[0], np.cumsum(chunks)]).astype(np.int32)
    q = rng.standard_normal((cu[-1], hq, d)).astype(np.float32)
    for causal in (True, False):
        out = oracle.paged_prefill(q, cu, k, v, bt, totals, causal)
        o64 = oracle.paged_prefill(q, cu, k, v, bt, totals, causal, f64=True)
        for n in range(4):
            kk, vv = np_gather(k, bt[n], totals[n]), np_gather(v, bt[n], totals[n])
            for i in range(chunks[n]):
                cnt = [prefixes[n] + i + 1] * hq if causal else None
                ref = np_attend(q[cu[n] + i], kk, vv, 1 / 8.0, cnt)
                close(out[cu[n] + i], ref, 1e-5, 1e-6)
                close(o64[cu[n] + i], ref, 1e-12, 1e-13)


def test_first_prefill_batched_matches_numpy():
    rng = np.random.default_rng(11)
    hq, hkv, d = 4, 2, 16
    ntok = [5, 12, 1]
    starts = [0, 7, 30]
    cum = np.concatenate([[0], np.cumsum(ntok)]).astype(np.int32)
    offsets = (cum[:-1] * hq * d).astype(np.int32)
    kv_off = (cum[:-1] * hkv * d).astype(np.int32)
    q = rng.standard_normal((cum[-1], hq, d)).astype(np.float32)
    k = rng.standard_normal((cum[-1], hkv, d)).astype(np.float32)
    v = rng.standard_normal((cum[-1], hkv, d)).astype(np.float32)
    out = oracle.first_prefill_batched(q, k, v, hq, hkv, d, offsets, kv_off, ntok, cum, starts,
                                       0.3, cum[-1])
    for e in range(3):
        for r in range(ntok[e]):
            ref = np_attend(q[cum[e] + r], k[cum[e]:cum[e + 1]], v[cum[e]:cum[e + 1]], 0.3,
                            [r + 1] * hq)
            close(out[cum[e] + r], ref, 1e-5, 1e-6)


# ---------------------------------------------------------------------------
# step metadata and fused RoPE + append
# ---------------------------------------------------------------------------

def py_slots(table, cu, start, bs=PAGE):
    """Pure-Python walk of the reference's host loops (engine_server.cpp:731-787)."""
    out = []
    for e in range(len(start)):
        for i in range(cu[e + 1] - cu[e]):
            pos = start[e] + i
            blk = pos // bs
            if pos < 0 or blk >= table.shape[1] or table[e, blk] < 0:
                out.append(-1)
            else:
                out.append(int(table[e, blk]) * bs + pos % bs)
    return np.array(out, dtype=np.int64)


def test_build_slots_matches_python_walk():
    rng = np.random.default_rng(3)
    n, mb = 6, 5
    table = rng.permutation(200)[: n * mb].reshape(n, mb).astype(np.int32)
    table[1, 3:] = -1
    table[4, 0] = -1
    counts = np.array([1, 17, 0, 40, 3, 9])
    cu = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    start = np.array([0, 30, 5, 50, 0, 70], dtype=np.int32)   # seq 5 runs past the table
    got = oracle.build_slots(table, cu, start, int(cu[-1]))
    assert np.array_equal(got, py_slots(table, cu, start))
    assert (got == -1).any() and (got >= 0).any()
    # decode form: one token per sequence at its current length
    lens = np.array([0, 15, 16, 63, 64, 79], dtype=np.int32)
    dec = oracle.build_slots(table, np.arange(n + 1, dtype=np.int32), lens, n)
    for b in range(n):
        want = table[b, lens[b] // PAGE] * PAGE + lens[b] % PAGE if lens[b] // PAGE < mb else -1
        want = -1 if lens[b] // PAGE < mb and table[b, lens[b] // PAGE] < 0 else want
        assert dec[b] == want


def np_rope_f32(x, cos, sin):
    """float32 Neox rotation with separately rounded products and sums (numpy float32 ops)."""
    half = cos.shape[1]
    x = x.astype(np.float32).copy()
    x1, x2 = x[..., :half].copy(), x[..., half:2 * half].copy()
    c, s = cos[:, None, :], sin[:, None, :]
    x[..., :half] = (x1 * c) - (x2 * s)
    x[..., half:2 * half] = (x2 * c) + (x1 * s)
    return x


def _to_bits(x32, dtype):
    if dtype == 1:
        return x32.astype(np.float16).view(np.uint16)
    return torch.from_numpy(x32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _from_bits(b, dtype):
    if dtype == 1:
        return b.view(np.float16).astype(np.float32)
    return torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).float().numpy()


@pytest.mark.parametrize("dtype", [0, 1, 2])
@pytest.mark.parametrize("rot", [64, 32])
def test_rope_append_matches_numpy(dtype, rot):
    rng = np.random.default_rng(10 + dtype)
    T, hq, hkv, d, nb = 7, 6, 2, 64, 12
    q32 = rng.standard_normal((T, hq, d)).astype(np.float32)
    k32 = rng.standard_normal((T, hkv, d)).astype(np.float32)
    v32 = rng.standard_normal((T, hkv, d)).astype(np.float32)
    pos = rng.integers(0, 5000, T)
    inv = 1.0 / (10000.0 ** (np.arange(rot // 2) * 2.0 / rot))
    ang = (pos[:, None] * inv[None, :]).astype(np.float32)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    slots = np.array([3, -1, 17, 40, 0, 191, 100], dtype=np.int64)
    if dtype == 0:
        q, k, v = q32.copy(), k32.copy(), v32.copy()
        kp = np.zeros((nb, PAGE, hkv, d), np.float32)
    else:
        q, k, v = _to_bits(q32, dtype), _to_bits(k32, dtype), _to_bits(v32, dtype)
        kp = np.zeros((nb, PAGE, hkv, d), np.uint16)
    vp = kp.copy()
    qin, kin = q.copy(), k.copy()
    oracle.rope_append(q, k, v, kp, vp, slots, cos, sin, dtype)
    if dtype == 0:
        want_q, want_k = np_rope_f32(qin, cos, sin), np_rope_f32(kin, cos, sin)
    else:
        want_q = _to_bits(np_rope_f32(_from_bits(qin, dtype), cos, sin), dtype)
        want_k = _to_bits(np_rope_f32(_from_bits(kin, dtype), cos, sin), dtype)
    assert np.array_equal(q.view(np.uint32 if dtype == 0 else np.uint16),
                          want_q.view(np.uint32 if dtype == 0 else np.uint16))
    assert np.array_equal(k.view(np.uint32 if dtype == 0 else np.uint16),
                          want_k.view(np.uint32 if dtype == 0 else np.uint16))
    if rot < d:   # dims past rotary_dim untouched
        assert np.array_equal(q[..., rot:], qin[..., rot:])
    kr, vr = kp.reshape(-1, hkv, d), vp.reshape(-1, hkv, d)
    for t, s in enumerate(slots):
        if s < 0:
            continue
        assert np.array_equal(kr[s], k[t]) and np.array_equal(vr[s], v[t])
    written = set(int(s) for s in slots if s >= 0)
    untouched = [r for r in range(nb * PAGE) if r not in written]
    assert not kr[untouched].any() and not vr[untouched].any()


def test_rope_reference_known_answer_and_invariants():
    # tests/test_ops.cu:51-61: T=1, H=4, D=64, q = 0.1, cos = sin = 0.5 -> x1' = 0, x2' = 0.1
    T, H, D = 1, 4, 64
    q = np.full((T, H, D), 0.1, np.float32)
    k = np.zeros((T, 1, D), np.float32)
    cos = np.full((T, D // 2), 0.5, np.float32)
    kp = np.zeros((1, PAGE, 1, D), np.float32)
    oracle.rope_append(q, k, k.copy(), kp, kp.copy(), np.array([-1]), cos, cos.copy(), 0)
    assert np.all(np.abs(q[..., : D // 2]) < 0.01) and np.all(np.abs(q[..., D // 2:] - 0.1) < 0.01)
    # angle 0 is the identity; true angles keep each pair's norm
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 2, 128)).astype(np.float32)
    y = x.copy()
    one, zero = np.ones((3, 64), np.float32), np.zeros((3, 64), np.float32)
    kp = np.zeros((1, PAGE, 2, 128), np.float32)
    oracle.rope_append(None, y, y.copy(), kp, kp.copy(), np.full(3, -1), one, zero, 0)
    assert np.array_equal(y, x)
    ang = rng.uniform(-50, 50, (3, 64)).astype(np.float32)
    z = x.copy()
    oracle.rope_append(None, z, z.copy(), kp, kp.copy(), np.full(3, -1), np.cos(ang).astype(np.float32),
                       np.sin(ang).astype(np.float32), 0)
    n0 = np.hypot(x[..., :64], x[..., 64:])
    n1 = np.hypot(z[..., :64], z[..., 64:])
    assert np.allclose(n0, n1, rtol=1e-5, atol=1e-6)
