"""Prefix caches (Hash / Radix) and the block allocator, on the CPU.

* Golden traces: oracle/prefix_cache_trace.cpp drives the PrefixCache API through
  an engine-like seeded op sequence; the committed traces were produced by the
  reference's own sources (tests/golden/make_prefix_cache_golden.py).  This
  build's driver (oracle/_bin/trace_ours, over lightllm_amd/csrc/prefix_cache_*.cpp)
  must print the same lines.
* Where the reference tree is present, the reference's own test programs
  (tests/test_prefix_cache.cpp, tests/test_radix_engine.cpp) are compiled against
  this build's headers and sources (oracle/_ref/*_ours) and must pass, and
  fresh seeds are diffed live against the reference build.
* Sanitizers: this build's host C++ (allocator, caches, C handle API, host Tensor)
  runs under AddressSanitizer + UndefinedBehaviorSanitizer, with leak checks: the
  trace driver (oracle/_bin/trace_ours_san), the reference's test programs built on
  this build's sources (oracle/_ref/*_ours_san), and a seeded serving-workload
  driver (tests/cpp/test_host_san.cpp).
* The allocator handle (C ABI, metadata-only storage) follows the reference's
  allocator checks (tests/test_paged_attention_v2.cu:610-637) and the FIFO /
  hash-probe / eviction rules of src/kv_cache/block_allocator.cpp:33-147.
"""
import glob
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden", "prefix_cache")
TRACE_OURS = os.path.join(ROOT, "oracle", "_bin", "trace_ours")
TRACE_SAN = os.path.join(ROOT, "oracle", "_bin", "trace_ours_san")
HOST_SAN = os.path.join(ROOT, "tests", "cpp", "_bin", "test_host_san")
REF_DIR = os.path.join(ROOT, "oracle", "_ref")


def _trace(exe, policy, bs, seed, n_ops, pool, leaks=False):
    env = dict(os.environ, ASAN_OPTIONS=f"detect_leaks={int(leaks)}")
    r = subprocess.run([exe, policy, str(bs), str(seed), str(n_ops), str(pool)],
                       capture_output=True, text=True, env=env, timeout=120)
    return r.returncode, [l for l in r.stdout.splitlines() if l]


def _parse(name):
    base = os.path.basename(name)[:-len(".trace")]
    policy, bs, seed, ops, pool = base.split("_")
    return policy, int(bs[2:]), int(seed[4:]), int(ops[3:]), int(pool[4:])


GOLDEN_FILES = sorted(glob.glob(os.path.join(GOLDEN, "*.trace")))


def test_golden_traces_present():
    assert len(GOLDEN_FILES) >= 8
    assert os.path.exists(TRACE_OURS), "run make -C oracle all"


@pytest.mark.parametrize("path", GOLDEN_FILES, ids=[os.path.basename(p) for p in GOLDEN_FILES])
def test_trace_matches_reference_golden(path):
    policy, bs, seed, ops, pool = _parse(path)
    with open(path) as f:
        golden = [l for l in f.read().splitlines() if l]
    rc, ours = _trace(TRACE_OURS, policy, bs, seed, ops, pool)
    assert rc == 0
    # our build runs every op (no use-after-free); the golden prefix must agree line by line
    assert len(ours) == ops + 1
    for i, (g, o) in enumerate(zip(golden, ours)):
        assert g == o, f"line {i}: reference {g!r} vs ours {o!r}"


@pytest.mark.parametrize("path", GOLDEN_FILES[:4], ids=[os.path.basename(p) for p in GOLDEN_FILES[:4]])
def test_trace_under_sanitizers(path):
    """The same golden traces from this build's caches built with ASan + UBSan (and leak
    checks): no memory error, no undefined behaviour, the same lines."""
    assert os.path.exists(TRACE_SAN), "run make -C oracle all"
    policy, bs, seed, ops, pool = _parse(path)
    with open(path) as f:
        golden = [l for l in f.read().splitlines() if l]
    rc, ours = _trace(TRACE_SAN, policy, bs, seed, ops, pool, leaks=True)
    assert rc == 0
    assert ours[:len(golden)] == golden[:len(ours)] and len(ours) == ops + 1


def _build_host_san():
    if not os.path.exists(HOST_SAN):
        subprocess.run(["make", "-C", os.path.join(ROOT, "tests", "cpp"), "san"], check=True,
                       capture_output=True, timeout=600)


@pytest.mark.parametrize("seed", [1, 7, 42])
def test_host_code_under_sanitizers(seed):
    """Seeded serving workload over BlockAllocator (host and metadata-only pools, both
    policies), the C handle API and the host Tensor, built with ASan + UBSan
    (tests/cpp/test_host_san.cpp): every check passes and the sanitizers report nothing
    (they abort on the first finding, leaks included)."""
    _build_host_san()
    r = subprocess.run([HOST_SAN, str(seed)], capture_output=True, text=True, timeout=300,
                       env=dict(os.environ, ASAN_OPTIONS="detect_leaks=1",
                                UBSAN_OPTIONS="print_stacktrace=1"))
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert " 0 failed" in r.stdout, r.stdout[-2000:]


def test_traces_exercise_every_op_kind():
    kinds = {"new": 0, "extend": 0, "release": 0, "probe": 0, "evict=": 0}
    hits = 0
    for p in GOLDEN_FILES:
        with open(p) as f:
            for line in f:
                for k in kinds:
                    if k in line:
                        kinds[k] += 1
                if " matched=" in line and " matched=0 " not in line:
                    hits += 1
    assert all(v > 0 for v in kinds.values()), kinds
    assert hits > 50


_have_ref = os.path.exists(os.path.join(REF_DIR, "trace_ref"))


@pytest.mark.skipif(not _have_ref, reason="reference tree not built here (oracle/_ref)")
@pytest.mark.parametrize("policy", ["hash", "radix"])
@pytest.mark.parametrize("seed", [11, 12, 13, 14])
def test_trace_live_vs_reference(policy, seed):
    for bs, pool in ((16, 40), (2, 24)):
        rc_ref, ref = _trace(os.path.join(REF_DIR, "trace_ref"), policy, bs, seed, 500, pool)
        rc, ours = _trace(TRACE_OURS, policy, bs, seed, 500, pool)
        assert rc == 0 and len(ours) == 501
        if rc_ref == 0:
            assert ref == ours
        else:   # reference stopped at a use-after-free: compare what it completed
            assert ref == ours[:len(ref)]


@pytest.mark.skipif(not os.path.exists(os.path.join(REF_DIR, "test_prefix_cache_ours")),
                    reason="reference tests not built here (oracle/_ref)")
@pytest.mark.parametrize("prog", ["test_prefix_cache_ours", "test_radix_engine_ours",
                                  "test_prefix_cache_ours_san", "test_radix_engine_ours_san"])
def test_reference_cache_tests_pass_on_this_build(prog):
    """The reference's own cache test programs on this build's sources (the _san builds under
    ASan + UBSan with leak checks)."""
    r = subprocess.run([os.path.join(REF_DIR, prog)], capture_output=True, text=True, timeout=300,
                       env=dict(os.environ, ASAN_OPTIONS="detect_leaks=1"))
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "FAIL" not in r.stdout.replace("0 failed", "")


# ---------------------------------------------------------------------------
# allocator handle through the C ABI, no device storage
# ---------------------------------------------------------------------------

import torch  # noqa: E402
from lightllm_amd import kv_cache as kc  # noqa: E402


def _alloc(n=64, policy=kc.POLICY_HASH, bs=16):
    return kc.BlockAllocator(n, bs, 2, 64, policy=policy, device=None)


def test_allocator_regression_gate():
    # tests/test_paged_attention_v2.cu:610-637
    a = _alloc()
    assert a.num_blocks == 64 and a.num_free() == 64
    b0, b1 = a.allocate(0x123), a.allocate(0x456)
    assert b0 >= 0 and b1 >= 0 and a.num_free() == 62
    a.release(b0)
    a.release(b1)
    assert a.num_free() == 64
    blocks = [a.allocate() for _ in range(64)]
    assert all(b >= 0 for b in blocks) and a.num_free() == 0
    assert a.allocate() == -1
    for b in blocks:
        a.release(b)
    assert a.num_free() == 64


def test_allocator_fifo_order():
    # free list is a deque: pop front, push back (block_allocator.cpp:81-93,138-147)
    a = _alloc(8)
    first = [a.allocate() for _ in range(3)]
    assert first == [0, 1, 2]
    a.release(1)
    assert [a.allocate() for _ in range(5)] == [3, 4, 5, 6, 7]
    assert a.allocate() == 1


def test_allocator_refcount_and_hash_probe():
    a = _alloc(8)
    toks = list(range(32))
    n_new, blocks = a.allocate_tokens(toks, 0)   # allocates and registers both blocks
    assert n_new == 2 and len(blocks) == 2
    assert a.token_hash(blocks[0]) == kc.hash_tokens(toks[:16])
    matched, ids = a.find_cached_prefix(toks + [99], 0)
    assert matched == 32 and ids == blocks
    # Hash policy: allocate(hash) of a cached block returns it with ref + 1
    h = kc.hash_tokens(toks[:16])
    assert a.find_by_hash(h) == blocks[0]
    assert a.allocate(h) == blocks[0]
    assert a.ref_count(blocks[0]) == 2
    a.release(blocks[0])
    a.release(blocks[0])
    assert a.ref_count(blocks[0]) == 0
    # at ref 0 the block returns to the free list (block_allocator.cpp:138-147) while the
    # hash cache only drops its entry's ref to 0 and keeps it as evictable
    # (hash_prefix_cache.cpp:129-145): the reference's stale entry is kept as is
    assert a.num_free() == 7
    assert a.find_by_hash(h) == blocks[0]
    assert a.evict_lru() in blocks


def test_allocator_evicts_lru_on_exhaustion():
    a = _alloc(4)
    ids = []
    for i in range(4):
        toks = [1000 * i + t for t in range(16)]
        n_new, b = a.allocate_tokens(toks, 0)
        assert n_new == 1
        ids += b
    assert a.num_free() == 0
    for b in ids:
        a.release(b)   # ref 0: back on the free list, cache entry kept as evictable
    assert a.num_free() == 4
    assert a.prefix_cache_size() == 4
    # evictable entries leave in LRU order (oldest access first, hash_prefix_cache.cpp:151-202)
    assert a.evict_lru() == ids[0]
    assert a.prefix_cache_size() == 3
    a.reset()
    assert a.num_free() == 4 and a.prefix_cache_size() == 0


def test_blocks_for_budget():
    """Pool sizing for a byte budget in the pool's element type (K and V pages)."""
    f = kc.BlockAllocator.blocks_for_budget
    # Llama-3-8B heads (8 x 128) in fp16: 64 KiB per page, 4.39 million pages in 288 GB
    assert f(288_000_000_000, 16, 8, 128, torch.float16) == 288_000_000_000 // (16 * 8 * 128 * 2 * 2)
    assert f(1 << 30, 16, 2, 64, torch.float32) == 2 * f(1 << 30, 16, 2, 128, torch.float32)
    assert f(1 << 30, 16, 2, 64, torch.bfloat16) == 2 * f(1 << 30, 16, 2, 64, torch.float32)
    assert f(0, 16, 2, 64, torch.float16) == 0
    assert f(1 << 62, 1, 1, 1, torch.float16) == 2**31 - 1   # capped
    with pytest.raises(ValueError):
        f(1 << 30, 0, 2, 64, torch.float16)


def test_hash_tokens_is_fnv1a_64():
    # FNV-1a 64 (offset basis 14695981039346656037, prime 1099511628211) over each token
    # taken as one uint32 value (hash_prefix_cache.cpp:23-30); published test vector:
    # FNV-1a 64 of the single octet 0x61 ("a") is 0xaf63dc4c8601ec8c.
    assert kc.hash_tokens([]) == 0xCBF29CE484222325
    assert kc.hash_tokens([0x61]) == 0xAF63DC4C8601EC8C
    # a negative token hashes as its uint32 image
    h = 0xCBF29CE484222325
    for t in (-1, 5):
        h ^= t & 0xFFFFFFFF
        h = (h * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    assert kc.hash_tokens([-1, 5]) == h


def test_cxx_api_cpu_program():
    exe = os.path.join(ROOT, "tests", "cpp", "_bin", "test_cxx_api")
    if not os.path.exists(exe):
        pytest.skip("tests/cpp not built")
    r = subprocess.run([exe, "cpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failed" in r.stdout
