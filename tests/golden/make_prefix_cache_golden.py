"""Writes the prefix-cache golden traces under tests/golden/prefix_cache/.

Each trace is the stdout of oracle/prefix_cache_trace.cpp built against the
reference's own sources (oracle/_ref/trace_ref: src/kv_cache/hash_prefix_cache.cpp
and radix_prefix_cache.cpp of wjb554/lightllm, compiled by `make -C oracle ref`
with AddressSanitizer).  The reference radix cache reads freed trie nodes after
some prune/merge sequences (RadixPrefixCache::remove through stale block->node
entries, src/kv_cache/radix_prefix_cache.cpp:373-377); the sanitizer stops the
program there, so such a trace holds the operations completed before that
point and the test compares that prefix.

Run in a tree where the reference is present:
    make -C oracle ref && python tests/golden/make_prefix_cache_golden.py
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
TRACE_REF = os.path.join(ROOT, "oracle", "_ref", "trace_ref")
OUT = os.path.join(HERE, "prefix_cache")

# (policy, block_size, seed, n_ops, pool_blocks)
CASES = [
    ("hash", 16, 1, 400, 64),
    ("hash", 16, 2, 400, 24),
    ("hash", 4, 3, 400, 32),
    ("hash", 1, 4, 300, 16),
    ("radix", 16, 1, 400, 64),
    ("radix", 16, 2, 400, 24),
    ("radix", 16, 5, 400, 48),
    ("radix", 4, 3, 400, 32),
    ("radix", 4, 6, 400, 96),
    ("radix", 1, 4, 300, 16),
    ("radix", 1, 7, 300, 64),
]


def case_name(policy, bs, seed, n_ops, pool):
    return f"{policy}_bs{bs}_seed{seed}_ops{n_ops}_pool{pool}.trace"


def main():
    if not os.path.exists(TRACE_REF):
        sys.exit(f"{TRACE_REF} missing: run make -C oracle ref (needs the reference tree)")
    os.makedirs(OUT, exist_ok=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0")
    for c in CASES:
        r = subprocess.run([TRACE_REF, c[0], str(c[1]), str(c[2]), str(c[3]), str(c[4])],
                           capture_output=True, text=True, env=env)
        lines = [l for l in r.stdout.splitlines() if l]
        with open(os.path.join(OUT, case_name(*c)), "w") as f:
            f.write("\n".join(lines) + "\n")
        status = "complete" if r.returncode == 0 else f"stopped by the sanitizer (exit {r.returncode})"
        print(f"{case_name(*c)}: {len(lines) - 1} ops, {status}")


if __name__ == "__main__":
    main()
