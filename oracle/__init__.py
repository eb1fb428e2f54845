"""CPU oracle of the paged KV-cache hot path -- TEST INFRASTRUCTURE ONLY.

ctypes + numpy wrapper over oracle/libcpu_ref.so, the C restatement of the
reference's CPU attention / gather / append code (see cpu_ref.c for the
file:line each function follows).  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg import this module, and only as the checker or
the CPU baseline; the product library never calls it.

Pinning (what each function is checked against) is listed in oracle/cpu_ref.h;
no function is left unpinned.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_double, c_float, c_int, c_int64, c_size_t, c_uint, c_uint32, c_void_p

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libcpu_ref.so")
REF_DIR = os.path.join(_HERE, "_ref")
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} missing: run make -C oracle")
        _lib = ctypes.CDLL(LIB_PATH)
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


# ---------------------------------------------------------------------------
# generators and rounding
# ---------------------------------------------------------------------------

def fill_random(n: int, seed: int) -> np.ndarray:
    """tests/test_paged_attention_v2.cu:58-64 LCG, values in [-1, 1)."""
    out = np.empty(n, dtype=np.float32)
    lib().llo_fill_random(_p(out), c_size_t(n), c_uint(seed))
    return out


def rng_randf(n: int, state: int) -> tuple[np.ndarray, int]:
    """tests/test_attention_fp16.cpp:31-38 LCG (rand_vec form, [-1, 1))."""
    out = np.empty(n, dtype=np.float32)
    st = c_uint32(state)
    lib().llo_rng_randf_fill(_p(out), c_size_t(n), ctypes.byref(st))
    return out, st.value


def f32_to_f16_bits(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().llo_f32_to_f16_array(_p(x), _p(out), c_size_t(x.size))
    return out


def f16_bits_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().llo_f16_to_f32_array(_p(b), _p(out), c_size_t(b.size))
    return out


def f32_to_bf16_bits(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().llo_f32_to_bf16_array(_p(x), _p(out), c_size_t(x.size))
    return out


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().llo_bf16_to_f32_array(_p(b), _p(out), c_size_t(b.size))
    return out


# ---------------------------------------------------------------------------
# copies (work on raw bytes of any dtype)
# ---------------------------------------------------------------------------

def append_slots(k_pool: np.ndarray, v_pool: np.ndarray, k_src, v_src, slots) -> None:
    """In place: row i of k_src/v_src -> pool row slots[i] (negative skipped)."""
    nb, bs, hkv, d = k_pool.shape
    k_src = np.ascontiguousarray(k_src, dtype=k_pool.dtype)
    v_src = np.ascontiguousarray(v_src, dtype=k_pool.dtype)
    slots = np.ascontiguousarray(slots, dtype=np.int64)
    lib().llo_append_slots(_p(k_pool), _p(v_pool), _p(k_src), _p(v_src), _p(slots),
                           c_int64(slots.size), hkv, d, k_pool.itemsize)


def build_slots(block_table, cu, start_pos, num_tokens: int, block_size: int = 16) -> np.ndarray:
    """Slot mapping of a step (-1 outside the table)."""
    bt = _i32(block_table)
    cu, start = _i32(cu), _i32(start_pos)
    out = np.full(num_tokens, -7, dtype=np.int64)
    lib().llo_build_slots(_p(out), _p(bt), bt.shape[1], _p(cu), _p(start), start.size, num_tokens,
                          block_size)
    return out


def rope_append(q, k, v, k_pool, v_pool, slots, cos, sin, dtype: int) -> None:
    """In place: RoPE on q (or None) and k, then k / v rows appended at slots.  Arrays hold fp32
    values (dtype 0) or fp16 / bf16 bit patterns as uint16 (dtype 1 / 2), contiguous."""
    want = np.float32 if dtype == 0 else np.uint16
    for a in (q, k, v, k_pool, v_pool):
        if a is not None:
            assert a.dtype == want and a.flags.c_contiguous
    cos, sin = _f32(cos), _f32(sin)
    slots = np.ascontiguousarray(slots, dtype=np.int64)
    t, hkv, d = k.shape
    hq = q.shape[1] if q is not None else 0
    lib().llo_rope_append(_p(q) if q is not None else None, _p(k), _p(v), _p(k_pool), _p(v_pool),
                          _p(slots), _p(cos), _p(sin), t, hq, hkv, d, 2 * cos.shape[1], dtype)


def scatter_prefill(k_pool, v_pool, k_src, v_src, start_pos: int, n_tokens: int, table) -> None:
    nb, bs, hkv, d = k_pool.shape
    k_src = np.ascontiguousarray(k_src, dtype=k_pool.dtype)
    v_src = np.ascontiguousarray(v_src, dtype=k_pool.dtype)
    table = _i32(table)
    lib().llo_scatter_prefill(_p(k_pool), _p(v_pool), _p(k_src), _p(v_src), start_pos, n_tokens,
                              _p(table), bs, hkv, d, k_pool.itemsize)


def scatter_prefill_batched(k_pool, v_pool, k_flat, v_flat, kv_offsets, start_poss, token_cumsum,
                            flat_bt, max_blocks: int) -> None:
    nb, bs, hkv, d = k_pool.shape
    k_flat = np.ascontiguousarray(k_flat, dtype=k_pool.dtype)
    v_flat = np.ascontiguousarray(v_flat, dtype=k_pool.dtype)
    kv_offsets, start_poss, token_cumsum, flat_bt = map(_i32, (kv_offsets, start_poss,
                                                               token_cumsum, flat_bt))
    lib().llo_scatter_prefill_batched(_p(k_pool), _p(v_pool), _p(k_flat), _p(v_flat), hkv, d,
                                      _p(kv_offsets), _p(start_poss), _p(token_cumsum),
                                      _p(flat_bt), max_blocks, kv_offsets.size, bs,
                                      k_pool.itemsize)


def reconstruct_kv(k_pool, v_pool, table, seq_len: int):
    """Contiguous [seq_len, Hkv, D] of one sequence (same dtype as the pool)."""
    nb, bs, hkv, d = k_pool.shape
    table = _i32(table)
    k = np.empty((seq_len, hkv, d), dtype=k_pool.dtype)
    v = np.empty_like(k)
    lib().llo_reconstruct_kv(_p(k), _p(v), _p(k_pool), _p(v_pool), _p(table), seq_len, bs, hkv, d,
                             k_pool.itemsize)
    return k, v


# ---------------------------------------------------------------------------
# attention (float32 inputs; fp16/bf16 pools are widened exactly by the caller)
# ---------------------------------------------------------------------------

def cpu_attention(q, k, v, f64: bool = False) -> np.ndarray:
    """q [T, Hq, D] against contiguous k/v [L, Hkv, D] (all T rows see all L keys)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    t, hq, d = q.shape
    seq_len, hkv = k.shape[0], k.shape[1]
    if f64:
        out = np.zeros((t, hq, d), dtype=np.float64)
        lib().llo_cpu_attention_f64(_p(q), t, hq, d, _p(k), seq_len, hkv, _p(v), _p(out))
    else:
        out = np.zeros((t, hq, d), dtype=np.float32)
        lib().llo_cpu_attention(_p(q), t, hq, d, _p(k), seq_len, hkv, _p(v), _p(out))
    return out


def paged_decode(q, k_pool, v_pool, block_table, seq_lens, f64: bool = False,
                 nthreads: int = 1) -> np.ndarray:
    """Batched decode: reconstruct_kv + cpu_attention per sequence.  q [B, Hq, D]."""
    q, k_pool, v_pool = _f32(q), _f32(k_pool), _f32(v_pool)
    block_table, seq_lens = _i32(block_table), _i32(seq_lens)
    b, hq, d = q.shape
    nb, bs, hkv, _ = k_pool.shape
    mb = block_table.shape[1]
    if f64:
        out = np.zeros((b, hq, d), dtype=np.float64)
        lib().llo_paged_decode_f64(_p(q), _p(k_pool), _p(v_pool), _p(block_table), _p(seq_lens), b,
                                   hq, hkv, d, bs, mb, _p(out), nthreads)
    else:
        out = np.zeros((b, hq, d), dtype=np.float32)
        lib().llo_paged_decode(_p(q), _p(k_pool), _p(v_pool), _p(block_table), _p(seq_lens), b, hq,
                               hkv, d, bs, mb, _p(out), nthreads)
    return out


def splitk_partials(q, k_pool, v_pool, block_table, seq_lens, num_splits: int) -> np.ndarray:
    q, k_pool, v_pool = _f32(q), _f32(k_pool), _f32(v_pool)
    block_table, seq_lens = _i32(block_table), _i32(seq_lens)
    b, hq, d = q.shape
    nb, bs, hkv, _ = k_pool.shape
    part = np.zeros((b, hq, num_splits, d + 2), dtype=np.float32)
    lib().llo_splitk_partials(_p(q), _p(k_pool), _p(v_pool), _p(block_table), _p(seq_lens), b, hq,
                              hkv, d, bs, block_table.shape[1], num_splits, _p(part))
    return part


def splitk_merge(partial) -> np.ndarray:
    partial = _f32(partial)
    b, hq, s, d2 = partial.shape
    out = np.zeros((b, hq, d2 - 2), dtype=np.float32)
    lib().llo_splitk_merge(_p(partial), b, hq, d2 - 2, s, _p(out))
    return out


def prefill_attention(q, k, v, causal: bool, f64: bool = False) -> np.ndarray:
    """q [P, Hq, D] against contiguous k/v [total, Hkv, D]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    p, hq, d = q.shape
    total, hkv = k.shape[0], k.shape[1]
    if f64:
        out = np.zeros((p, hq, d), dtype=np.float64)
        lib().llo_prefill_attention_f64(_p(q), p, hq, d, _p(k), total, hkv, _p(v), int(causal), _p(out))
    else:
        out = np.zeros((p, hq, d), dtype=np.float32)
        lib().llo_prefill_attention(_p(q), p, hq, d, _p(k), total, hkv, _p(v), int(causal), _p(out))
    return out


def prefill_attention_test_causal(q, k, v) -> np.ndarray:
    """tests/test_paged_prefill.cu:164-210 form (att_len = seq_len - (P-1-t))."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    p, hq, d = q.shape
    out = np.zeros((p, hq, d), dtype=np.float32)
    lib().llo_prefill_attention_test_causal(_p(q), p, hq, d, _p(k), k.shape[0], k.shape[1], _p(v),
                                            _p(out))
    return out


def paged_prefill(q, cu_q, k_pool, v_pool, block_table, seq_lens, causal: bool,
                  f64: bool = False, nthreads: int = 1) -> np.ndarray:
    q, k_pool, v_pool = _f32(q), _f32(k_pool), _f32(v_pool)
    cu_q, block_table, seq_lens = _i32(cu_q), _i32(block_table), _i32(seq_lens)
    tq, hq, d = q.shape
    nb, bs, hkv, _ = k_pool.shape
    n = seq_lens.size
    if f64:
        out = np.zeros((tq, hq, d), dtype=np.float64)
        lib().llo_paged_prefill_f64(_p(q), _p(cu_q), _p(k_pool), _p(v_pool), _p(block_table),
                                    _p(seq_lens), n, hq, hkv, d, bs, block_table.shape[1],
                                    int(causal), _p(out), nthreads)
    else:
        out = np.zeros((tq, hq, d), dtype=np.float32)
        lib().llo_paged_prefill(_p(q), _p(cu_q), _p(k_pool), _p(v_pool), _p(block_table),
                                _p(seq_lens), n, hq, hkv, d, bs, block_table.shape[1], int(causal),
                                _p(out), nthreads)
    return out


def first_prefill_batched(q, k, v, hq, hkv, d, offsets, kv_offsets, num_tokens, token_cumsum,
                          start_poss, scale: float, out_rows: int) -> np.ndarray:
    q, k, v = _f32(q), _f32(k), _f32(v)
    offsets, kv_offsets, num_tokens, token_cumsum, start_poss = map(
        _i32, (offsets, kv_offsets, num_tokens, token_cumsum, start_poss))
    out = np.zeros(out_rows * hq * d, dtype=np.float32)
    n = offsets.size
    lib().llo_first_prefill_batched(_p(out), _p(q), _p(k), _p(v), hq, hkv, d, _p(offsets),
                                    _p(kv_offsets), _p(num_tokens), _p(token_cumsum),
                                    _p(start_poss), n, int(token_cumsum[-1]), c_float(scale))
    return out.reshape(out_rows, hq, d)


def fnv1a_tokens(tokens) -> int:
    t = _i32(tokens)
    lib().llo_fnv1a_tokens.restype = ctypes.c_uint64
    return int(lib().llo_fnv1a_tokens(_p(t), t.size))


def omp_max_threads() -> int:
    return int(lib().llo_omp_max_threads())
