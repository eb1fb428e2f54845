"""ctypes binding of liblightllm_kv.so (the C ABI declared in include/lightllm_kv.h).

The library is built in-tree by ``__graft_entry__.build()`` (or ``make -C
lightllm_amd/csrc``).  There is no fallback: if the library is missing or
fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_int64, c_size_t, c_uint64, c_void_p, c_char_p

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblightllm_kv.so")

DTYPE_F32, DTYPE_F16, DTYPE_BF16, DTYPE_I32 = 0, 1, 2, 3
STATUS = {0: "ok", 1: "invalid argument", 2: "unsupported", 3: "workspace too small",
          4: "HIP error", 5: "pool exhausted"}


class LLKVError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{message} (status {status}: {STATUS.get(status, '?')})")
        self.status = status


_lib = None

# name -> (restype, argtypes)
_SIGS = {
    "llkv_last_error": (c_char_p, []),
    "llkv_status_string": (c_char_p, [c_int]),
    "llkv_abi_version": (c_int, []),
    "llkv_append": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int,
                            c_int, c_void_p]),
    "llkv_scatter_prefill": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p,
                                     c_int, c_int, c_int, c_int, c_int, c_void_p]),
    "llkv_scatter_prefill_batched": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                             c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                             c_int, c_int, c_int, c_int, c_void_p]),
    "llkv_gather": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_int,
                            c_int64, c_int, c_int, c_int, c_int, c_void_p]),
    "llkv_build_slots": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int, c_int, c_int,
                                 c_void_p]),
    "llkv_rope_append": (c_int, [c_void_p] * 8 + [c_int] * 6 + [c_void_p]),
    "llkv_paged_decode_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int, c_int]),
    "llkv_paged_decode": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                  c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_int,
                                  c_void_p, c_size_t, c_void_p]),
    "llkv_paged_decode_noalloc_max_bytes": (c_size_t, []),
    "llkv_paged_decode_schedule": (c_int, [c_int] * 9 + [POINTER(c_int), POINTER(c_int)]),
    "llkv_paged_decode_noalloc": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                          c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                                          c_float, c_int, c_void_p]),
    "llkv_paged_decode_append": (c_int, [c_void_p] * 8 + [c_int] * 8 + [c_float, c_int, c_void_p,
                                                                         c_size_t, c_void_p]),
    "llkv_paged_prefill_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                                                     c_int]),
    "llkv_paged_prefill": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p,
                                   c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                                   c_int, c_float, c_int, c_void_p, c_size_t, c_void_p]),
    "llkv_first_prefill_batched": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                                           c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                           c_int, c_int, c_float, c_int, c_void_p]),
    "llkv_allocator_create": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                                      POINTER(c_void_p)]),
    "llkv_allocator_destroy": (None, [c_void_p]),
    "llkv_blocks_for_budget": (c_int, [c_uint64, c_int, c_int, c_int, c_int]),
    "llkv_allocator_allocate": (c_int, [c_void_p, c_uint64]),
    "llkv_allocator_allocate_tokens": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_int,
                                               POINTER(c_int)]),
    "llkv_allocator_release": (None, [c_void_p, c_int]),
    "llkv_allocator_find_by_hash": (c_int, [c_void_p, c_uint64]),
    "llkv_allocator_find_cached_prefix": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_int,
                                                  POINTER(c_int)]),
    "llkv_allocator_insert_cached_blocks": (None, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_int]),
    "llkv_allocator_evict_lru": (c_int, [c_void_p]),
    "llkv_allocator_increment_ref": (None, [c_void_p, c_int]),
    "llkv_allocator_reset": (c_int, [c_void_p]),
    "llkv_allocator_num_free": (c_int, [c_void_p]),
    "llkv_allocator_num_blocks": (c_int, [c_void_p]),
    "llkv_allocator_ref_count": (c_int, [c_void_p, c_int]),
    "llkv_allocator_token_hash": (c_uint64, [c_void_p, c_int]),
    "llkv_allocator_prefix_cache_size": (c_size_t, [c_void_p]),
    "llkv_allocator_k_storage": (c_void_p, [c_void_p]),
    "llkv_allocator_v_storage": (c_void_p, [c_void_p]),
    "llkv_allocator_storage_bytes": (c_size_t, [c_void_p]),
    "llkv_hash_tokens": (c_uint64, [c_void_p, c_int]),
}


def load_library(path: str | None = None):
    """Load liblightllm_kv.so (once).  Raises if it is absent: no fallback path exists."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise ImportError(f"{p} not found: build it with __graft_entry__.build() "
                          "(make -C lightllm_amd/csrc)")
    lib = ctypes.CDLL(p, mode=ctypes.RTLD_GLOBAL)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def lib():
    return load_library()


def check(status: int) -> None:
    if status != 0:
        msg = lib().llkv_last_error().decode(errors="replace")
        raise LLKVError(status, msg)


def library_path() -> str:
    return LIB_PATH


def last_error() -> str:
    return lib().llkv_last_error().decode(errors="replace")


def status_string(status: int) -> str:
    return lib().llkv_status_string(status).decode(errors="replace")
