"""lightllm_amd -- MI355X (gfx950) paged KV-cache hot path of wjb554/lightllm.

The product is liblightllm_kv.so (HIP kernels + C ABI + C++ operator API,
sources in lightllm_amd/csrc, ABI in include/lightllm_kv.h).  This package is
the Python binding used by the tests and the benchmark.
"""
from ._lib import LIB_PATH, LLKVError, check, lib, load_library  # noqa: F401

__all__ = ["LIB_PATH", "LLKVError", "check", "lib", "load_library"]
