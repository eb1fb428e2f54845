"""The C ABI library (lightllm_amd/liblightllm_kv.so) on the CPU: it loads, exports
every function include/lightllm_kv.h declares, and rejects bad arguments with the
documented status before touching a device.  No compute calls are made here."""
import ctypes
import os
import re

import pytest

from lightllm_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lightllm_kv.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(llkv_\w+)\s*\(", src)))


def test_header_declares_the_path():
    names = _declared()
    for n in ("llkv_append", "llkv_gather", "llkv_scatter_prefill", "llkv_scatter_prefill_batched",
              "llkv_paged_decode", "llkv_paged_decode_workspace_size", "llkv_paged_prefill",
              "llkv_first_prefill_batched", "llkv_allocator_create", "llkv_hash_tokens"):
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(L.library_path())
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_bindings_cover_the_header():
    missing = [n for n in _declared() if n not in L._SIGS]
    assert not missing, missing


def test_version_and_status_strings():
    lib = L.lib()
    assert lib.llkv_abi_version() == 4
    assert L.status_string(0) == "ok"
    assert "invalid" in L.status_string(1)
    assert "unsupported" in L.status_string(2) or "support" in L.status_string(2)
    assert L.status_string(99)


def _err(rc):
    return rc, L.last_error()


def test_append_rejects_null_pointers():
    lib = L.lib()
    rc, msg = _err(lib.llkv_append(None, None, None, None, None, 4, 2, 64, 0, None))
    assert rc == 1 and "null" in msg
    # zero rows is a no-op, as the reference's loops over zero tokens
    assert lib.llkv_append(None, None, None, None, None, 0, 2, 64, 0, None) == 0


def test_decode_argument_checks():
    lib = L.lib()
    d = lib.llkv_paged_decode
    # D > 256 throws in the reference (src/kv_cache/paged_attention.cu:543-544)
    rc, msg = _err(d(None, None, None, None, None, None, 4, 14, 2, 300, 16, 8, 128, 0, 0.1, 0,
                     None, 0, None))
    assert rc == 2 and "256" in msg
    rc, msg = _err(d(None, None, None, None, None, None, 4, 14, 3, 64, 16, 8, 128, 0, 0.1, 0,
                     None, 0, None))
    assert rc == 1 and "multiple" in msg
    # unsupported dtype (dispatch.h:38-40)
    rc, _ = _err(d(None, None, None, None, None, None, 4, 14, 2, 64, 16, 8, 128, 0, 0.1, 7,
                   None, 0, None))
    assert rc in (1, 2)


def test_decode_workspace_size():
    lib = L.lib()
    ws = lib.llkv_paged_decode_workspace_size
    # one split needs no partials
    assert ws(64, 14, 2, 64, 16, 2049, 1) == 0
    # fixed S=8: fp32 partial rows of D plus one lse per (seq, head, split)
    n = 64 * 14 * 8
    assert ws(64, 14, 2, 64, 16, 2049, 8) >= n * (64 + 1) * 4
    # grows with the split count and never shrinks with a longer context
    assert ws(64, 14, 2, 64, 16, 2049, 16) > ws(64, 14, 2, 64, 16, 2049, 8)
    assert ws(64, 14, 2, 64, 16, 32768, 0) >= ws(64, 14, 2, 64, 16, 2048, 0)


def test_decode_rejects_small_workspace():
    lib = L.lib()
    need = lib.llkv_paged_decode_workspace_size(4, 14, 2, 64, 16, 4096, 8)
    assert need > 0
    fake = ctypes.c_void_p(0x1000)   # never dereferenced: the size check fails first
    rc, msg = _err(lib.llkv_paged_decode(fake, fake, fake, fake, fake, fake, 4, 14, 2, 64, 16,
                                         256, 4096, 8, 0.125, 0, fake, need - 1, None))
    assert rc == 3 and "workspace" in msg


def test_table_position_overflow_rejected():
    """max_blocks_per_seq * block_size must fit the kernels' int token positions."""
    lib = L.lib()
    fake = ctypes.c_void_p(0x1000)   # never dereferenced: the checks fail first
    rc, msg = _err(lib.llkv_paged_decode(fake, fake, fake, fake, fake, fake, 1, 14, 2, 64, 16,
                                         1 << 28, 4096, 0, 0.125, 0, fake, 1 << 20, None))
    assert rc == 2 and "too large" in msg
    rc, msg = _err(lib.llkv_paged_prefill(fake, fake, fake, fake, fake, 1 << 28, fake, fake, 1, 16,
                                          16, 4096, 14, 2, 64, 16, 1, 0.125, 1, fake, 1 << 20, None))
    assert rc == 2 and "too large" in msg


def test_prefill_argument_checks():
    lib = L.lib()
    rc, msg = _err(lib.llkv_paged_prefill(None, None, None, None, None, 8, None, None, 1, 16, 16,
                                          16, 14, 2, 512, 16, 1, 0.1, 0, None, 0, None))
    assert rc == 2 and "256" in msg


def test_rope_append_argument_checks():
    lib = L.lib()
    fake = ctypes.c_void_p(0x1000)   # never dereferenced: the checks fail first
    rc, msg = _err(lib.llkv_rope_append(fake, fake, fake, fake, fake, fake, fake, fake, 4, 8, 2, 64,
                                        63, 1, None))
    assert rc == 1 and "rotary_dim" in msg
    rc, msg = _err(lib.llkv_rope_append(fake, fake, fake, fake, fake, fake, fake, fake, 4, 8, 2, 64,
                                        80, 1, None))
    assert rc == 1 and "rotary_dim" in msg
    rc, msg = _err(lib.llkv_rope_append(None, None, fake, fake, fake, fake, fake, fake, 4, 8, 2, 64,
                                        64, 1, None))
    assert rc == 1 and "null" in msg
    rc, msg = _err(lib.llkv_rope_append(fake, fake, fake, fake, fake, fake, fake, fake, 4, 8, 2, 64,
                                        64, 7, None))
    assert rc == 1 and "dtype" in msg
    assert lib.llkv_rope_append(None, None, None, None, None, None, None, None, 0, 8, 2, 64, 64, 1,
                                None) == 0   # nothing to do
    rc, msg = _err(lib.llkv_build_slots(None, None, 4, None, None, 2, 5, 16, None))
    assert rc == 1 and "null" in msg


def test_prefill_workspace_size():
    lib = L.lib()
    ws = lib.llkv_paged_prefill_workspace_size
    # key ranges under two minimum chunks (16 tiles): no chunking, no workspace
    assert ws(8, 4096, 512, 900, 14, 64, 16, 1) == 0
    # enough (sequence, query block, head) units to fill the GPU unsplit: no workspace
    assert ws(64, 32768, 512, 4608, 14, 64, 16, 1) == 0
    # configuration 4 (keys up to 4608): chunked; a 256-byte header (the main kernel's
    # split decision), then per partial row an fp32 log-sum-exp and D fp32 values
    hdr = 256
    n = ws(8, 4096, 512, 4608, 14, 64, 16, 1)
    assert n > hdr and (n - hdr) % (128 * (4 + 64 * 4)) == 0
    # fp32 and bf16 pools take the same plan and the same partial rows
    n32 = ws(8, 4096, 512, 4608, 14, 64, 16, 0)
    assert n32 == n
    assert ws(8, 4096, 512, 4608, 14, 64, 16, 2) == n32
    # shapes outside the MFMA kernels (head_dim 67, page size 8) run unsplit: no workspace
    assert ws(8, 4096, 512, 4608, 14, 67, 16, 0) == 0
    assert ws(8, 4096, 512, 4608, 14, 64, 8, 1) == 0
    # head_dim 256 on the MFMA kernels: chunked, the same fp32 partial rows for every pool type
    n16 = ws(8, 4096, 512, 4608, 16, 256, 16, 1)
    n32 = ws(8, 4096, 512, 4608, 16, 256, 16, 0)
    assert n16 > 0 and n32 == n16 and (n16 - hdr) % (128 * (4 + 256 * 4)) == 0


def test_hash_tokens_abi():
    lib = L.lib()
    arr = (ctypes.c_int * 1)(0x61)
    assert lib.llkv_hash_tokens(arr, 1) == 0xAF63DC4C8601EC8C


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(ImportError):
        L.load_library(str(tmp_path / "liblightllm_kv.so"))
