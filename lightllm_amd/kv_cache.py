"""Python mirror of the reference's paged KV-cache operator API
(include/lightllm/kv_cache/paged_attention.h:31-145 and
block_allocator.h:37-186 of wjb554/lightllm), over the C ABI.

Torch provides device memory and the stream; every computation runs in the
gfx950 kernels of liblightllm_kv.so.  Device index arrays are int32 (block
tables, lengths, offsets) except slot mappings (int64).
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional, Sequence

import torch

from ._lib import DTYPE_BF16, DTYPE_F16, DTYPE_F32, check, lib

_TORCH_TO_DT = {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}
_DT_TO_TORCH = {v: k for k, v in _TORCH_TO_DT.items()}

POLICY_HASH, POLICY_RADIX = 0, 1
STORAGE_DEVICE, STORAGE_HOST, STORAGE_NONE = 0, 1, 2


def dtype_code(t: torch.dtype) -> int:
    try:
        return _TORCH_TO_DT[t]
    except KeyError:
        raise ValueError(f"unsupported dtype {t}") from None


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream=None):
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _require(t: torch.Tensor, dtype: torch.dtype, name: str):
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")


class BlockAllocator:
    """Block pool + prefix cache (reference BlockAllocator semantics, implemented in
    C++).  K/V pools are torch tensors [num_blocks, block_size, Hkv, D] on `device`
    (or none with device=None, metadata only)."""

    def __init__(self, num_blocks: int, block_size: int, num_kv_heads: int, head_dim: int,
                 policy: int = POLICY_HASH, kv_dtype: torch.dtype = torch.float32,
                 device: Optional[str] = "cuda"):
        self.num_blocks, self.block_size = num_blocks, block_size
        self.num_kv_heads, self.head_dim = num_kv_heads, head_dim
        self.kv_dtype, self.policy = kv_dtype, policy
        h = ctypes.c_void_p()
        check(lib().llkv_allocator_create(num_blocks, block_size, num_kv_heads, head_dim, policy,
                                          dtype_code(kv_dtype), STORAGE_NONE, ctypes.byref(h)))
        self._h = h
        if device is not None:
            shape = (num_blocks, block_size, num_kv_heads, head_dim)
            self.k_storage = torch.zeros(shape, dtype=kv_dtype, device=device)
            self.v_storage = torch.zeros(shape, dtype=kv_dtype, device=device)
        else:
            self.k_storage = self.v_storage = None

    @staticmethod
    def blocks_for_budget(budget_bytes: int, block_size: int, num_kv_heads: int, head_dim: int,
                          kv_dtype: torch.dtype) -> int:
        """Pages (K and V) that fit `budget_bytes` in the pool's element type."""
        n = lib().llkv_blocks_for_budget(budget_bytes, block_size, num_kv_heads, head_dim,
                                         dtype_code(kv_dtype))
        if n < 0:
            raise ValueError("blocks_for_budget: bad arguments")
        return n

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            lib().llkv_allocator_destroy(h)
            self._h = None

    # ---- allocation --------------------------------------------------------
    def allocate(self, token_hash: int = 0) -> int:
        return lib().llkv_allocator_allocate(self._h, token_hash)

    def allocate_tokens(self, tokens: Sequence[int], start_pos: int):
        """Returns (n_new, all_block_ids)."""
        arr = (ctypes.c_int * max(1, len(tokens)))(*tokens)
        cap = len(tokens) // self.block_size + 2
        out = (ctypes.c_int * cap)()
        cnt = ctypes.c_int(0)
        n_new = lib().llkv_allocator_allocate_tokens(self._h, arr, len(tokens), start_pos, out, cap,
                                                     ctypes.byref(cnt))
        return n_new, list(out[: cnt.value])

    def release(self, block_id: int) -> None:
        lib().llkv_allocator_release(self._h, block_id)

    def find_by_hash(self, token_hash: int) -> int:
        return lib().llkv_allocator_find_by_hash(self._h, token_hash)

    def find_cached_prefix(self, tokens: Sequence[int], start_pos: int):
        """Returns (matched_tokens, block_ids)."""
        arr = (ctypes.c_int * max(1, len(tokens)))(*tokens)
        cap = len(tokens) // self.block_size + 2
        out = (ctypes.c_int * cap)()
        n = ctypes.c_int(0)
        matched = lib().llkv_allocator_find_cached_prefix(self._h, arr, len(tokens), start_pos, out,
                                                          cap, ctypes.byref(n))
        return matched, list(out[: n.value])

    def insert_cached_blocks(self, tokens: Sequence[int], start_pos: int,
                             block_ids: Sequence[int]) -> None:
        arr = (ctypes.c_int * max(1, len(tokens)))(*tokens)
        ids = (ctypes.c_int * max(1, len(block_ids)))(*block_ids)
        lib().llkv_allocator_insert_cached_blocks(self._h, arr, len(tokens), start_pos, ids,
                                                  len(block_ids))

    def evict_lru(self) -> int:
        return lib().llkv_allocator_evict_lru(self._h)

    def increment_ref(self, block_id: int) -> None:
        lib().llkv_allocator_increment_ref(self._h, block_id)

    def reset(self) -> None:
        check(lib().llkv_allocator_reset(self._h))
        if self.k_storage is not None:
            self.k_storage.zero_()
            self.v_storage.zero_()

    # ---- inspection --------------------------------------------------------
    def num_free(self) -> int:
        return lib().llkv_allocator_num_free(self._h)

    def ref_count(self, block_id: int) -> int:
        return lib().llkv_allocator_ref_count(self._h, block_id)

    def token_hash(self, block_id: int) -> int:
        return lib().llkv_allocator_token_hash(self._h, block_id)

    def prefix_cache_size(self) -> int:
        return lib().llkv_allocator_prefix_cache_size(self._h)


def hash_tokens(tokens: Sequence[int]) -> int:
    arr = (ctypes.c_int * max(1, len(tokens)))(*tokens)
    return lib().llkv_hash_tokens(arr, len(tokens))


# ---------------------------------------------------------------------------
# Operators
# ---------------------------------------------------------------------------

def append_kv(k: torch.Tensor, v: torch.Tensor, slot_mapping: torch.Tensor,
              k_pool: torch.Tensor, v_pool: torch.Tensor, stream=None) -> None:
    """KV append by slot mapping: row i of k/v -> pool row slot_mapping[i] (int64, <0 skips)."""
    _require(slot_mapping, torch.int64, "slot_mapping")
    _require(k, k_pool.dtype, "k")
    _require(v, k_pool.dtype, "v")
    hkv, d = k_pool.shape[2], k_pool.shape[3]
    check(lib().llkv_append(_ptr(k_pool), _ptr(v_pool), _ptr(k), _ptr(v), _ptr(slot_mapping),
                            k.shape[0], hkv, d, dtype_code(k_pool.dtype), _stream(stream)))


def build_slots(block_table: torch.Tensor, cu_tokens: torch.Tensor, start_pos: torch.Tensor,
                num_tokens: int, block_size: int = 16, out: Optional[torch.Tensor] = None,
                stream=None) -> torch.Tensor:
    """Device slot mapping: token t of sequence n (rows cu_tokens[n]..) sits at position
    start_pos[n] + t - cu_tokens[n]; slot = table[n][pos // bs] * bs + pos % bs, or -1 outside
    the table (the reference's write_decode_kv / scatter_prefill_kv host loops)."""
    for name, t in (("block_table", block_table), ("cu_tokens", cu_tokens), ("start_pos", start_pos)):
        _require(t, torch.int32, name)
    if out is None:
        out = torch.empty(num_tokens, dtype=torch.int64, device=block_table.device)
    _require(out, torch.int64, "out")
    check(lib().llkv_build_slots(_ptr(out), _ptr(block_table), block_table.shape[1], _ptr(cu_tokens),
                                 _ptr(start_pos), start_pos.shape[0], num_tokens, block_size,
                                 _stream(stream)))
    return out


def rope_append(q: Optional[torch.Tensor], k: torch.Tensor, v: torch.Tensor, slot_mapping: torch.Tensor,
                cos: torch.Tensor, sin: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                stream=None) -> None:
    """Fused RoPE + KV append: q [T, Hq, D] (or None) and k [T, Hkv, D] rotated in place over the
    first 2 * cos.shape[1] dims (Neox halves), then the k and v rows written to pool rows
    slot_mapping[t] (<0 skips).  cos / sin: fp32 [T, rotary_dim / 2]."""
    _require(slot_mapping, torch.int64, "slot_mapping")
    _require(k, k_pool.dtype, "k")
    _require(v, k_pool.dtype, "v")
    if q is not None:
        _require(q, k_pool.dtype, "q")
    _require(cos, torch.float32, "cos")
    _require(sin, torch.float32, "sin")
    t, hkv, d = k.shape
    hq = q.shape[1] if q is not None else 0
    check(lib().llkv_rope_append(_ptr(q), _ptr(k), _ptr(v), _ptr(k_pool), _ptr(v_pool),
                                 _ptr(slot_mapping), _ptr(cos), _ptr(sin), t, hq, hkv, d,
                                 2 * cos.shape[1], dtype_code(k_pool.dtype), _stream(stream)))


def scatter_prefill_kv(k: torch.Tensor, v: torch.Tensor, start_pos: int, n_tokens: int,
                       block_table: torch.Tensor, max_blocks: int, allocator: BlockAllocator,
                       stream=None) -> None:
    """Reference scatter_prefill_kv_gpu (paged_attention.h:95-102)."""
    _require(block_table, torch.int32, "block_table")
    _require(k, allocator.kv_dtype, "k")
    _require(v, allocator.kv_dtype, "v")
    check(lib().llkv_scatter_prefill(_ptr(allocator.k_storage), _ptr(allocator.v_storage), _ptr(k),
                                     _ptr(v), start_pos, n_tokens, _ptr(block_table), max_blocks,
                                     allocator.num_kv_heads, allocator.head_dim, allocator.block_size,
                                     dtype_code(allocator.kv_dtype), _stream(stream)))


def scatter_prefill_kv_batched(k_flat: torch.Tensor, v_flat: torch.Tensor, kv_offsets, num_tokens,
                               start_poss, token_cumsum, flat_bt, max_blocks: int, n: int,
                               p_total: int, allocator: BlockAllocator, stream=None) -> None:
    """Reference scatter_prefill_kv_batched_gpu_dispatch (paged_attention.h:116-124)."""
    for name, t in (("kv_offsets", kv_offsets), ("num_tokens", num_tokens),
                    ("start_poss", start_poss), ("token_cumsum", token_cumsum), ("flat_bt", flat_bt)):
        _require(t, torch.int32, name)
    check(lib().llkv_scatter_prefill_batched(
        _ptr(allocator.k_storage), _ptr(allocator.v_storage), _ptr(k_flat), _ptr(v_flat),
        allocator.num_kv_heads, allocator.head_dim, _ptr(kv_offsets), _ptr(num_tokens),
        _ptr(start_poss), _ptr(token_cumsum), _ptr(flat_bt), max_blocks, n, p_total,
        allocator.block_size, dtype_code(allocator.kv_dtype), _stream(stream)))


def gather_kv(k_pool: torch.Tensor, v_pool: torch.Tensor, block_table: torch.Tensor,
              cu_seqlens: torch.Tensor, total_tokens: int, stream=None):
    """Block-table gather into contiguous [total_tokens, Hkv, D] (reconstruct_kv on device)."""
    _require(block_table, torch.int32, "block_table")
    _require(cu_seqlens, torch.int32, "cu_seqlens")
    nb, bs, hkv, d = k_pool.shape
    kd = torch.empty((total_tokens, hkv, d), dtype=k_pool.dtype, device=k_pool.device)
    vd = torch.empty_like(kd)
    check(lib().llkv_gather(_ptr(kd), _ptr(vd), _ptr(k_pool), _ptr(v_pool), _ptr(block_table),
                            block_table.shape[1], _ptr(cu_seqlens), cu_seqlens.shape[0] - 1,
                            total_tokens, hkv, d, bs, dtype_code(k_pool.dtype), _stream(stream)))
    return kd, vd


def decode_workspace_bytes(num_seqs: int, hq: int, hkv: int, d: int, block_size: int,
                           max_seq_len: int, num_splits: int = 0) -> int:
    return lib().llkv_paged_decode_workspace_size(num_seqs, hq, hkv, d, block_size, max_seq_len,
                                                  num_splits)


DECODE_SCHEDULES = ("one_split", "unit", "splits", "balanced", "generic")


def decode_schedule(num_seqs: int, hq: int, hkv: int, d: int, max_seq_len: int, dtype: torch.dtype,
                    num_splits: int = 0, block_size: int = 16, with_append: bool = False):
    """(schedule name, key splits) that paged_decode / paged_decode_append take for this shape on
    the current device (llkv_paged_decode_schedule): one_split runs one kernel, unit one kernel
    (splits == 1) or 16-wave splits and a merge kernel, splits and balanced a merge kernel after
    the split kernel."""
    kind, splits = ctypes.c_int(), ctypes.c_int()
    check(lib().llkv_paged_decode_schedule(num_seqs, hq, hkv, d, block_size, max_seq_len, num_splits,
                                           dtype_code(dtype), int(with_append), ctypes.byref(kind),
                                           ctypes.byref(splits)))
    return DECODE_SCHEDULES[kind.value], splits.value


_WS: dict = {}


def _workspace(nbytes: int, device) -> torch.Tensor:
    """Workspace for the split partials of decode and prefill, cached per device and grown
    on demand.  Calls that share it must be ordered on one stream."""
    key = str(device)
    ws = _WS.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WS[key] = ws
    return ws


def paged_decode(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                 block_table: torch.Tensor, seq_lens: torch.Tensor, max_seq_len: int,
                 num_splits: int = 0, scale: Optional[float] = None,
                 out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None,
                 stream=None) -> torch.Tensor:
    """Paged decode attention over pools [nb, bs, Hkv, D]; q [B, Hq, D]."""
    _require(q, k_pool.dtype, "q")
    _require(block_table, torch.int32, "block_table")
    _require(seq_lens, torch.int32, "seq_lens")
    b, hq, d = q.shape
    nb, bs, hkv, _ = k_pool.shape
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if out is None:
        out = torch.empty_like(q)
    ws = decode_workspace_bytes(b, hq, hkv, d, bs, max_seq_len, num_splits)
    if ws and (workspace is None or workspace.numel() * workspace.element_size() < ws):
        workspace = _workspace(ws, q.device)
    check(lib().llkv_paged_decode(_ptr(out), _ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(block_table),
                                  _ptr(seq_lens), b, hq, hkv, d, bs, block_table.shape[1],
                                  max_seq_len, num_splits, scale, dtype_code(q.dtype),
                                  _ptr(workspace) if ws else None, ws, _stream(stream)))
    return out


def paged_decode_append(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                        k_pool: torch.Tensor, v_pool: torch.Tensor, block_table: torch.Tensor,
                        seq_lens: torch.Tensor, max_seq_len: int, num_splits: int = 0,
                        scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                        workspace: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Fused KV append + paged decode: the new rows k_new / v_new [B, Hkv, D] go to position
    seq_lens[b] - 1 of each sequence (seq_lens count the new token), then decode attention over
    [0, seq_lens[b]); equal to append_kv followed by paged_decode."""
    _require(q, k_pool.dtype, "q")
    _require(k_new, k_pool.dtype, "k_new")
    _require(v_new, k_pool.dtype, "v_new")
    _require(block_table, torch.int32, "block_table")
    _require(seq_lens, torch.int32, "seq_lens")
    b, hq, d = q.shape
    nb, bs, hkv, _ = k_pool.shape
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if out is None:
        out = torch.empty_like(q)
    ws = decode_workspace_bytes(b, hq, hkv, d, bs, max_seq_len, num_splits)
    if ws and (workspace is None or workspace.numel() * workspace.element_size() < ws):
        workspace = _workspace(ws, q.device)
    check(lib().llkv_paged_decode_append(_ptr(out), _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(k_pool),
                                         _ptr(v_pool), _ptr(block_table), _ptr(seq_lens), b, hq, hkv,
                                         d, bs, block_table.shape[1], max_seq_len, num_splits, scale,
                                         dtype_code(q.dtype), _ptr(workspace) if ws else None, ws,
                                         _stream(stream)))
    return out


def paged_attention(q: torch.Tensor, block_table: torch.Tensor, max_blocks_per_seq: int,
                    seq_lens: torch.Tensor, allocator: BlockAllocator,
                    max_seq_len: Optional[int] = None) -> torch.Tensor:
    """Reference paged_attention (paged_attention.h:31-36).  Like the reference, reads
    seq_lens back to size the launch unless max_seq_len is given."""
    if max_seq_len is None:
        max_seq_len = int(seq_lens.max().item()) if seq_lens.numel() else 0
    bt = block_table.view(-1, max_blocks_per_seq)
    return paged_decode(q, allocator.k_storage, allocator.v_storage, bt, seq_lens, max_seq_len)


def paged_prefill(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                  block_table: torch.Tensor, cu_q: torch.Tensor, seq_lens: torch.Tensor,
                  max_q_len: int, max_seq_len: int, causal: bool = True,
                  scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                  stream=None, workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Varlen paged prefill: q [total_q, Hq, D], sequence n owns rows cu_q[n]:cu_q[n+1].
    workspace: uint8 device buffer for the key-chunk partials (default: a cached one);
    pass an empty tensor to run every key range unsplit."""
    _require(q, k_pool.dtype, "q")
    for name, t in (("block_table", block_table), ("cu_q", cu_q), ("seq_lens", seq_lens)):
        _require(t, torch.int32, name)
    tq, hq, d = q.shape
    nb, bs, hkv, _ = k_pool.shape
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if out is None:
        out = torch.empty_like(q)
    n = seq_lens.shape[0]
    ws_bytes = lib().llkv_paged_prefill_workspace_size(n, tq, max_q_len, max_seq_len, hq, d, bs,
                                                       dtype_code(q.dtype))
    if workspace is None and ws_bytes:
        workspace = _workspace(ws_bytes, q.device)
    ws_ptr = _ptr(workspace) if workspace is not None else None
    ws_len = workspace.numel() if workspace is not None else 0
    check(lib().llkv_paged_prefill(_ptr(out), _ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(block_table),
                                   block_table.shape[1], _ptr(cu_q), _ptr(seq_lens),
                                   n, tq, max_q_len, max_seq_len, hq, hkv, d, bs,
                                   1 if causal else 0, scale, dtype_code(q.dtype), ws_ptr, ws_len,
                                   _stream(stream)))
    return out


def prefill_paged_attention(q: torch.Tensor, block_table: torch.Tensor, max_blocks: int,
                            seq_len: torch.Tensor, allocator: BlockAllocator,
                            causal: bool = False) -> torch.Tensor:
    """Reference prefill_paged_attention (paged_attention.h:71-77): one sequence, seq_len is a
    device int32 [1] holding history + P."""
    p = q.shape[0]
    total = int(seq_len.reshape(-1)[0].item())
    cu = torch.tensor([0, p], dtype=torch.int32, device=q.device)
    bt = block_table.reshape(1, -1)[:, :max_blocks].contiguous()
    return paged_prefill(q, allocator.k_storage, allocator.v_storage, bt, cu,
                         seq_len.reshape(-1)[:1].contiguous(), p, total, causal)


def first_prefill_attn_batched(out: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                               hq: int, hkv: int, d: int, offsets, kv_offsets, num_tokens,
                               token_cumsum, start_poss, n: int, p_total: int, scale: float,
                               stream=None, max_tokens: int = 0) -> None:
    """Reference first_prefill_attn_batched_gpu_dispatch (paged_attention.h:138-145).
    offsets / kv_offsets are element offsets of row starts; max_tokens is a host upper bound
    of num_tokens (0: p_total)."""
    for name, t in (("offsets", offsets), ("kv_offsets", kv_offsets), ("num_tokens", num_tokens),
                    ("token_cumsum", token_cumsum), ("start_poss", start_poss)):
        _require(t, torch.int32, name)
    check(lib().llkv_first_prefill_batched(_ptr(out), _ptr(q), _ptr(k), _ptr(v), hq, hkv, d,
                                           _ptr(offsets), _ptr(kv_offsets), _ptr(num_tokens),
                                           _ptr(token_cumsum), _ptr(start_poss), n, p_total, max_tokens,
                                           scale, dtype_code(q.dtype), _stream(stream)))
