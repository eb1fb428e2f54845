"""Seeded synthetic inputs for the five configurations of the paged KV-cache path
(the benchmark configurations 1-5), built on the host with torch's CPU generator.

Each builder returns plain host tensors (pools [num_blocks, 16, Hkv, D], int32
block tables padded with -1, int32 lengths, int64 slot mappings), so tests and
the benchmark can move them to the device and hand the same bytes to the CPU
oracle.  Block tables are drawn from a seeded random permutation of the pool
("assigned in random order").
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import torch

PAGE = 16


@dataclass
class DecodeCase:
    name: str
    q: torch.Tensor            # [B, Hq, D]
    k_pool: torch.Tensor       # [nb, 16, Hkv, D]
    v_pool: torch.Tensor
    block_table: torch.Tensor  # [B, max_blocks] int32, -1 padded
    seq_lens: torch.Tensor     # [B] int32 (keys attended, after the append)
    k_new: Optional[torch.Tensor] = None   # [B, Hkv, D] appended token (pos = len-1)
    v_new: Optional[torch.Tensor] = None
    slots: Optional[torch.Tensor] = None   # [B] int64
    scale: float = 0.125
    splits: List[int] = field(default_factory=lambda: [0])

    @property
    def max_seq_len(self) -> int:
        return int(self.seq_lens.max().item()) if self.seq_lens.numel() else 0


@dataclass
class PrefillCase:
    name: str
    q: torch.Tensor            # [total_q, Hq, D]
    k_pool: torch.Tensor
    v_pool: torch.Tensor
    block_table: torch.Tensor  # [N, max_blocks]
    cu_q: torch.Tensor         # [N+1] int32
    seq_lens: torch.Tensor     # [N] int32 (history + chunk)
    k_chunk: torch.Tensor      # [total_q, Hkv, D] chunk K/V to append before attention
    v_chunk: torch.Tensor
    slots: torch.Tensor        # [total_q] int64
    causal: bool = True
    scale: float = 0.125

    @property
    def max_q_len(self) -> int:
        return int((self.cu_q[1:] - self.cu_q[:-1]).max().item())

    @property
    def max_seq_len(self) -> int:
        return int(self.seq_lens.max().item())


def _pool(nb: int, hkv: int, d: int, dtype: torch.dtype, g: torch.Generator):
    k = torch.randn(nb, PAGE, hkv, d, generator=g).to(dtype)
    v = torch.randn(nb, PAGE, hkv, d, generator=g).to(dtype)
    return k, v


def _tables(lengths: List[int], perm: torch.Tensor, max_blocks: int, start: int = 0):
    """Consecutive slices of `perm` as each sequence's pages; returns table, next index."""
    b = len(lengths)
    table = torch.full((b, max_blocks), -1, dtype=torch.int32)
    pos = start
    for i, L in enumerate(lengths):
        n = (L + PAGE - 1) // PAGE
        table[i, :n] = perm[pos:pos + n]
        pos += n
    return table, pos


def _slots_for(table: torch.Tensor, positions: List[int]) -> torch.Tensor:
    return torch.tensor([int(table[i, p // PAGE]) * PAGE + p % PAGE for i, p in enumerate(positions)],
                        dtype=torch.int64)


def decode_case(name: str, B: int, hq: int, hkv: int, d: int, lengths: List[int], nb: int,
                dtype: torch.dtype, seed: int, append: bool = True, k_outlier_frac: float = 0.0,
                splits: Optional[List[int]] = None, max_blocks: Optional[int] = None) -> DecodeCase:
    """Decode over `lengths` cached tokens; with append=True one new token per sequence is
    appended at position L and the decode attends L+1 keys."""
    g = torch.Generator().manual_seed(seed)
    total_lens = [L + (1 if append else 0) for L in lengths]
    need = sum((L + PAGE - 1) // PAGE for L in total_lens)
    if need > nb:
        raise ValueError(f"{name}: pool of {nb} blocks < {need} needed")
    k_pool, v_pool = _pool(nb, hkv, d, dtype, g)
    if k_outlier_frac > 0:
        mask = torch.rand(k_pool.shape, generator=g) < k_outlier_frac
        k_pool = torch.where(mask, (k_pool.float() * 8).to(dtype), k_pool)
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    mb = max_blocks or max((L + PAGE - 1) // PAGE for L in total_lens)
    table, _ = _tables(total_lens, perm, mb)
    q = torch.randn(B, hq, d, generator=g).to(dtype)
    case = DecodeCase(name, q, k_pool, v_pool, table, torch.tensor(total_lens, dtype=torch.int32),
                      scale=1.0 / math.sqrt(d), splits=splits or [0])
    if append:
        case.k_new = torch.randn(B, hkv, d, generator=g).to(dtype)
        case.v_new = torch.randn(B, hkv, d, generator=g).to(dtype)
        case.slots = _slots_for(table, lengths)
    return case


def config1(seed: int = 1) -> DecodeCase:
    """B=1, Qwen2.5-0.5B shape (14/2/64) fp32, context 512, pool 4096 blocks."""
    return decode_case("cfg1", 1, 14, 2, 64, [512], 4096, torch.float32, seed, append=False)


def config2(seed: int = 2, nb: int = 32768) -> DecodeCase:
    """B=64 fp32, contexts U[128, 2048], one appended token each, pool 32768 blocks."""
    g = torch.Generator().manual_seed(seed + 1000)
    lengths = torch.randint(128, 2049, (64,), generator=g).tolist()
    return decode_case("cfg2", 64, 14, 2, 64, lengths, nb, torch.float32, seed, append=True)


def config3(seed: int = 3) -> DecodeCase:
    """B=16, context 32768 each, fp16 K/V with 1% of K entries x8, splits 4 and 16."""
    return decode_case("cfg3", 16, 14, 2, 64, [32768] * 16, 16 * 2048, torch.float16, seed,
                       append=False, k_outlier_frac=0.01, splits=[4, 16, 0])


def prefill_case(name: str, hq: int, hkv: int, d: int, prefixes: List[int], chunks: List[int],
                 share_groups: Dict[int, List[int]], nb: int, dtype: torch.dtype, seed: int,
                 causal: bool = True) -> PrefillCase:
    """Chunked prefill: sequence n has a cached prefix of prefixes[n] tokens and a new chunk of
    chunks[n] tokens.  share_groups maps a representative sequence to the sequences that reuse
    its prefix pages (same physical blocks, as a radix-tree hit).  Shared prefixes must be
    page-aligned."""
    g = torch.Generator().manual_seed(seed)
    n = len(prefixes)
    k_pool, v_pool = _pool(nb, hkv, d, dtype, g)
    perm = torch.randperm(nb, generator=g).to(torch.int32).tolist()
    totals = [p + c for p, c in zip(prefixes, chunks)]
    mb = max((t + PAGE - 1) // PAGE for t in totals)
    table = torch.full((n, mb), -1, dtype=torch.int32)
    owner = {}
    for rep, members in share_groups.items():
        for m in members:
            owner[m] = rep
    pos = 0
    prefix_pages: Dict[int, List[int]] = {}
    for i in range(n):
        rep = owner.get(i, i)
        npref = prefixes[i] // PAGE
        if prefixes[i] % PAGE and rep != i:
            raise ValueError("shared prefixes must be page aligned")
        if rep in prefix_pages:
            pages = prefix_pages[rep][:npref]
        else:
            pages = perm[pos:pos + npref]
            pos += npref
            prefix_pages[rep] = pages
        rest = (totals[i] + PAGE - 1) // PAGE - npref
        tail = perm[pos:pos + rest]
        pos += rest
        row = pages + tail
        table[i, :len(row)] = torch.tensor(row, dtype=torch.int32)
    cu = [0]
    for c in chunks:
        cu.append(cu[-1] + c)
    total_q = cu[-1]
    q = torch.randn(total_q, hq, d, generator=g).to(dtype)
    k_chunk = torch.randn(total_q, hkv, d, generator=g).to(dtype)
    v_chunk = torch.randn(total_q, hkv, d, generator=g).to(dtype)
    slots = []
    for i in range(n):
        for t in range(chunks[i]):
            p = prefixes[i] + t
            slots.append(int(table[i, p // PAGE]) * PAGE + p % PAGE)
    return PrefillCase(name, q, k_pool, v_pool, table, torch.tensor(cu, dtype=torch.int32),
                       torch.tensor(totals, dtype=torch.int32), k_chunk, v_chunk,
                       torch.tensor(slots, dtype=torch.int64), causal, 1.0 / math.sqrt(d))


CFG4_PREFIXES = [0, 256, 1024, 4096, 4096, 4096, 2048, 512]


def config4(seed: int = 4, nb: int = 4096, dtype=torch.float16) -> PrefillCase:
    """8 x 512-token chunks over prefixes {0,256,1024,4096,4096,4096,2048,512}; the three 4096
    prefixes share physical pages; causal; 14/2/64 fp16 (dtype: the same shape in another
    element type)."""
    return prefill_case("cfg4", 14, 2, 64, CFG4_PREFIXES, [512] * 8, {3: [3, 4, 5]}, nb,
                        dtype, seed)


@dataclass
class MixedCase:
    decode: DecodeCase
    prefill: PrefillCase


def device_pools(nb: int, hkv: int, d: int, dtype: torch.dtype, seed: int, device):
    """N(0,1) pools generated on the device (multi-GB pools are never built on the host)."""
    g = torch.Generator(device=device).manual_seed(seed)
    k = torch.randn(nb, PAGE, hkv, d, generator=g, device=device, dtype=torch.float32).to(dtype)
    v = torch.randn(nb, PAGE, hkv, d, generator=g, device=device, dtype=torch.float32).to(dtype)
    return k, v


def config5(seed: int = 5, nb: int = 262144, n_decode: int = 256, n_prefill: int = 4,
            chunk: int = 1024, prefix: int = 2048) -> MixedCase:
    """Llama-3-8B attention (32/8/128) fp16: 256 decode sequences, contexts lognormal(median
    1024, sigma 1) clipped to [16, 16384], plus 4 chunks of 1024 tokens on one shared
    2048-token prefix; pool 262144 blocks shared by both parts.  The pools are left empty
    (k_pool/v_pool None): build them on the device with device_pools()."""
    g = torch.Generator().manual_seed(seed)
    hq, hkv, d, dtype = 32, 8, 128, torch.float16
    z = torch.randn(n_decode, generator=g, dtype=torch.float64)
    lengths = torch.exp(math.log(1024.0) + z).round().clamp(16, 16384).to(torch.int64).tolist()
    k_pool = v_pool = None
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    total_lens = [L + 1 for L in lengths]
    mbd = max((L + PAGE - 1) // PAGE for L in total_lens)
    dtable, pos = _tables(total_lens, perm, mbd)
    q = torch.randn(n_decode, hq, d, generator=g).to(dtype)
    dec = DecodeCase("cfg5-decode", q, k_pool, v_pool, dtable,
                     torch.tensor(total_lens, dtype=torch.int32), scale=1.0 / math.sqrt(d))
    dec.k_new = torch.randn(n_decode, hkv, d, generator=g).to(dtype)
    dec.v_new = torch.randn(n_decode, hkv, d, generator=g).to(dtype)
    dec.slots = _slots_for(dtable, lengths)
    # prefill: shared prefix pages then private chunk pages, from the rest of the permutation
    npref = prefix // PAGE
    shared = perm[pos:pos + npref].tolist()
    pos += npref
    per_chunk = (chunk + PAGE - 1) // PAGE
    mbp = npref + per_chunk
    ptable = torch.full((n_prefill, mbp), -1, dtype=torch.int32)
    for i in range(n_prefill):
        own = perm[pos:pos + per_chunk].tolist()
        pos += per_chunk
        ptable[i] = torch.tensor(shared + own, dtype=torch.int32)
    cu = torch.arange(0, (n_prefill + 1) * chunk, chunk, dtype=torch.int32)
    total_q = n_prefill * chunk
    pq = torch.randn(total_q, hq, d, generator=g).to(dtype)
    kc = torch.randn(total_q, hkv, d, generator=g).to(dtype)
    vc = torch.randn(total_q, hkv, d, generator=g).to(dtype)
    slots = []
    for i in range(n_prefill):
        for t in range(chunk):
            p = prefix + t
            slots.append(int(ptable[i, p // PAGE]) * PAGE + p % PAGE)
    pre = PrefillCase("cfg5-prefill", pq, k_pool, v_pool, ptable, cu,
                      torch.full((n_prefill,), prefix + chunk, dtype=torch.int32), kc, vc,
                      torch.tensor(slots, dtype=torch.int64), True, 1.0 / math.sqrt(d))
    return MixedCase(dec, pre)


# ---------------------------------------------------------------------------
# Algorithmic work (exact tokens, no page padding, no split partials)
# ---------------------------------------------------------------------------

def decode_bytes(case: DecodeCase, exact_tokens: bool = True) -> int:
    B, hq, d = case.q.shape
    hkv = case.k_new.shape[1] if case.k_pool is None else case.k_pool.shape[2]
    es = case.q.element_size()
    lens = case.seq_lens.to(torch.int64)
    toks = int(lens.sum()) if exact_tokens else int(((lens + PAGE - 1) // PAGE * PAGE).sum())
    kv = toks * hkv * d * es * 2
    qo = B * hq * d * case.q.element_size() * 2
    tables = int(((lens + PAGE - 1) // PAGE).sum()) * 4 + B * 4
    return kv + qo + tables


def append_bytes(case: DecodeCase) -> int:
    B = case.k_new.shape[0]
    hkv, d = case.k_new.shape[1], case.k_new.shape[2]
    return 2 * B * hkv * d * case.k_new.element_size() * 2 + 8 * B


def prefill_flops(case: PrefillCase) -> int:
    """4*D FLOP per unmasked (query, key) pair per q head."""
    hq, d = case.q.shape[1], case.q.shape[2]
    pairs = 0
    cu = case.cu_q.tolist()
    for i, L in enumerate(case.seq_lens.tolist()):
        P = cu[i + 1] - cu[i]
        if case.causal:
            pairs += sum(L - P + t + 1 for t in range(P))
        else:
            pairs += P * L
    return pairs * hq * 4 * d
