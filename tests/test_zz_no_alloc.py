"""llkv_paged_decode_noalloc (split partials in the library's device array, no workspace)
against llkv_paged_decode with a workspace: identical bits on two calls in a row, the second
smaller, over the fixed-split and the balanced schedules; a shape beyond the array is
rejected."""
import math

import numpy as np
import pytest
import torch

from lightllm_amd import kv_cache as kc
from lightllm_amd import workloads as wl
from lightllm_amd._lib import lib
from lightllm_amd.kv_cache import _ptr, dtype_code

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _bits(t):
    t = t.detach().cpu().contiguous()
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32).numpy()


def _noalloc(q, kp, vp, table, lens, max_len, num_splits=0):
    b, hq, d = q.shape
    out = torch.full_like(q, float("nan"))
    rc = lib().llkv_paged_decode_noalloc(_ptr(out), _ptr(q), _ptr(kp), _ptr(vp), _ptr(table), _ptr(lens),
                                         b, hq, kp.shape[2], d, kp.shape[1], table.shape[1], max_len,
                                         num_splits, 1.0 / math.sqrt(d), dtype_code(q.dtype), None)
    return rc, out


def _case(B, hq, hkv, d, lo, hi, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (B,), generator=g).tolist()
    nb = sum((L + 15) // 16 for L in lens) + 8
    return wl.decode_case(f"noalloc{seed}", B, hq, hkv, d, lens, nb, dtype, seed, append=False)


@pytest.mark.parametrize("name,first,second", [
    ("fixed_split_fp32", (64, 14, 2, 64, 128, 2048, torch.float32, 1), (8, 14, 2, 64, 1, 700, torch.float32, 2)),
    ("balanced_fp16", (300, 32, 8, 128, 1, 1500, torch.float16, 3), (40, 32, 8, 128, 1, 300, torch.float16, 4)),
])
def test_noalloc_matches_workspace_decode(name, first, second):
    print(f"no-alloc decode {name}", flush=True)
    for args in (first, second):
        c = _case(*args)
        q, kp, vp = c.q.to(DEV), c.k_pool.to(DEV), c.v_pool.to(DEV)
        table, lens = c.block_table.to(DEV), c.seq_lens.to(DEV)
        ref = kc.paged_decode(q, kp, vp, table, lens, c.max_seq_len)
        rc, out = _noalloc(q, kp, vp, table, lens, c.max_seq_len)
        torch.cuda.synchronize()
        assert rc == 0, lib().llkv_last_error()
        assert np.array_equal(_bits(out), _bits(ref)), f"{name} B={args[0]}: outputs differ"


def test_noalloc_rejects_shapes_beyond_the_array():
    cap = lib().llkv_paged_decode_noalloc_max_bytes()
    assert cap == 16 << 20
    # fixed 64-way split of 1024 x 64 heads: 1024 * 64 * 64 * (128 + 1) * 4 bytes of partials
    assert kc.decode_workspace_bytes(1024, 64, 8, 128, 16, 32768, 64) > cap
    q = torch.zeros(1024, 64, 128, dtype=torch.float16, device=DEV)
    kp = torch.zeros(4, 16, 8, 128, dtype=torch.float16, device=DEV)
    table = torch.zeros(1024, 2048, dtype=torch.int32, device=DEV)
    lens = torch.zeros(1024, dtype=torch.int32, device=DEV)
    rc, _ = _noalloc(q, kp, kp, table, lens, 32768, num_splits=64)
    assert rc == 3 and b"scratch" in lib().llkv_last_error() and b"workspace" in lib().llkv_last_error()
