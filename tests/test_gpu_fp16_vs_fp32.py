"""fp16 pools against fp32 pools on the same data, as the reference's
tests/test_attention_fp16.cpp does (its tests 1-6, :293-600): the same LCG inputs
(rng_seed / rng_randf, :31-38, values in [-1, 1) by rand_vec, :98-103), the same
shapes and seeds, blocks taken from a fresh allocator and filled by the prefill
scatter (setup_kv_blocks, :186-231), and the same thresholds on max |fp16 - fp32|
and the cosine similarity of the two outputs.  Everything runs through the
reference-signature Python mirror over the C ABI.
"""
import numpy as np
import pytest
import torch

from lightllm_amd import kv_cache as kc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


class Lcg:
    """rng_state = rng_state * 1103515245 + 12345 (mod 2^32); rng_randf = (state & 0x7FFFFFFF) / 2^31."""

    def __init__(self, seed: int):
        self.state = seed & 0xFFFFFFFF

    def rand_vec(self, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        s = self.state
        for i in range(n):
            s = (s * 1103515245 + 12345) & 0xFFFFFFFF
            out[i] = np.float32(np.float32(s & 0x7FFFFFFF) / np.float32(2147483648.0)) * np.float32(2.0) - np.float32(1.0)
        self.state = s
        return out


def setup_kv_blocks(alloc: kc.BlockAllocator, k: np.ndarray, v: np.ndarray, seq_len: int):
    n_blocks = (seq_len + alloc.block_size - 1) // alloc.block_size
    ids = [alloc.allocate(0) for _ in range(n_blocks)]
    assert min(ids) >= 0, "block pool exhausted"
    bt = torch.tensor(ids, dtype=torch.int32, device=DEV)
    shape = (seq_len, alloc.num_kv_heads, alloc.head_dim)
    kt = torch.from_numpy(k).reshape(shape).to(alloc.kv_dtype).to(DEV)
    vt = torch.from_numpy(v).reshape(shape).to(alloc.kv_dtype).to(DEV)
    kc.scatter_prefill_kv(kt, vt, 0, seq_len, bt, n_blocks, alloc)
    torch.cuda.synchronize()
    return bt, n_blocks


def run_pair(seed, hq, hkv, d, seq_len, num_blocks, q_rows, mode, causal=True, num_splits=None):
    """The reference's fp32 run and fp16 run of one test; returns (fp32 out, fp16 out) as float64."""
    g = Lcg(seed)
    k = g.rand_vec(seq_len * hkv * d)
    v = g.rand_vec(seq_len * hkv * d)
    q = g.rand_vec(q_rows * hq * d)
    outs = []
    for dt in (torch.float32, torch.float16):
        alloc = kc.BlockAllocator(num_blocks, 16, hkv, d, kc.POLICY_HASH, dt, device=DEV)
        bt, nb = setup_kv_blocks(alloc, k, v, seq_len)
        qt = torch.from_numpy(q).reshape(q_rows, hq, d).to(dt).to(DEV)
        sl = torch.tensor([seq_len], dtype=torch.int32, device=DEV)
        if mode == "decode":
            if num_splits is None:
                o = kc.paged_attention(qt, bt, nb, sl, alloc)
            else:
                o = kc.paged_decode(qt, alloc.k_storage, alloc.v_storage, bt.view(1, -1), sl, seq_len,
                                    num_splits=num_splits)
        else:
            o = kc.prefill_paged_attention(qt, bt, nb, sl, alloc, causal=causal)
        torch.cuda.synchronize()
        outs.append(o.float().cpu().numpy().astype(np.float64).reshape(-1))
    return outs[0], outs[1]


def agree(ref, res, what, max_err_bar, cos_bar):
    max_err = float(np.abs(ref - res).max())
    cos = float(np.dot(ref, res) / (np.linalg.norm(ref) * np.linalg.norm(res)))
    print(f"  {what}: max_err={max_err:.6f} cos_sim={cos:.6f}", flush=True)
    assert np.all(np.isfinite(res)) and np.all(np.isfinite(ref))
    assert max_err < max_err_bar, f"{what}: max_err {max_err} >= {max_err_bar}"
    assert cos > cos_bar, f"{what}: cos_sim {cos} <= {cos_bar}"


# (name, seed, Hq, Hkv, D, seq_len, pool blocks, rows, mode, max_err bar, cos bar) as in the
# reference's tests 1-5 (:293-538); the Split-K case also runs with the reference's fixed
# SPLIT_K = 4 (paged_attention.cu:31).
CASES = [
    ("decode_baseline", 42, 2, 2, 64, 32, 8, 1, "decode", 0.01, 0.999, None),
    ("decode_v2", 99, 2, 2, 128, 32, 8, 1, "decode", 0.01, 0.999, None),
    ("decode_splitk", 777, 2, 2, 64, 512, 64, 1, "decode", 0.05, 0.995, None),
    ("decode_splitk_S4", 777, 2, 2, 64, 512, 64, 1, "decode", 0.05, 0.995, 4),
    ("prefill_paged", 123, 2, 2, 64, 32, 8, 32, "prefill", 0.01, 0.999, None),
    ("prefill_flash", 456, 2, 2, 64, 128, 32, 128, "prefill", 0.01, 0.999, None),
]


@pytest.mark.parametrize("name,seed,hq,hkv,d,seq_len,nb,rows,mode,err_bar,cos_bar,splits", CASES,
                         ids=[c[0] for c in CASES])
def test_fp16_pool_agrees_with_fp32_pool(name, seed, hq, hkv, d, seq_len, nb, rows, mode, err_bar,
                                         cos_bar, splits):
    ref, res = run_pair(seed, hq, hkv, d, seq_len, nb, rows, mode, num_splits=splits)
    agree(ref, res, name, err_bar, cos_bar)


def test_fp16_outputs_finite():
    """The reference's test 6 (:546-600): D=128 fp16 decode over 64 keys and a non-causal
    32-token prefill, every output element finite."""
    g = Lcg(888)
    hq = hkv = 2
    d = 128
    k = g.rand_vec(64 * hkv * d)
    v = g.rand_vec(64 * hkv * d)
    q = g.rand_vec(1 * hq * d)
    alloc = kc.BlockAllocator(16, 16, hkv, d, kc.POLICY_HASH, torch.float16, device=DEV)
    bt, nb = setup_kv_blocks(alloc, k, v, 64)
    o = kc.paged_attention(torch.from_numpy(q).reshape(1, hq, d).half().to(DEV), bt, nb,
                           torch.tensor([64], dtype=torch.int32, device=DEV), alloc)
    assert torch.isfinite(o.float()).all()
    k2 = g.rand_vec(32 * hkv * d)
    v2 = g.rand_vec(32 * hkv * d)
    q2 = g.rand_vec(32 * hq * d)
    alloc2 = kc.BlockAllocator(8, 16, hkv, d, kc.POLICY_HASH, torch.float16, device=DEV)
    bt2, nb2 = setup_kv_blocks(alloc2, k2, v2, 32)
    o2 = kc.prefill_paged_attention(torch.from_numpy(q2).reshape(32, hq, d).half().to(DEV), bt2, nb2,
                                    torch.tensor([32], dtype=torch.int32, device=DEV), alloc2,
                                    causal=False)
    torch.cuda.synchronize()
    assert torch.isfinite(o2.float()).all()
