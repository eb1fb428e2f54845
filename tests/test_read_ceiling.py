"""The read-ceiling kernels read exactly a decode batch's K and V rows.

bench.py's read ceiling (lightllm_amd/csrc/read_ceiling.hip, a measurement-only
library) bounds the decode by the time of reading the same bytes.  That bound
only holds if the kernels read those bytes and no others:

* CPU: bench.ceiling_items lists each (page, kv head) piece of the batch once,
  with the byte offset of its row 0 and the rows that hold tokens, as a
  brute-force walk of the block table gives them.
* GPU: with its checksum flag set (timed runs pass 0; the loads are the same
  code), each wave of the flat and the decode-structured kernels stores the XOR
  of every 32-bit word it loaded; the XOR over the waves must equal
  the host's XOR over exactly the batch's K and V rows (a missing or extra
  piece changes it).
"""
import numpy as np
import pytest
import torch

import bench
from lightllm_amd import workloads as wl


def _case(B, hkv, d, dtype, seed, lmax=700):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(0, lmax + 1, (B,), generator=g, dtype=torch.int32)
    lens[0] = 1
    lens[1 % B] = 16
    lens[2 % B] = 17
    mb = max(1, (int(lens.max()) + 15) // 16)
    nb = int(sum((int(L) + 15) // 16 for L in lens)) + 5
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    table, _ = wl._tables([int(L) for L in lens], perm, mb)
    return lens, table, nb


def _pieces_brute(table, lens, hkv, piece):
    """(byte offset of row 0, rows) of every (sequence, page, kv head) piece, by walking the table."""
    out = []
    row = piece * hkv
    for b in range(table.shape[0]):
        L = int(lens[b])
        for p in range((L + 15) // 16):
            phys = int(table[b, p])
            for kvh in range(hkv):
                out.append((phys * 16 * row + kvh * piece, min(16, L - 16 * p)))
    return out


@pytest.mark.parametrize("B,hkv,d,esize", [(9, 2, 64, 4), (5, 8, 128, 2), (3, 1, 256, 2)])
def test_ceiling_items_list_each_piece_once(B, hkv, d, esize):
    lens, table, _ = _case(B, hkv, d, None, seed=B * 7 + hkv)
    piece = d * esize
    items = bench.ceiling_items(torch, table, lens, hkv, piece, "cpu").numpy()
    got = [(int(x) >> 5, int(x) & 31) for x in items]
    assert got == _pieces_brute(table.numpy(), lens.numpy(), hkv, piece)
    assert all(1 <= r <= 16 for _, r in got)


def _host_xor(k, v, table, lens):
    """XOR of the 32-bit words of the batch's K and V rows (pools [nb, 16, Hkv, D])."""
    acc = np.uint32(0)
    for pool in (k, v):
        words = pool.view(np.uint32).reshape(pool.shape[0], 16, -1)   # [page, row, Hkv*D words]
        for b in range(table.shape[0]):
            L = int(lens[b])
            for p in range((L + 15) // 16):
                rows = words[int(table[b, p]), : min(16, L - 16 * p)]
                acc ^= np.bitwise_xor.reduce(rows, axis=None)
    return acc


@pytest.mark.gpu
@pytest.mark.parametrize("B,hkv,d,dtype", [(12, 2, 64, torch.float32), (6, 8, 128, torch.float16),
                                           (4, 2, 64, torch.float16), (3, 1, 256, torch.bfloat16)])
def test_ceiling_kernels_read_exactly_the_batch_rows(B, hkv, d, dtype):
    print(f"read ceiling checksum B={B} Hkv={hkv} D={d} {dtype}", flush=True)
    lens, table, nb = _case(B, hkv, d, dtype, seed=B + d)
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(3)
    k = torch.randn(nb, 16, hkv, d, generator=g).to(dtype)
    v = torch.randn(nb, 16, hkv, d, generator=g).to(dtype)
    want = _host_xor(k.contiguous().view(torch.int16 if dtype != torch.float32 else torch.int32).numpy(),
                     v.contiguous().view(torch.int16 if dtype != torch.float32 else torch.int32).numpy(),
                     table.numpy(), lens.numpy())
    kd, vd = k.to(dev), v.to(dev)
    esize, piece = k.element_size(), d * k.element_size()
    lib = bench._ceiling_lib()
    nwg = lib.llkv_rc_flat_resident(piece)
    assert nwg > 0
    items = bench.ceiling_items(torch, table, lens, hkv, piece, dev)
    tb, ln = table.to(dev), lens.to(dev)
    st = torch.cuda.current_stream().cuda_stream
    for splits in (0, 1, 3):   # 0: the flat kernel; S > 0: the decode-structured one
        nsink = 4 * (nwg if splits == 0 else splits * hkv * B)   # one word per wave
        sink = torch.full((nsink,), -1, dtype=torch.int32, device=dev)
        if splits == 0:
            rc = lib.llkv_rc_flat(kd.data_ptr(), vd.data_ptr(), items.data_ptr(), int(items.numel()), piece,
                                  piece * hkv, nwg, sink.data_ptr(), 1, st)
        else:
            rc = lib.llkv_rc_chain(kd.data_ptr(), vd.data_ptr(), tb.data_ptr(), ln.data_ptr(), tb.shape[1], B,
                                   hkv, splits, piece, sink.data_ptr(), 1, st)
        assert rc == 0
        torch.cuda.synchronize()
        got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
        assert got == want, f"splits={splits}: checksum {got:#x} against {want:#x}"
    # bench.py's own calls of the kernels run on the same inputs
    _, (flat, chain) = bench.read_ceiling(torch, [(kd, vd)], table, lens, hkv, d, esize, 3, 1, timed=False)
    flat(0)
    chain(0)
    torch.cuda.synchronize()
