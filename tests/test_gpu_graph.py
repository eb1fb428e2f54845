"""HIP-graph capture of the hot path: append, decode under each automatic schedule (balanced,
fixed splits + merge kernel, the 16-wave unit kernel, one split per unit) and chunked prefill
(device-side split decision + merge kernel) captured once and replayed.  Every replay follows
eager work that changes the inputs, and each replay's outputs must equal an eager call's on the
same inputs bit for bit: the kernels are deterministic, and no launch of the path records a
memset or allocates while captured."""
import pytest
import torch

from lightllm_amd import kv_cache as kc
from lightllm_amd import workloads as wl

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def say(msg):
    print(msg, flush=True)


def _decode_setup(name, B, hq, hkv, d, lengths, dtype, seed):
    need = sum((L + 1 + 15) // 16 for L in lengths)
    c = wl.decode_case(name, B, hq, hkv, d, lengths, need + 8, dtype, seed=seed)
    kp, vp = c.k_pool.to(DEV), c.v_pool.to(DEV)
    q = c.q.to(DEV)
    kn, vn, slots = c.k_new.to(DEV), c.v_new.to(DEV), c.slots.to(DEV)
    bt, sl = c.block_table.to(DEV), c.seq_lens.to(DEV)
    out = torch.empty_like(q)
    ws = torch.empty(kc.decode_workspace_bytes(B, hq, hkv, d, 16, c.max_seq_len, 0) or 1,
                     dtype=torch.uint8, device=DEV)

    def run(o):
        kc.append_kv(kn, vn, slots, kp, vp)
        kc.paged_decode(q, kp, vp, bt, sl, c.max_seq_len, out=o, workspace=ws)
    run.schedule = kc.decode_schedule(B, hq, hkv, d, c.max_seq_len, dtype)[0]
    return q, out, run


def _prefill_setup(name, hq, hkv, d, prefixes, chunks, dtype, seed):
    nb = sum((p + n + 15) // 16 for p, n in zip(prefixes, chunks)) + 4
    c = wl.prefill_case(name, hq, hkv, d, prefixes, chunks, {}, nb, dtype, seed=seed)
    kp, vp = c.k_pool.to(DEV), c.v_pool.to(DEV)
    kc.append_kv(c.k_chunk.to(DEV), c.v_chunk.to(DEV), c.slots.to(DEV), kp, vp)
    q = c.q.to(DEV)
    bt, cu, sl = c.block_table.to(DEV), c.cu_q.to(DEV), c.seq_lens.to(DEV)
    out = torch.empty_like(q)
    ws = torch.empty(max(1, kc.lib().llkv_paged_prefill_workspace_size(
        len(chunks), int(c.cu_q[-1]), c.max_q_len, c.max_seq_len, hq, d, 16, kc.dtype_code(dtype))),
        dtype=torch.uint8, device=DEV)

    def run(o):
        kc.paged_prefill(q, kp, vp, bt, cu, sl, c.max_q_len, c.max_seq_len, causal=True, out=o,
                         workspace=ws)
    return q, out, run


def test_graph_replays_match_eager():
    g = torch.Generator().manual_seed(77)
    lognormal = torch.exp(torch.randn(256, generator=g) + 6.0).clamp(16, 4096).int().tolist()
    setups = [
        # many uneven sequences: balanced schedule + its merge
        ("balanced", _decode_setup("g_bal", 256, 32, 8, 128, lognormal, torch.float16, 1)),
        # few long sequences: fixed splits + merge kernel
        ("split", _decode_setup("g_split", 4, 14, 2, 64, [6000, 3000, 9000, 100], torch.float32, 2)),
        # mid-size batch of mid contexts: 16-wave unit kernel
        ("unit", _decode_setup("g_unit", 24, 32, 8, 128, [700] * 24, torch.float16, 3)),
        # many short sequences: one split per unit on 4-wave work-groups
        ("onesplit", _decode_setup("g_one", 512, 14, 2, 64, [100] * 512, torch.bfloat16, 4)),
        # uneven cached prefixes: key chunks + merge kernel
        ("prefill_split", _prefill_setup("g_pf", 14, 2, 64, [0, 256, 1024, 4096, 2048, 512],
                                         [512] * 6, torch.float16, 5)),
        # even prefixes: the device drops the planned split, the merge kernel returns
        ("prefill_even", _prefill_setup("g_pfe", 14, 2, 64, [2048] * 2, [2048] * 2, torch.float16, 6)),
    ]
    # each decode setup runs the schedule it is named for
    for name, (q, out, run) in setups:
        if hasattr(run, "schedule"):
            say(f"{name}: schedule {run.schedule}")
            assert run.schedule == {"split": "splits", "onesplit": "one_split"}.get(name, name)
    # eager warm-up (library load, workspace first touch)
    for _, (q, out, run) in setups:
        run(out)
    torch.cuda.synchronize()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for _, (q, out, run) in setups:
                run(out)
    torch.cuda.synchronize()

    gen = torch.Generator(device=DEV).manual_seed(9)
    prev = [out.clone() for _, (q, out, run) in setups]
    for rep in range(3):
        # eager work between replays: new queries, and eager outputs for them
        refs = []
        for _, (q, out, run) in setups:
            q.copy_(torch.randn(q.shape, generator=gen, device=DEV, dtype=torch.float32).to(q.dtype))
            ref = torch.empty_like(out)
            run(ref)
            refs.append(ref)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for (name, (q, out, run)), ref in zip(setups, refs):
            same = torch.equal(out, ref)
            say(f"replay {rep} {name}: {'identical' if same else 'DIFFERS'}")
            assert same, f"replay {rep}: {name} differs from the eager call"
        # the replay recomputed: new queries give new outputs
        for i, (name, (q, out, run)) in enumerate(setups):
            assert not torch.equal(out, prev[i]), f"replay {rep}: {name} output unchanged"
            prev[i] = out.clone()
