"""Benchmark of the paged KV-cache hot path on one MI355X.

Headline metric: paged decode at B=64, configuration 2 --
Qwen2.5-0.5B attention (14 q / 2 kv heads, head_dim 64), fp32, contexts
U[128, 2048], pool 32768 pages.  One step = one layer of a decode step: KV
append of the 64 new tokens by slot mapping, then paged decode attention
over the updated tables, as the one call an engine makes
(llkv_paged_decode_append; its results equal llkv_append then
llkv_paged_decode bit for bit, and that two-call step is reported beside it).  Steps rotate over --layers independent K/V pools
(one per layer, as in a model), so the KV bytes of a step are not resident
in the 256 MB last-level cache from the previous step.

Reported: value = achieved algorithmic HBM GB/s of paged decode (exact
tokens; HIP events around a HIP-graph replay of --steps decode calls),
us per layer (graph replay of --steps append + decode steps), the decode
roofline fraction, the CPU baseline (the C oracle = the reference's
reconstruct_kv + cpu_attention, on this host), and configuration 4's paged
prefill as MFMA utilisation.

  python bench.py [--gpus 1] [--steps 200] [--warmup 20]

Profiling helpers (the commands that produce the summaries under profiles/):
  python bench.py --calibrate-copy          a plain 256 MiB device copy, the
                                            reference point for FETCH_SIZE /
                                            WRITE_SIZE scaling
  python bench.py --rocprof-summary DIR     per-kernel averages of the rocprofv3
                                            CSV files (kernel trace, counters)
                                            found under DIR
  python bench.py --rocprof-traffic FETCH_DIR WRITE_DIR CAL_FETCH_DIR CAL_WRITE_DIR
                                            HBM bytes per call of the library's
                                            kernels from FETCH_SIZE / WRITE_SIZE
                                            runs of a --profile-target and of
                                            --calibrate-copy
  python bench.py --rocprof-mfma DIR        MFMA busy % of the prefill kernels from
                                            an SQ_VALU_MFMA_BUSY_CYCLES +
                                            GRBM_GUI_ACTIVE counter run
  python bench.py --profile-target NAME     eager calls of one workload (cfg2_decode,
                                            cfg3_decode, cfg5_decode, cfg4_prefill,
                                            cfg5_prefill, ceiling_cfg2/3/5) for rocprofv3
  python bench.py --read-ceiling CFG        read ceiling of decode configuration CFG
                                            (cfg2, cfg3, cfg5) beside its decode

Read ceiling: measurement-only kernels (lightllm_amd/csrc/read_ceiling.hip, their
own library) read exactly a decode batch's K/V rows -- the same page ids, the
same (page, kv head) pieces, the same rotated pools, HIP-graph replays -- and
nothing else.  Their time bounds any decode of that batch on this GPU;
roofline.frac_of_ceiling = ceiling time / decode time.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
COPY_CAL_BYTES = 256 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_cfg2_traffic.txt")
FP16_MFMA_PEAK_TFLOPS = 2500.0
FP32_MFMA_PEAK_TFLOPS = 157.3
METRIC = "paged decode µs/layer + achieved HBM GB/s (% peak) at B=64; prefill MFMA %"


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it, with family / model / stepping (a virtualised
    host may report a generic model name)."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" in line:
                    k, v = line.split(":", 1)
                    info.setdefault(k.strip(), v.strip())
                if not line.strip() and info:
                    break
    except OSError:
        pass
    name = info.get("model name") or platform.processor() or "unknown"
    extra = ", ".join(f"{k} {info[k]}" for k in ("cpu family", "model", "stepping") if k in info)
    return f"{name} ({extra})" if extra else name


def cpu_threads() -> int:
    """Host threads this process may use (the affinity mask; the GPU box gives a job 16)."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def bench_decode(args, torch, kc, wl):
    dev = torch.device("cuda:0")
    case = wl.config2()
    L = args.layers
    B, hq, d = case.q.shape
    hkv = case.k_pool.shape[2]
    nb = case.k_pool.shape[0]
    # layer 0 pools = the host-generated case; other layers: device-generated pools
    kps, vps = [case.k_pool.to(dev)], [case.v_pool.to(dev)]
    for layer in range(1, L):
        k, v = wl.device_pools(nb, hkv, d, torch.float32, 100 + layer, dev)
        kps.append(k)
        vps.append(v)
    g = torch.Generator().manual_seed(77)
    qs = [case.q.to(dev)] + [torch.randn(B, hq, d, generator=g).to(dev) for _ in range(1, L)]
    kn = [case.k_new.to(dev)] + [torch.randn(B, hkv, d, generator=g).to(dev) for _ in range(1, L)]
    vn = [case.v_new.to(dev)] + [torch.randn(B, hkv, d, generator=g).to(dev) for _ in range(1, L)]
    table = case.block_table.to(dev)
    lens = case.seq_lens.to(dev)
    slots = case.slots.to(dev)
    outs = [torch.empty_like(q) for q in qs]
    max_len = case.max_seq_len
    ws = kc._workspace(kc.decode_workspace_bytes(B, hq, hkv, d, 16, max_len), dev)
    stream = torch.cuda.current_stream()

    def step(i, ev=None):
        layer = i % L
        kc.append_kv(kn[layer], vn[layer], slots, kps[layer], vps[layer])
        if ev is not None:
            ev[0].record(stream)
        kc.paged_decode(qs[layer], kps[layer], vps[layer], table, lens, max_len, out=outs[layer],
                        workspace=ws)
        if ev is not None:
            ev[1].record(stream)

    def decode_only(i):
        layer = i % L
        kc.paged_decode(qs[layer], kps[layer], vps[layer], table, lens, max_len, out=outs[layer],
                        workspace=ws)

    def step_fused(i):   # the same append + decode as one llkv_paged_decode_append call
        layer = i % L
        kc.paged_decode_append(qs[layer], kn[layer], vn[layer], kps[layer], vps[layer], table, lens,
                               max_len, out=outs[layer], workspace=ws)

    for i in range(args.warmup):
        step(i)
        step_fused(i)
    torch.cuda.synchronize()

    # The timed loops run as HIP graph replays (one launch for K steps), the way a
    # serving loop issues them: per-call host work (Python, ctypes) is outside.
    def replay_us(fn, k):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                for i in range(k):
                    fn(i)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        cur = torch.cuda.current_stream()
        t0.record(cur)
        graph.replay()
        t1.record(cur)
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) * 1e3 / k

    step_us = replay_us(step, args.steps)
    dec_us = replay_us(decode_only, args.steps)
    fused_us = replay_us(step_fused, args.steps)
    sched = kc.decode_schedule(B, hq, hkv, d, max_len, torch.float32)
    ceiling, _ = read_ceiling(torch, list(zip(kps, vps)), table, lens, hkv, d, 4,
                              sched[1] if sched[0] == "splits" else 0, args.steps)

    # Eager loop with HIP events around each decode call (host-launch gaps included).
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    torch.cuda.synchronize()
    for i in range(args.steps):
        step(i, evs[i])
    torch.cuda.synchronize()
    eager_us = [a_.elapsed_time(b_) * 1e3 for a_, b_ in evs]

    # correctness spot check of layer 0 against the oracle (double)
    import numpy as np
    import oracle
    ke, ve = case.k_pool.numpy().copy(), case.v_pool.numpy().copy()
    oracle.append_slots(ke, ve, case.k_new.numpy(), case.v_new.numpy(), case.slots.numpy())
    ref = oracle.paged_decode(case.q.numpy(), ke, ve, case.block_table.numpy(),
                              case.seq_lens.numpy(), f64=True, nthreads=min(16, os.cpu_count() or 1))
    got = outs[0].cpu().numpy().astype(np.float64)
    err = np.abs(got - ref)
    ok = bool(np.all(err <= 1e-6 + 1e-5 * np.abs(ref)))

    dec_bytes = wl.decode_bytes(case)
    dec_bytes_pages = wl.decode_bytes(case, exact_tokens=False)
    app_bytes = wl.append_bytes(case)
    return {
        "case": case, "host_pools": (ke, ve), "step_ms": fused_us / 1e3, "step_two_calls_us": step_us,
        "decode_us_mean": dec_us, "decode_us_eager_median": statistics.median(eager_us),
        "decode_bytes": dec_bytes, "decode_bytes_pages": dec_bytes_pages, "append_bytes": app_bytes,
        "pool_bytes": 2 * kps[0].numel() * kps[0].element_size(),
        "parity_ok": ok, "max_abs_err": float(err.max()),
        "schedule": sched, "ceiling": ceiling,
    }


def bench_prefill(args, torch, kc, wl, dtype=None):
    dev = torch.device("cuda:0")
    case = wl.config4() if dtype is None else wl.config4(dtype=dtype)
    kp, vp = case.k_pool.to(dev), case.v_pool.to(dev)
    kc.append_kv(case.k_chunk.to(dev), case.v_chunk.to(dev), case.slots.to(dev), kp, vp)
    q = case.q.to(dev)
    bt, cu, sl = case.block_table.to(dev), case.cu_q.to(dev), case.seq_lens.to(dev)
    out = torch.empty_like(q)
    run = lambda: kc.paged_prefill(q, kp, vp, bt, cu, sl, case.max_q_len, case.max_seq_len,
                                   causal=True, out=out)
    for _ in range(5):
        run()
    torch.cuda.synchronize()
    us = _graph_us(torch, lambda i: run(), max(20, args.steps // 4))
    flops = wl.prefill_flops(case)
    tflops = flops / (us * 1e-6) / 1e12
    peak = FP32_MFMA_PEAK_TFLOPS if case.q.dtype == torch.float32 else FP16_MFMA_PEAK_TFLOPS
    return {"us": us, "flop": flops, "tflops": tflops, "mfma_frac": tflops / peak}


def _graph_us(torch, fn, n, warm_replays=3, timed_replays=5):
    """Per-call time of fn over a HIP graph of n calls: warm replays, then the
    median of timed replays (each bracketed by HIP events on the launch stream)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for i in range(n):
                fn(i)
    torch.cuda.synchronize()
    for _ in range(warm_replays):
        graph.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(timed_replays):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        graph.replay()
        b.record()
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b) * 1e3 / n)
    return statistics.median(times)


CEIL_LIB = os.path.join(ROOT, "lightllm_amd", "liblightllm_kv_ceiling.so")
_ceil = None


def _ceiling_lib():
    """The measurement-only read-ceiling kernels (lightllm_amd/csrc/read_ceiling.hip)."""
    global _ceil
    if _ceil is None:
        import ctypes
        from ctypes import c_int, c_int64, c_void_p
        if not os.path.exists(CEIL_LIB):
            raise SystemExit(f"{CEIL_LIB} is missing: run __graft_entry__.build()")
        lib = ctypes.CDLL(CEIL_LIB)
        lib.llkv_rc_flat.argtypes = [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int64, c_int, c_void_p,
                                     c_int, c_void_p]
        lib.llkv_rc_chain.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                      c_int, c_void_p, c_int, c_void_p]
        lib.llkv_rc_flat_resident.argtypes = [c_int]
        _ceil = lib
    return _ceil


def ceiling_items(torch, table, lens, hkv, piece_bytes, dev):
    """The batch's (page, kv head) pieces in the pool, in decode order (sequence, page, kv
    head): int64 (byte offset of the piece's row 0) << 5 | rows holding tokens."""
    import numpy as np
    t = table.cpu().numpy().astype(np.int64)
    L = lens.cpu().numpy().astype(np.int64)
    row = piece_bytes * hkv
    items = []
    for b in range(t.shape[0]):
        n = int((L[b] + 15) // 16)
        if n == 0:
            continue
        p = np.arange(n)
        rows = np.minimum(16, L[b] - 16 * p)
        base = t[b, :n] * 16 * row
        it = ((base[:, None] + np.arange(hkv)[None, :] * piece_bytes) << 5) | rows[:, None]
        items.append(it.reshape(-1))
    return torch.from_numpy(np.concatenate(items)).to(dev)


def read_ceiling(torch, pools, table, lens, hkv, d, esize, splits, calls, timed=True):
    """Per-call time of the read-ceiling kernels over a batch's exact pages, HIP-graph replays of
    `calls` calls rotating over `pools` [(k, v)], as the decode benches run: 'flat' (pure read
    of the (page, kv head) pieces, one resident set of work-groups) and, for splits > 0,
    'chain' (the fixed-split decode's length -> table -> page walk on 4-wave work-groups, no
    arithmetic; reported for the fixed-split schedule only)."""
    lib = _ceiling_lib()
    dev = pools[0][0].device
    piece = d * esize
    items = ceiling_items(torch, table, lens, hkv, piece, dev)
    nwg = lib.llkv_rc_flat_resident(piece)
    if nwg <= 0:
        raise RuntimeError("read ceiling: no resident work-groups")
    tb, ln = table.to(dev), lens.to(dev)
    # one checksum word per wave (4 per work-group) of either kernel
    sink = torch.zeros(4 * max(nwg, max(splits, 1) * hkv * tb.shape[0]), dtype=torch.int32, device=dev)
    res = {"pieces": int(items.numel()), "workgroups": nwg}

    def flat(i):
        k, v = pools[i % len(pools)]
        st = torch.cuda.current_stream().cuda_stream
        rc = lib.llkv_rc_flat(k.data_ptr(), v.data_ptr(), items.data_ptr(), int(items.numel()), piece,
                              piece * hkv, nwg, sink.data_ptr(), 0, st)
        assert rc == 0, rc

    def chain(i):
        k, v = pools[i % len(pools)]
        st = torch.cuda.current_stream().cuda_stream
        rc = lib.llkv_rc_chain(k.data_ptr(), v.data_ptr(), tb.data_ptr(), ln.data_ptr(), tb.shape[1],
                               tb.shape[0], hkv, splits, piece, sink.data_ptr(), 0, st)
        assert rc == 0, rc

    if not timed:   # the calls only (rocprofv3 runs)
        return res, (flat, chain)
    for i in range(2 * len(pools)):
        flat(i)
    torch.cuda.synchronize()
    res["flat_us"] = _graph_us(torch, flat, calls)
    if splits > 0:
        res["chain_us"] = _graph_us(torch, chain, calls)
        res["chain_splits"] = splits
    return res, (flat, chain)


def ceiling_setup(torch, kc, wl, name):
    """Pools, tables and the decode call of one decode configuration, as the main bench builds
    them (configuration 2: 8 layer pools; 3: 2; 5: its one 262144-page pool)."""
    dev = torch.device("cuda:0")
    if name == "cfg5":
        case = wl.config5().decode
        pools = [wl.device_pools(262144, 8, 128, torch.float16, 55, dev)]
    else:
        case = wl.config2() if name == "cfg2" else wl.config3()
        nb, hkv, d = case.k_pool.shape[0], case.k_pool.shape[2], case.k_pool.shape[3]
        layers = 8 if name == "cfg2" else 2
        pools = [wl.device_pools(nb, hkv, d, case.k_pool.dtype, 100 + i, dev) for i in range(layers)]
    B, hq, d = case.q.shape
    hkv = pools[0][0].shape[2]
    q, bt, sl = case.q.to(dev), case.block_table.to(dev), case.seq_lens.to(dev)
    out = torch.empty_like(q)
    ml = case.max_seq_len
    ws = kc._workspace(kc.decode_workspace_bytes(B, hq, hkv, d, 16, ml), dev)
    dec = lambda i: kc.paged_decode(q, pools[i % len(pools)][0], pools[i % len(pools)][1], bt, sl, ml,
                                    out=out, workspace=ws)
    sched = kc.decode_schedule(B, hq, hkv, d, ml, case.q.dtype)
    return {"case": case, "pools": pools, "table": bt, "lens": sl, "hkv": hkv, "d": d,
            "esize": case.q.element_size(), "decode": dec, "bytes": wl.decode_bytes(case),
            "schedule": sched, "splits": sched[1] if sched[0] == "splits" else 0}


def ceiling_fields(rc, decode_us, nbytes):
    """Bench-line fields of a read-ceiling result: the ceiling as a rate over the decode's own
    algorithmic bytes, and the decode's fraction of it (ceiling time / decode time)."""
    out = {"ceiling_us": round(rc["flat_us"], 2),
           "ceiling_GBps": round(nbytes / (rc["flat_us"] * 1e-6) / 1e9, 1),
           "frac_of_ceiling": round(rc["flat_us"] / decode_us, 4)}
    if "chain_us" in rc:
        out["chain_ceiling_us"] = round(rc["chain_us"], 2)
        out["chain_splits"] = rc["chain_splits"]
    return out


def read_ceiling_mode(torch, kc, wl, name, calls):
    """--read-ceiling NAME: the read ceiling of one decode configuration and its decode, HIP-graph
    replays of `calls` calls over the same rotated pools; one JSON line."""
    st = ceiling_setup(torch, kc, wl, name)
    for i in range(3):
        st["decode"](i)
    torch.cuda.synchronize()
    dec_us = _graph_us(torch, st["decode"], calls)
    rc, _ = read_ceiling(torch, st["pools"], st["table"], st["lens"], st["hkv"], st["d"], st["esize"],
                         st["splits"], calls)
    line = {"read_ceiling": name, "decode_us": round(dec_us, 2),
            "decode_GBps": round(st["bytes"] / (dec_us * 1e-6) / 1e9, 1),
            "decode_schedule": list(st["schedule"]), "bytes_per_call": st["bytes"],
            "pieces": rc["pieces"], "workgroups": rc["workgroups"], "pools_rotated": len(st["pools"])}
    line.update(ceiling_fields(rc, dec_us, st["bytes"]))
    print(json.dumps(line), flush=True)


def bench_other_configs(torch, kc, wl):
    """Configurations 3 and 5 (decode HBM rate, prefill MFMA rate), HIP-graph replays."""
    dev = torch.device("cuda:0")
    res = {}
    c1 = wl.config1()
    q1, bt1, sl1 = c1.q.to(dev), c1.block_table.to(dev), c1.seq_lens.to(dev)
    kp1, vp1 = c1.k_pool.to(dev), c1.v_pool.to(dev)
    o1 = torch.empty_like(q1)
    us1 = _graph_us(torch, lambda i: kc.paged_decode(q1, kp1, vp1, bt1, sl1, c1.max_seq_len, out=o1), 50)
    res["cfg1_decode"] = {"us": round(us1, 2), "GBps": round(wl.decode_bytes(c1) / (us1 * 1e-6) / 1e9, 1)}
    c3 = wl.config3()
    pools = [wl.device_pools(c3.k_pool.shape[0], 2, 64, torch.float16, 30 + i, dev) for i in range(2)]
    q, bt, sl = c3.q.to(dev), c3.block_table.to(dev), c3.seq_lens.to(dev)
    out = torch.empty_like(q)
    for S in (0, 16):
        us = _graph_us(torch, lambda i: kc.paged_decode(q, pools[i % 2][0], pools[i % 2][1], bt, sl,
                                                       c3.max_seq_len, num_splits=S, out=out), 20)
        res[f"cfg3_decode_S{S}"] = {"us": round(us, 2),
                                    "GBps": round(wl.decode_bytes(c3) / (us * 1e-6) / 1e9, 1),
                                    "GBps_page_granular": round(wl.decode_bytes(c3, exact_tokens=False)
                                                                / (us * 1e-6) / 1e9, 1)}
        if S == 0:
            s3 = kc.decode_schedule(c3.q.shape[0], c3.q.shape[1], 2, 64, c3.max_seq_len, torch.float16)
            rc3, _ = read_ceiling(torch, pools, bt, sl, 2, 64, 2,
                                  s3[1] if s3[0] == "splits" else 0, 20)
            res["cfg3_decode_S0"]["schedule"] = list(s3)
            res["cfg3_decode_S0"].update(ceiling_fields(rc3, us, wl.decode_bytes(c3)))
    del pools
    m5 = wl.config5()
    dec, pre = m5.decode, m5.prefill
    kp, vp = wl.device_pools(262144, 8, 128, torch.float16, 55, dev)
    dq, dbt, dsl = dec.q.to(dev), dec.block_table.to(dev), dec.seq_lens.to(dev)
    kn, vn, dsl_slots = dec.k_new.to(dev), dec.v_new.to(dev), dec.slots.to(dev)
    pq, pbt, pcu, psl = pre.q.to(dev), pre.block_table.to(dev), pre.cu_q.to(dev), pre.seq_lens.to(dev)
    pk, pv, pslots = pre.k_chunk.to(dev), pre.v_chunk.to(dev), pre.slots.to(dev)
    dout, pout = torch.empty_like(dq), torch.empty_like(pq)

    def step(i):
        kc.append_kv(kn, vn, dsl_slots, kp, vp)
        kc.append_kv(pk, pv, pslots, kp, vp)
        kc.paged_decode(dq, kp, vp, dbt, dsl, dec.max_seq_len, out=dout)
        kc.paged_prefill(pq, kp, vp, pbt, pcu, psl, pre.max_q_len, pre.max_seq_len, True, out=pout)

    # 20 calls per graph, so that the replay's start-up cost is spread thin
    n5 = 20
    step_us = _graph_us(torch, step, n5)
    dec_us = _graph_us(torch, lambda i: kc.paged_decode(dq, kp, vp, dbt, dsl, dec.max_seq_len, out=dout), n5)
    pre_us = _graph_us(torch, lambda i: kc.paged_prefill(pq, kp, vp, pbt, pcu, psl, pre.max_q_len,
                                                         pre.max_seq_len, True, out=pout), n5)
    pf = wl.prefill_flops(pre)
    rc5, _ = read_ceiling(torch, [(kp, vp)], dbt, dsl, 8, 128, 2, 0, n5)
    res["cfg5_step"] = {"us": round(step_us, 1), "decode_us": round(dec_us, 1),
                        "decode_GBps": round(wl.decode_bytes(dec) / (dec_us * 1e-6) / 1e9, 1),
                        "decode_GBps_page_granular": round(wl.decode_bytes(dec, exact_tokens=False)
                                                           / (dec_us * 1e-6) / 1e9, 1),
                        "decode_ceiling": ceiling_fields(rc5, dec_us, wl.decode_bytes(dec)),
                        "prefill_us": round(pre_us, 1),
                        "prefill_mfma_frac": round(pf / (pre_us * 1e-6) / 1e12 / FP16_MFMA_PEAK_TFLOPS, 4)}
    res["rope_append_cfg5_step"] = bench_rope_append(torch, kc, dec, pre, kp, vp, dsl_slots, pslots)
    del kp, vp
    res["first_prefill_fp32_8x512"] = bench_first_prefill(torch, kc)
    return res


def bench_first_prefill(torch, kc):
    """Batched first prefill as EngineServer::step issues it (fp32, contiguous K/V): 8 entries
    of 512 tokens, Qwen2.5-0.5B heads (14/2/64), causal within each entry."""
    import numpy as np
    dev = torch.device("cuda:0")
    hq, hkv, d, ntok = 14, 2, 64, [512] * 8
    n = len(ntok)
    cum = np.concatenate([[0], np.cumsum(ntok)]).astype(np.int32)
    ptot = int(cum[-1])
    g = torch.Generator(device="cpu").manual_seed(8)
    q, k, v = (torch.randn(ptot, h, d, generator=g).to(dev) for h in (hq, hkv, hkv))
    out = torch.empty_like(q)
    t32 = lambda a: torch.as_tensor(a, dtype=torch.int32).to(dev)
    args = (out, q, k, v, hq, hkv, d, t32(cum[:-1] * hq * d), t32(cum[:-1] * hkv * d), t32(ntok),
            t32(cum), t32(np.zeros(n)), n, ptot, 1.0 / math.sqrt(d))
    us = _graph_us(torch, lambda i: kc.first_prefill_attn_batched(*args, max_tokens=max(ntok)), 10)
    flops = sum(p * (p + 1) / 2 for p in ntok) * 4 * d * hq
    tf = flops / (us * 1e-6) / 1e12
    return {"us": round(us, 1), "TFLOPs": round(tf, 1), "mfma_frac_of_fp32_peak": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)}


def rope_append_bytes(T, hq, hkv, d, rot, esize):
    """Algorithmic bytes of one llkv_rope_append call: q and k read + written in place, k and v
    rows written to the pool, v read, cos / sin and the int64 slots read once."""
    return (T * hq * d * esize * 2 + T * hkv * d * esize * 2 + T * hkv * d * esize * 3
            + T * (rot // 2) * 4 * 2 + T * 8)


def bench_rope_append(torch, kc, dec, pre, kp, vp, dec_slots, pre_slots):
    """Fused RoPE + KV append over configuration 5's step tokens (256 decode tokens + 4 x 1024
    prefill tokens, 32/8/128 fp16) into its 262144-page pool; HIP-graph replays.  The CPU
    baseline is the oracle's restatement (rotate q and k, then the row copies), 1 thread."""
    import numpy as np
    import oracle
    dev = torch.device("cuda:0")
    hq, d = dec.q.shape[1], dec.q.shape[2]
    hkv = kp.shape[2]
    T = dec.q.shape[0] + pre.q.shape[0]
    g = torch.Generator(device=dev).manual_seed(77)
    q = torch.randn(T, hq, d, generator=g, device=dev).to(torch.float16)
    k = torch.randn(T, hkv, d, generator=g, device=dev).to(torch.float16)
    v = torch.randn(T, hkv, d, generator=g, device=dev).to(torch.float16)
    slots = torch.cat([dec_slots, pre_slots])
    pos = torch.cat([dec.seq_lens.double() - 1,
                     torch.cat([torch.arange(int(L) - n, int(L)).double() for L, n in
                                zip(pre.seq_lens.tolist(), (pre.cu_q[1:] - pre.cu_q[:-1]).tolist())])])
    inv = 1.0 / (500000.0 ** (torch.arange(d // 2).double() * 2.0 / d))
    ang = pos[:, None] * inv[None, :]
    cos, sin = torch.cos(ang).float().to(dev), torch.sin(ang).float().to(dev)
    us = _graph_us(torch, lambda i: kc.rope_append(q, k, v, slots, cos, sin, kp, vp), 20)
    nbytes = rope_append_bytes(T, hq, hkv, d, d, 2)
    gbps = nbytes / (us * 1e-6) / 1e9
    # CPU baseline: the oracle on the same tokens into a host pool of the touched pages only
    qh = q.cpu().view(torch.int16).numpy().view(np.uint16).copy()
    kh = k.cpu().view(torch.int16).numpy().view(np.uint16).copy()
    vh = v.cpu().view(torch.int16).numpy().view(np.uint16).copy()
    sl = slots.cpu().numpy()
    rows = np.unique(sl[sl >= 0])
    remap = np.full(int(sl.max()) + 1, -1, dtype=np.int64)
    remap[rows] = np.arange(rows.size)
    hs = remap[sl]
    pool = np.zeros(((rows.size + 15) // 16, 16, hkv, d), np.uint16)
    ch, sh = cos.cpu().numpy(), sin.cpu().numpy()
    times = []
    for _ in range(5):
        qq, kk = qh.copy(), kh.copy()
        t0 = time.perf_counter()
        oracle.rope_append(qq, kk, vh, pool, pool.copy(), hs, ch, sh, 1)
        times.append(time.perf_counter() - t0)
    cpu_us = statistics.median(times) * 1e6
    return {"tokens": T, "us": round(us, 2), "bytes": nbytes, "GBps": round(gbps, 1),
            "roofline_frac": round(gbps / HBM_PEAK_GBS, 4),
            "cpu_baseline": {"us": round(cpu_us, 1), "GBps": round(nbytes / (cpu_us * 1e-6) / 1e9, 2),
                             "cores": 1, "kind": "port",
                             "sample": "the same tokens, oracle rope_append (fp16 via fp32), median of 5"}}


def cpu_baseline(dec, budget_s: float):
    """The oracle (reference CPU path restated in C: reconstruct_kv + cpu_attention) on
    configuration 2's layer-0 inputs, 1 thread, median of >= 5 runs after one warmup."""
    import numpy as np
    import oracle
    case = dec["case"]
    ke, ve = dec["host_pools"]
    q = case.q.numpy()
    bt, sl = case.block_table.numpy(), case.seq_lens.numpy()
    args = (q, ke, ve, bt, sl)
    oracle.paged_decode(*args, nthreads=1)
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - t_start < budget_s and len(times) < 50):
        t = time.perf_counter()
        oracle.paged_decode(*args, nthreads=1)
        times.append(time.perf_counter() - t)
    med = statistics.median(times)
    nthr = cpu_threads()
    tt = []
    for _ in range(5):
        t = time.perf_counter()
        oracle.paged_decode(*args, nthreads=nthr)
        tt.append(time.perf_counter() - t)
    med_n = statistics.median(tt)
    gbs = dec["decode_bytes"] / med / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"configuration 2 decode (64 seqs, 14/2/64 fp32), whole batch per run, "
                      f"median of {len(times)} runs: {med * 1e6:.0f} us/layer",
            "us_per_layer": round(med * 1e6, 1),
            "threads_all": {"threads": nthr, "us_per_layer": round(med_n * 1e6, 1),
                            "GB/s": round(dec["decode_bytes"] / med_n / 1e9, 3)},
            "cpu_model": cpu_model(), "nproc": os.cpu_count()}


def _time_cpu(fn, runs_min: int, budget_s: float):
    fn()   # warm-up (page-in, thread start)
    times = []
    t_start = time.perf_counter()
    while len(times) < runs_min or (time.perf_counter() - t_start < budget_s and len(times) < 50):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return statistics.median(times), len(times)


def cpu_baseline_prefill(torch, wl, budget_s: float):
    """The oracle's paged prefill (the reference's cpu_prefill_attention_causal,
    tests/test_paged_prefill.cu:164-210, restated in C) on configuration 4's whole batch:
    1 thread (as the reference) and every thread of the host, median of >= 3 runs."""
    import numpy as np
    import oracle
    c = wl.config4()
    kp, vp = c.k_pool.float().numpy(), c.v_pool.float().numpy()
    oracle.append_slots(kp, vp, c.k_chunk.float().numpy(), c.v_chunk.float().numpy(), c.slots.numpy())
    args = (c.q.float().numpy(), c.cu_q.numpy(), kp, vp, c.block_table.numpy(), c.seq_lens.numpy(), True)
    flops = wl.prefill_flops(c)
    t1, n1 = _time_cpu(lambda: oracle.paged_prefill(*args, nthreads=1), 3, budget_s)
    nthr = cpu_threads()
    tn, nn = _time_cpu(lambda: oracle.paged_prefill(*args, nthreads=nthr), 3, budget_s / 3)
    return {"value": round(flops / t1 / 1e9, 3), "unit": "GFLOP/s", "cores": 1, "kind": "port",
            "sample": f"configuration 4's whole batch (8 x 512 causal rows on cached prefixes, "
                      f"14/2/64 fp16 widened to fp32), median of {n1} runs: {t1 * 1e6:.0f} us",
            "us": round(t1 * 1e6, 1),
            "threads_all": {"threads": nthr, "us": round(tn * 1e6, 1),
                            "GFLOP/s": round(flops / tn / 1e9, 3), "runs": nn},
            "cpu_model": cpu_model(), "nproc": os.cpu_count()}


def cpu_baseline_decode_cfg3(torch, wl, budget_s: float):
    """The oracle's decode (reconstruct_kv + cpu_attention) on configuration 3 (16 x 32768
    tokens, fp16 K/V widened to fp32): 1 thread and every host thread."""
    import oracle
    c = wl.config3()
    args = (c.q.float().numpy(), c.k_pool.float().numpy(), c.v_pool.float().numpy(),
            c.block_table.numpy(), c.seq_lens.numpy())
    nbytes = wl.decode_bytes(c)
    t1, n1 = _time_cpu(lambda: oracle.paged_decode(*args, nthreads=1), 3, budget_s)
    nthr = cpu_threads()
    tn, nn = _time_cpu(lambda: oracle.paged_decode(*args, nthreads=nthr), 3, budget_s / 3)
    return {"value": round(nbytes / t1 / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"configuration 3's whole batch (16 x 32768 tokens), median of {n1} runs: "
                      f"{t1 * 1e6:.0f} us",
            "us": round(t1 * 1e6, 1),
            "threads_all": {"threads": nthr, "us": round(tn * 1e6, 1),
                            "GB/s": round(nbytes / tn / 1e9, 3), "runs": nn},
            "cpu_model": cpu_model(), "nproc": os.cpu_count()}


def calibrate_copy(torch) -> None:
    """Plain device-to-device copy of COPY_CAL_BYTES, five times: under rocprofv3 --pmc its
    FETCH_SIZE / WRITE_SIZE per dispatch (KiB) against the known bytes gives the scale
    factor applied to the decode kernels' counters."""
    dev = torch.device("cuda:0")
    src = torch.ones(COPY_CAL_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "device copy", "bytes_read": COPY_CAL_BYTES,
                      "bytes_written": COPY_CAL_BYTES, "launches": 5}))


def _short_name(n: str) -> str:
    """A kernel name without its argument list, demangled where rocprofv3 left it mangled."""
    import re
    import subprocess
    if n.startswith("_Z"):
        # binutils' c++filt predates the _Float16 mangling (DF16_); spell it as
        # IEEE half (Dh) and rename afterwards
        try:
            d = subprocess.run(["c++filt", n.replace("DF16_", "Dh")], capture_output=True,
                               text=True).stdout.strip()
            n = d.replace("half", "_Float16") if d else n
        except OSError:
            pass
    n = n.replace("(anonymous namespace)::", "")
    return re.sub(r"\(.*", "", n).replace("void ", "").strip()[:100]


def rocprof_summary(path: str) -> None:
    """Print per-kernel averages from rocprofv3 CSV output under `path`: kernel-trace
    durations (*kernel_trace.csv) and counter values (*counter_collection.csv)."""
    import csv
    import glob
    import re
    import subprocess

    for f in sorted(glob.glob(os.path.join(path, "**", "*kernel_trace.csv"), recursive=True)):
        agg = {}
        for r in csv.DictReader(open(f)):
            d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            agg.setdefault(_short_name(r["Kernel_Name"]), []).append(d)
        print(f"# kernel trace: {os.path.relpath(f, path)}")
        print(f"{'calls':>7} {'avg_us':>9} {'median_us':>9} {'min_us':>8} {'max_us':>8}  kernel")
        for n, ds in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
            print(f"{len(ds):7d} {statistics.fmean(ds):9.2f} {statistics.median(ds):9.2f} "
                  f"{min(ds):8.2f} {max(ds):8.2f}  {n}")
    for f in sorted(glob.glob(os.path.join(path, "**", "*counter_collection.csv"), recursive=True)):
        agg = {}
        for r in csv.DictReader(open(f)):
            key = (_short_name(r["Kernel_Name"]), r["Counter_Name"])
            agg.setdefault(key, []).append(float(r["Counter_Value"]))
        print(f"# counters: {os.path.relpath(f, path)}")
        print(f"{'dispatches':>10} {'mean_per_dispatch':>18}  counter  kernel")
        for (n, c), v in sorted(agg.items()):
            print(f"{len(v):10d} {statistics.fmean(v):18.1f}  {c}  {n}")


def _counter_means(path: str, counter: str):
    """{kernel short name: mean counter value per dispatch} from rocprofv3 CSV under path."""
    import csv
    import glob
    import re
    out = {}
    for f in glob.glob(os.path.join(path, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            if r["Counter_Name"] != counter:
                continue
            out.setdefault(_short_name(r["Kernel_Name"]), []).append(float(r["Counter_Value"]))
    return {k: statistics.fmean(v) for k, v in out.items()}


def rocprof_traffic(fetch_dir, write_dir, cal_fetch_dir, cal_write_dir, match="llkv::") -> None:
    """Per-call HBM traffic of the library's kernels in a --profile-target run: FETCH_SIZE
    and WRITE_SIZE (KiB per dispatch) of each kernel whose name contains `match`, each
    scaled by bytes / counter of the plain copy of --calibrate-copy."""
    cf = _counter_means(cal_fetch_dir, "FETCH_SIZE")
    cw = _counter_means(cal_write_dir, "WRITE_SIZE")
    copy_f = max((v for k, v in cf.items() if "copyBuffer" in k or "copy" in k.lower()), default=None)
    copy_w = max((v for k, v in cw.items() if "copyBuffer" in k or "copy" in k.lower()), default=None)
    f_scale = COPY_CAL_BYTES / copy_f if copy_f else None
    w_scale = COPY_CAL_BYTES / copy_w if copy_w else None
    fetch = _counter_means(fetch_dir, "FETCH_SIZE")
    write = _counter_means(write_dir, "WRITE_SIZE")
    print(f"copy calibration: {COPY_CAL_BYTES} B read -> FETCH_SIZE {copy_f:.1f}, "
          f"{COPY_CAL_BYTES} B written -> WRITE_SIZE {copy_w:.1f}")
    print(f"scale: fetch {f_scale:.3f} B per unit, write {w_scale:.3f} B per unit")
    total = 0.0
    for k in sorted(set(fetch) | set(write)):
        if match not in k or "copy_rows" in k:   # the workload's own kernels, not its set-up
            continue
        fb = fetch.get(k, 0.0) * f_scale
        wb = write.get(k, 0.0) * w_scale
        total += fb + wb
        print(f"{k}: read {fb / 1e6:.3f} MB, written {wb / 1e6:.3f} MB per dispatch")
    print(f"traffic_bytes_per_call: {total:.0f}")


def rocprof_mfma(path: str, match="llkv::prefill_mfma", xcds: int = 8, simds: int = 1024) -> None:
    """MFMA utilisation of the matching kernels from a counter run with SQ_VALU_MFMA_BUSY_CYCLES
    and GRBM_GUI_ACTIVE: busy cycles / (active cycles of one XCD x SIMDs).  rocprofv3 sums
    GRBM_GUI_ACTIVE over the XCDs, so one XCD's active cycles are that sum / xcds."""
    busy = _counter_means(path, "SQ_VALU_MFMA_BUSY_CYCLES")
    active = _counter_means(path, "GRBM_GUI_ACTIVE")
    valu = _counter_means(path, "SQ_INSTS_VALU")
    mfma = _counter_means(path, "SQ_INSTS_MFMA")
    for k in sorted(busy):
        if match not in k:
            continue
        cyc = active.get(k, 0.0) / xcds
        util = busy[k] / (cyc * simds) if cyc else 0.0
        print(f"{k}: SQ_VALU_MFMA_BUSY_CYCLES {busy[k]:.0f}, GRBM_GUI_ACTIVE {active.get(k, 0):.0f} "
              f"({cyc:.0f} per XCD), MFMA busy {100 * util:.1f} % of {simds} SIMDs; "
              f"SQ_INSTS_MFMA {mfma.get(k, 0):.0f}, SQ_INSTS_VALU {valu.get(k, 0):.0f} "
              f"(VALU / MFMA instructions {valu.get(k, 0) / max(mfma.get(k, 1), 1):.2f})")


def read_traffic():
    """HBM bytes per decode call measured by rocprofv3 (FETCH_SIZE + WRITE_SIZE, scaled by
    the copy calibration), recorded in profiles/decode_cfg2_traffic.txt as a line
    'traffic_bytes_per_call: N'."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_call:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def profile_target(torch, kc, wl, name: str, iters: int) -> None:
    """Eager launches of one workload for rocprofv3 (kernel trace or counters): warm-up, then
    `iters` calls, each on the workload's own inputs.  Prints one line naming what ran."""
    dev = torch.device("cuda:0")
    if name in ("cfg2_decode", "cfg3_decode"):
        case = wl.config2() if name == "cfg2_decode" else wl.config3()
        B, hq, d = case.q.shape
        hkv, nb = case.k_pool.shape[2], case.k_pool.shape[0]
        layers = 8 if name == "cfg2_decode" else 2
        pools = [wl.device_pools(nb, hkv, d, case.k_pool.dtype, 100 + i, dev) for i in range(layers)]
        q, bt, sl = case.q.to(dev), case.block_table.to(dev), case.seq_lens.to(dev)
        out = torch.empty_like(q)
        ml = case.max_seq_len
        ws = kc._workspace(kc.decode_workspace_bytes(B, hq, hkv, d, 16, ml), dev)
        fn = lambda i: kc.paged_decode(q, pools[i % layers][0], pools[i % layers][1], bt, sl, ml,
                                       out=out, workspace=ws)
        what = f"{name}: llkv_paged_decode, {layers} layer pools rotated, {wl.decode_bytes(case)} B per call"
    elif name in ("cfg5_decode", "cfg5_prefill"):
        m5 = wl.config5()
        kp, vp = wl.device_pools(262144, 8, 128, torch.float16, 55, dev)
        if name == "cfg5_decode":
            c = m5.decode
            q, bt, sl = c.q.to(dev), c.block_table.to(dev), c.seq_lens.to(dev)
            out = torch.empty_like(q)
            fn = lambda i: kc.paged_decode(q, kp, vp, bt, sl, c.max_seq_len, out=out)
            what = f"{name}: llkv_paged_decode, {wl.decode_bytes(c)} B per call"
        else:
            c = m5.prefill
            kc.append_kv(c.k_chunk.to(dev), c.v_chunk.to(dev), c.slots.to(dev), kp, vp)
            q, bt, cu, sl = c.q.to(dev), c.block_table.to(dev), c.cu_q.to(dev), c.seq_lens.to(dev)
            out = torch.empty_like(q)
            fn = lambda i: kc.paged_prefill(q, kp, vp, bt, cu, sl, c.max_q_len, c.max_seq_len, True,
                                            out=out)
            what = f"{name}: llkv_paged_prefill, {wl.prefill_flops(c)} FLOP per call"
    elif name.startswith("ceiling_"):
        st = ceiling_setup(torch, kc, wl, name[len("ceiling_"):])
        _, (flat, chain) = read_ceiling(torch, st["pools"], st["table"], st["lens"], st["hkv"], st["d"],
                                        st["esize"], st["splits"], 2, timed=False)
        fn = flat
        what = (f"{name}: llkv_rc_flat over the decode's pages, {len(st['pools'])} pools rotated, "
                f"{st['bytes']} B of decode per call")
    elif name == "cfg4_prefill":
        c = wl.config4()
        kp, vp = c.k_pool.to(dev), c.v_pool.to(dev)
        kc.append_kv(c.k_chunk.to(dev), c.v_chunk.to(dev), c.slots.to(dev), kp, vp)
        q, bt, cu, sl = c.q.to(dev), c.block_table.to(dev), c.cu_q.to(dev), c.seq_lens.to(dev)
        out = torch.empty_like(q)
        fn = lambda i: kc.paged_prefill(q, kp, vp, bt, cu, sl, c.max_q_len, c.max_seq_len, True, out=out)
        what = f"{name}: llkv_paged_prefill, {wl.prefill_flops(c)} FLOP per call"
    else:
        raise SystemExit(f"unknown profile target {name}")
    for i in range(3):
        fn(i)
    torch.cuda.synchronize()
    for i in range(iters):
        fn(i)
    torch.cuda.synchronize()
    print(json.dumps({"profile_target": what, "calls": iters}), flush=True)


PROFILE_TARGETS = ("cfg2_decode", "cfg3_decode", "cfg5_decode", "cfg4_prefill", "cfg5_prefill",
                   "ceiling_cfg2", "ceiling_cfg3", "ceiling_cfg5")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-other-configs", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true")
    ap.add_argument("--rocprof-summary", metavar="DIR")
    ap.add_argument("--rocprof-traffic", nargs=4, metavar="DIR")
    ap.add_argument("--rocprof-mfma", metavar="DIR")
    ap.add_argument("--profile-target", choices=PROFILE_TARGETS,
                    help="eager launches of one workload for rocprofv3, no JSON line")
    ap.add_argument("--profile-iters", type=int, default=20)
    ap.add_argument("--read-ceiling", choices=("cfg2", "cfg3", "cfg5"),
                    help="read ceiling of one decode configuration beside its decode, one JSON line")
    args = ap.parse_args()
    if args.rocprof_summary:
        rocprof_summary(args.rocprof_summary)
        return
    if args.rocprof_traffic:
        rocprof_traffic(*args.rocprof_traffic)
        return
    if args.rocprof_mfma:
        rocprof_mfma(args.rocprof_mfma)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build's path has no multi-GPU "
              "component (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.calibrate_copy:
        calibrate_copy(torch)
        return
    from lightllm_amd import kv_cache as kc
    from lightllm_amd import workloads as wl
    if args.profile_target:
        profile_target(torch, kc, wl, args.profile_target, args.profile_iters)
        return
    if args.read_ceiling:
        read_ceiling_mode(torch, kc, wl, args.read_ceiling, max(20, args.steps // 4))
        return

    dec = bench_decode(args, torch, kc, wl)
    pre = None if args.no_prefill else bench_prefill(args, torch, kc, wl)
    other = None if args.no_other_configs else bench_other_configs(torch, kc, wl)
    cpu = None if args.no_cpu_baseline else cpu_baseline(dec, args.cpu_budget)

    step_us = dec["step_ms"] * 1e3
    traffic = read_traffic()
    value = dec["decode_bytes"] / (dec["decode_us_mean"] * 1e-6) / 1e9
    step_gbs = (dec["decode_bytes"] + dec["append_bytes"]) / (step_us * 1e-6) / 1e9
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["step_ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) K/V/Q, random page permutation)",
        "config": {"workload": "cfg2: paged decode + KV append, B=64, Hq=14 Hkv=2 D=64 fp32, "
                               "L~U[128,2048]+1, pool 32768 x 16-token pages",
                   "batch": 64, "layers_rotated": args.layers,
                   "pool_bytes_per_layer": dec["pool_bytes"],
                   "touched_bytes_per_rotation": dec["decode_bytes_pages"] * args.layers},
        "us_per_layer": round(step_us, 2),
        "step": "llkv_paged_decode_append (KV append + decode in one call), HIP-graph replay of --steps steps",
        "step_GBps_incl_append": round(step_gbs, 1),
        "us_per_layer_two_calls": round(dec["step_two_calls_us"], 2),
        "decode_us": round(dec["decode_us_mean"], 2),
        "decode_us_eager_median": round(dec["decode_us_eager_median"], 2),
        "decode_GBps_page_granular": round(dec["decode_bytes_pages"] / (dec["decode_us_mean"] * 1e-6) / 1e9, 1),
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(value / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "llkv_paged_decode (automatic schedule for this batch, from "
                               "llkv_paged_decode_schedule: %s, S=%d; %s)" % (
                                   dec["schedule"][0], dec["schedule"][1],
                                   "decode_split_kernel<MfmaDecode<float,64,7>> then decode_merge_kernel<float,1>"
                                   if dec["schedule"][0] == "splits" else "the kernels of that schedule"),
                     "bytes_per_launch": dec["decode_bytes"],
                     **ceiling_fields(dec["ceiling"], dec["decode_us_mean"], dec["decode_bytes"]),
                     "ceiling_note": "read ceiling: lightllm_amd/csrc/read_ceiling.hip reads exactly this "
                                     "batch's K/V rows (same pages, pieces, rotated pools, graph replay) "
                                     "and nothing else; ceiling_GBps counts the decode's algorithmic bytes "
                                     "over that time, frac_of_ceiling = ceiling time / decode time",
                     "timing": "HIP events on the launch stream around a HIP-graph replay of "
                               f"--steps llkv_paged_decode calls ({args.layers} layer pools rotated, "
                               "so a rotation touches more than twice the 256 MB last-level cache)"},
        "parity_ok": dec["parity_ok"],
        "cpu_baseline": cpu,
    }
    if pre is not None:
        line["prefill_cfg4"] = {"us": round(pre["us"], 2), "TFLOPs": round(pre["tflops"], 1),
                                "mfma_frac": round(pre["mfma_frac"], 4), "flop": pre["flop"],
                                "note": "HIP-graph replays of one call on the same 6.2 MB of K/V "
                                        "(MFMA-bound: its inputs stay cache-resident)",
                                "cpu_baseline": None if args.no_cpu_baseline else
                                cpu_baseline_prefill(torch, wl, args.cpu_budget)}
        pre32 = bench_prefill(args, torch, kc, wl, dtype=torch.float32)
        line["prefill_cfg4_shape_fp32"] = {"us": round(pre32["us"], 2), "TFLOPs": round(pre32["tflops"], 1),
                                           "mfma_frac_of_fp32_peak": round(pre32["mfma_frac"], 4)}
    if other is not None:
        if not args.no_cpu_baseline:
            other["cfg3_decode_S0"]["cpu_baseline"] = cpu_baseline_decode_cfg3(torch, wl, args.cpu_budget)
        line["other_configs"] = other
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
