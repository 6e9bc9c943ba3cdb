"""Benchmark: SB-shape route n-gram memory layer forward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one forward of the SB-shape memory layer (d 1024, 184 routes, bf16 tables,
8 x 2048 tokens, hidden-state router) over resident synthetic inputs: router GEMM +
sign-pack, query projection, fused gather + sink readout, output projection, causal
conv.  Prints one JSON line with whole-job tokens/s, the fused kernel's roofline
(algorithmic bytes / HIP-event duration) and a CPU baseline (the oracle's PyTorch-CPU
restatement of the reference forward, timed on a bounded sample).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT), str(ROOT / "lngram-decode_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0
METRIC = "memory-layer tokens/s + % HBM roofline at SB shape; draft-step latency (us)"


EVENT_STRIDE = 5  # HIP events bracket every EVENT_STRIDE-th launch of a timed kernel in a timed loop


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_info() -> dict:
    """The host cores a CPU baseline ran on: CPU model, the NUMA nodes holding the cores this
    process may use, and their count."""
    cpus = sorted(os.sched_getaffinity(0))
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), model)
    except OSError:
        pass
    nodes = []
    base = Path("/sys/devices/system/node")
    for nd in sorted(base.glob("node[0-9]*")) if base.exists() else []:
        try:
            spec = (nd / "cpulist").read_text().strip()
        except OSError:
            continue
        mine = set()
        for part in filter(None, spec.split(",")):
            a, _, b = part.partition("-")
            mine.update(range(int(a), int(b or a) + 1))
        if mine & set(cpus):
            nodes.append(int(nd.name[4:]))
    return {"cpu_model": model, "numa_nodes": nodes, "affinity_cpus": len(cpus)}


def cpu_baseline(seconds: float) -> dict:
    """Oracle's PyTorch-CPU restatement of the reference SB forward (bf16, reference op order) on a
    bounded sample of the SB workload: 1 x 64-token windows, repeated for ~``seconds``."""
    import numpy as np
    import torch

    from lngram_hip import workloads
    from oracle import memory as om

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    w = workloads.SB.with_shape(1, 64)
    mem = workloads.build_memory(w, seed=0, device="cpu")
    sd = {k: v.detach() for k, v in mem.state_dict().items()}
    p = {k[len("module."):]: v for k, v in sd.items() if k.startswith("module.")}
    p["router.weight"] = sd["router.weight"]
    cfg = om.MemCfg(w.d_model, w.routes, w.mem_dim, w.q_heads, w.kv_heads, w.head_dim, eps=w.norm_eps)
    h = workloads.make_hidden(w, seed=1)

    def run(p, h, budget):
        ones = torch.ones(w.d_model, dtype=h.dtype)
        n_tok, t0 = 0, time.perf_counter()
        while True:
            h_norm = om.rms_norm(h, ones, w.norm_eps)
            q = om.router_logits(h_norm, p["router.weight"], work=torch.float32)
            codes = om.pack_route_codes(q.numpy(), 4)
            om.memory_forward(p, cfg, h, codes)
            n_tok += w.tokens
            el = time.perf_counter() - t0
            if el >= budget:
                return n_tok, el

    n_tok, el = run(p, h, seconds)
    n32, el32 = run({k: v.float() for k, v in p.items()}, h.float(), seconds / 2)
    del np
    return {"value": n_tok / el, "unit": "tokens/s", "cores": threads, "kind": "port", **host_info(),
            "sample": f"SB shape (d1024, R184, bf16) 1x64-token windows, {n_tok} tokens in {el:.1f} s, "
                      "oracle PyTorch-CPU restatement of the reference forward (router fp32, module bf16)",
            "fp32": {"value": n32 / el32, "unit": "tokens/s",
                     "sample": f"the same forward with fp32 parameters and hidden states, {n32} tokens in "
                               f"{el32:.1f} s"}}


def sdc_cpu_baseline(seconds: float) -> dict:
    """SD-C layer on the host cores, oracle restatements in the reference's op order: the SSM
    recurrence (fp64, ``ssm.py:58-65``), router features (``router.py:50-59``), fp32 router logits
    + sign-pack, and the bf16 module forward; 1 x 64-token windows repeated for ~``seconds``."""
    import torch

    from lngram_hip import workloads
    from oracle import memory as om

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    w = workloads.SDC.with_shape(1, 64)
    mem = workloads.build_memory(w, seed=0, device="cpu")
    sd = {k: v.detach() for k, v in mem.state_dict().items()}
    p = {k[len("module."):]: v for k, v in sd.items() if k.startswith("module.")}
    p["router.weight"] = sd["router.weight"]
    fsd = {k: v.detach() for k, v in mem.router_features.state_dict().items()}
    cfg = om.MemCfg(w.d_model, w.routes, w.mem_dim, w.q_heads, w.kv_heads, w.head_dim, eps=w.norm_eps)
    g = torch.Generator().manual_seed(7)
    E = (torch.randn(w.vocab, w.d_model, generator=g) * 0.02).to(w.dtype)
    tok = torch.randint(0, w.vocab, (w.batch, w.seq), generator=g)
    a = (0.9 + 0.099 * torch.rand(w.ssm_dim, generator=g)).numpy()
    u = torch.randn(w.batch, w.seq, w.ssm_dim, generator=g).numpy()
    h = workloads.make_hidden(w, seed=1)
    n_tok, t0 = 0, time.perf_counter()
    while True:
        s = torch.from_numpy(om.ssm_scan(a, u)).float()
        x = om.router_features(E[tok], fsd["start"], fsd["prev_norm.weight"], fsd["cur_norm.weight"], w.norm_eps, s)
        q = om.router_logits(x, p["router.weight"], work=torch.float32)
        om.memory_forward(p, cfg, h, om.pack_route_codes(q.numpy(), 4))
        n_tok += w.tokens
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": n_tok / el, "unit": "tokens/s", "cores": threads, "kind": "port", **host_info(),
            "sample": f"SD-C shape (d1024, R181, N256, bf16) 1x64-token windows, {n_tok} tokens in {el:.1f} s: "
                      "oracle SSM recurrence + router features + fp32 router + PyTorch-CPU module forward"}


def scaled_cpu_baseline(seconds: float) -> dict:
    """Scaled-table gather + sum on the host cores: the oracle's row formula (hashed slots), then
    the reference's embedding gather in bf16 and an fp32 sum over routes and orders (PyTorch-CPU), on
    a table grown 4x instead of 64x (0.8 GB instead of 13.1 GB, so that it is quick to fill; every
    row read is still a random 256 B row far outside the host's caches); 1 x 4096-token batches
    repeated for ~``seconds``."""
    import torch

    from oracle import memory as om

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    R, T, orders, sl, md = 184, 4096, (2, 3), 2, 128
    n2, n3 = R << (sl + 8), R << (sl + 12)
    g = torch.Generator().manual_seed(0)
    blk = (torch.randn(1 << 12, md, generator=g) * 0.02).to(torch.bfloat16)   # tiled: quick to fill
    tabs = [blk.repeat(n >> 12, 1) for n in (n2, n3)]            # row counts are multiples of 4096
    codes = torch.randint(0, 16, (1, T, R), generator=g, dtype=torch.uint8).numpy()
    n_tok, t0, i = 0, time.perf_counter(), 0
    while True:
        om.gather_sum_rows_torch(tabs, om.scaled_rows(codes, orders, 4, sl, seed=2024 + i))
        n_tok += T
        i += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    rows = R * ((T - 1) + (T - 2))
    gbs = i * (rows * md * 2 + T * md * 4 + T * R) / el / 1e9
    del tabs
    return {"value": n_tok / el, "unit": "tokens/s", "GBs": gbs, "cores": threads, "kind": "port", **host_info(),
            "sample": f"184 routes, orders (2,3), table grown 4x ({(n2 + n3) * md * 2 / 1e9:.1f} GB bf16), "
                      f"{i} x 4096-token batches in {el:.1f} s: oracle row formula + PyTorch-CPU gather, fp32 sum"}


def draft_cpu_baseline(seconds: float) -> dict:
    """The oracle's C++ port of the reference CPU drafter (``drafter.cpp`` per-token algorithm, fp32,
    bf16 tables, OpenMP over routes and vocabulary rows, online counts on) timed on the host cores:
    draft_tree over the 16-node tree + tree acceptance after the same 2048-token SD-B context, repeated
    for about ``seconds``."""
    import numpy as np

    from drafting import tree as dtree
    from lngram_hip import workloads
    from oracle import drafting as od
    from oracle.cdrafter import CppDrafterPort

    threads = len(os.sched_getaffinity(0))
    w = workloads.SDB_DRAFT
    cfg, t = workloads.build_draft_bundle(w, seed=0)
    c = CppDrafterPort(cfg, t, threads=threads, online=True)
    t0 = time.perf_counter()
    c.commit(workloads.make_context(w, seed=0))
    commit_s = time.perf_counter() - t0
    spec = dtree.tree16()

    def run(budget, least):
        steps, t_all = [], time.perf_counter()
        while True:
            t0 = time.perf_counter()
            node = c.draft_tree(spec)
            od.tree_accept(spec.parent, node, [node[i] for i in range(spec.n)])
            steps.append((time.perf_counter() - t0) * 1e6)
            if time.perf_counter() - t_all >= budget and len(steps) >= least:
                return steps

    steps = run(seconds * 2 / 3, 1)
    c.set_threads(1)
    one = run(seconds / 3, 3)
    return {"value": float(np.median(steps)), "unit": "us per draft step", "cores": threads, "kind": "port",
            **host_info(),
            "sample": f"{len(steps)} draft steps (16-node tree, 10 parent readouts over the full 32768 vocabulary, "
                      f"online counts) after committing the 2048-token context ({commit_s:.1f} s); C++ port of "
                      "drafting/cpu/drafter.cpp with OpenMP",
            "threads_1": {"value": float(np.median(one)), "unit": "us per draft step", "cores": 1,
                          "sample": f"{len(one)} of the same steps on one thread"}}


def draft_step(dev, iters: int, warmup: int):
    """Set up, and return the timing run of, the SD-B decode draft step on one GPU: the 2048-token
    context is committed, then one step = 16-node draft tree (10 parent readouts in 4 depths, top-3,
    online counts over the context) + codes of every node + verification gather [16, 182, 256] +
    greedy acceptance against a synthetic verifier argmax, ending when the accepted path and bonus
    token are on the host."""
    import torch

    from drafting import tree as dtree
    from drafting.gpu_drafter import GpuDrafter
    from lngram_hip import workloads

    w = workloads.SDB_DRAFT
    cfg, t = workloads.build_draft_bundle(w, seed=0)
    g = GpuDrafter((cfg, t), device=dev, max_len=w.context + 64, online=True)
    g.commit(workloads.make_context(w, seed=0))
    spec = dtree.tree16()
    n = spec.n
    first_child = [next((c for c in range(n) if spec.parent[c] == i), i) for i in range(n)]
    fc = torch.tensor(first_child, dtype=torch.long, device=dev)
    parent = torch.tensor(spec.parent, dtype=torch.int32, device=dev)
    # acceptance result in one device block (new tokens int64 [n], path int32 [n], path length int32),
    # brought to the host by one copy
    res = torch.empty(16 * n + 16, dtype=torch.uint8, device=dev)
    res_new, res_path = res[:8 * n].view(torch.int64), res[8 * n:12 * n].view(torch.int32)
    res_len = res[12 * n:12 * n + 4].view(torch.int32)
    host = torch.empty(16 * n + 16, dtype=torch.uint8).pin_memory()

    def run() -> dict:
        return _draft_run(g, spec, fc, parent, res, res_new, res_path, res_len, host, w, iters, warmup)

    return run


def _draft_run(g, spec, fc, parent, res, res_new, res_path, res_len, host, w, iters: int, warmup: int) -> dict:
    """Each case's whole step (the one-launch draft tree with its verification gather, the synthetic
    verifier argmax, the acceptance kernel and the copy of the result to pinned host memory) is
    captured once in one HIP graph; a timed step is one replay and one stream synchronisation."""
    import numpy as np
    import torch

    from lngram_hip import ops

    dev = res.device
    n = spec.n
    out = {}
    stream = torch.cuda.current_stream(dev)
    for case in ("all_accept", "reject_at_root"):
        def step():
            node_tok, rt = g.tree_step(spec, route_tokens=True)
            if case == "all_accept":
                argmax = node_tok[fc]                               # the verifier agrees with every top-1 child
            else:
                argmax = torch.full((n,), -1, dtype=torch.int64, device=dev)  # matches no drafted token
            ops.tree_accept(parent, node_tok, argmax, out=(res_path, res_len, res_new))
            host.copy_(res, non_blocking=True)
            return rt

        step()                                                      # eager once: errors surface here
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            keep = step()                                           # noqa: F841 (graph-owned outputs)
        wall, gpu = [], []
        for i in range(warmup + iters):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            e0.record(stream)
            graph.replay()
            e1.record(stream)
            stream.synchronize()
            el = time.perf_counter() - t0
            if i >= warmup:
                wall.append(el * 1e6)
                gpu.append(e0.elapsed_time(e1) * 1e3)
        k = int(host[12 * n:12 * n + 4].view(torch.int32)[0])
        out[case] = {"median_us": float(np.median(wall)), "p99_us": float(np.percentile(wall, 99)),
                     "gpu_median_us": float(np.median(gpu)), "accepted": k - 1}
        g.tree_error()            # the one-launch tree's error word is sticky: raises if any step's wait ran out
    # the draft + verify-gather step on its own (the tree with its verification route tokens, left on
    # the device for the verifier): the tree launch replayed from its graph, GPU and wall time
    g.tree_step(spec, route_tokens=True, graph=True)
    torch.cuda.synchronize()
    wall, gpu = [], []
    for i in range(warmup + iters):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(stream)
        g.tree_step(spec, route_tokens=True, graph=True)
        e1.record(stream)
        stream.synchronize()
        el = time.perf_counter() - t0
        if i >= warmup:
            wall.append(el * 1e6)
            gpu.append(e0.elapsed_time(e1) * 1e3)
    g.tree_error()
    wall_e, gpu_e = [], []
    for i in range(warmup + iters):   # the same launch issued directly (no graph)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(stream)
        g.tree_step(spec, route_tokens=True)
        e1.record(stream)
        stream.synchronize()
        el = time.perf_counter() - t0
        if i >= warmup:
            wall_e.append(el * 1e6)
            gpu_e.append(e0.elapsed_time(e1) * 1e3)
    g.tree_error()
    out["draft_verify_gather"] = {"median_us": float(np.median(wall)), "p99_us": float(np.percentile(wall, 99)),
                                  "gpu_median_us": float(np.median(gpu)),
                                  "direct_launch": {"median_us": float(np.median(wall_e)),
                                                    "p99_us": float(np.percentile(wall_e, 99)),
                                                    "gpu_median_us": float(np.median(gpu_e))},
                                  "note": "the 16-node tree and its verification route tokens [16, 182, 256] on the "
                                          "device (one launch, replayed from a graph), without the verifier stand-in, "
                                          "the acceptance and the host copy of the all_accept / reject_at_root steps"}
    e_bytes = w.vocab * w.d_model * 2
    alg = 4 * e_bytes + n * w.routes * 2 * w.mem_dim * 2 * 2 + 10 * w.routes * 2 * w.mem_dim * 2
    med = out["all_accept"]["gpu_median_us"]
    return {"workload": "SD-B decode draft step: d1024 V32768 R182 bf16, context 2048, gamma 4, 16-node tree, "
                        "online counts, verify-gather [16,182,256], greedy accept; the whole step (tree, synthetic "
                        "verifier argmax, acceptance, copy of the result to the host) replayed from one HIP graph "
                        "captured once per tree shape",
            "unit": "us", "iters": iters, **out, "target_us": 50.0,
            "algorithmic_bytes": alg, "achieved_GBs": alg / (med * 1e-6) / 1e9}


def _time_steps(step, steps: int, warmup: int, *kernels: str):
    """Mean wall ms per step over ``steps`` timed steps (after ``warmup``), bracketed by device
    synchronisations, and the mean HIP-event ms of each named kernel over the timed steps."""
    import contextlib

    import torch

    from lngram_hip import ops

    with torch.no_grad():
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        with contextlib.ExitStack() as stack:
            timers = {k: stack.enter_context(ops.KernelTimer(k, every=EVENT_STRIDE)) for k in kernels}
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                step()
            torch.cuda.synchronize()
            el = time.perf_counter() - t0
    return el / steps * 1e3, {k: t.mean_ms() for k, t in timers.items()}


def tiny_forward(dev, steps: int, warmup: int):
    """Set up, and return the timing run of, the tiny layer (d 128, 8 routes, mem_dim 32, fp32,
    4 x 128 tokens): launch-bound, tokens/s only."""
    import torch

    from lngram_hip import ops, workloads

    w = workloads.TINY
    mem = workloads.build_memory(w, seed=0, device=dev)
    h = workloads.make_hidden(w, seed=1, device=dev)
    ones = torch.ones(w.d_model, device=dev)

    def run() -> dict:
        ms, _ = _time_steps(lambda: mem(h, ops.rmsnorm(h, ones, w.norm_eps)), steps, warmup)
        return _tiny_result(w, ms)

    return run


def _tiny_result(w, ms: float) -> dict:
    return {"workload": "tiny layer: d128, R8, mem_dim 32, 4 query heads x 32, fp32, 4 x 128 tokens, hidden router",
            "tokens_per_s": w.tokens / (ms * 1e-3), "ms_per_step": ms,
            "note": "launch-bound (512 tokens): the roofline fraction is not meaningful"}


def chain_draft(dev, iters: int, warmup: int):
    """Set up, and return the timing run of, the reference's own drafter benchmark
    (``drafting/cpu_drafter.py:409-423``) on its published configuration's shapes (the SD-C bundle:
    R181, V32768, d1024, 256-channel SSM router and query term, count sketches K 16 per row and order,
    shortlist 64; ``results/evaluation/drafter/cpu_bench_sdc.json``): commit a 256-token random
    prompt, then per iteration time ``draft(4)`` (results on the host), divide by gamma, and commit
    the first drafted token."""
    import numpy as np
    import torch

    from drafting.gpu_drafter import GpuDrafter
    from lngram_hip import workloads

    w = workloads.SDC_DRAFT
    cfg, t = workloads.build_draft_bundle(w, seed=0)
    rng = np.random.default_rng(3)
    V, R, bits = cfg["vocab"], cfg["routes"], cfg["bits"]
    for n in cfg["ngrams"]:
        rows = R * (1 << (bits * n))
        t[f"sketch_ids_{n}"] = torch.from_numpy(rng.integers(0, V, (rows, 16)).astype(np.int32))
        t[f"sketch_counts_{n}"] = torch.from_numpy(rng.integers(0, 4, (rows, 16)).astype(np.int64))
    t["fallback"] = torch.from_numpy(rng.choice(V, size=64, replace=False).astype(np.int32))
    cfg = dict(cfg, sketch_k=16, shortlist_cap=64)
    gamma, plen = 4, 256
    g = GpuDrafter((cfg, t), device=dev, max_len=plen + warmup + iters + 16)
    prompt = [int(x) for x in np.random.default_rng(0).integers(0, V, plen)]

    def run() -> dict:
        g.reset()
        g.commit(prompt)
        per_tok = []
        for i in range(warmup + iters):
            t0 = time.perf_counter()
            out = g.draft(gamma)
            dt = time.perf_counter() - t0
            if i >= warmup:
                per_tok.append(dt / gamma * 1e6)
            g.commit(out.tokens[:1])
        a = np.asarray(per_tok)
        med = float(np.median(a))
        return {"workload": "the reference's drafter benchmark: SD-C bundle shapes (R181, V32768, d1024, N256, bf16 "
                            "tables), sketch K 16, shortlist 64, gamma 4, 256-token random prompt, one token committed "
                            "per draft",
                "unit": "us per drafted token", "iters": iters, "median_us": med,
                "p99_us": float(np.percentile(a, 99)), "mean_us": float(a.mean()),
                "reference_published": {"cpp_1_thread_us": 10312.791913747787, "cpp_4_threads_us": 3603.148739784956,
                                        "pytorch_us": 1317.1385508030653,
                                        "source": "results/evaluation/drafter/cpu_bench_sdc.json, cpu_bench_sdc_ref.json "
                                                  "(host CPU of the reference's evaluation box, fp16 tables)"},
                "vs_reference_cpp_1_thread": 10312.791913747787 / med}

    return run


def decode_step(dev, iters: int, warmup: int):
    """Set up, and return the timing run of, the cached decode step of the SB-shape memory layer:
    8 sequences with 2048 cached positions each take one new token (router codes, fused readout
    reading the code cache, output projection, conv over the cached window).  Eager launches and
    the fixed-shape step replayed from a HIP graph, both timed with device synchronisation per
    step; the state is rolled back after every step, so each reads 2048 cached positions."""
    import numpy as np
    import torch

    from ffnmem.infer import DecodeState, memory_codes, memory_model, memory_step, static_memory_step
    from lngram_hip import ops, workloads

    w = workloads.SB
    ctx = 2048
    mem = workloads.build_memory(w, seed=0, device=dev)
    model = memory_model(mem)
    h = workloads.make_hidden(w.with_shape(w.batch, ctx + 1), seed=1, device=dev)
    h_norm = ops.rmsnorm(h, torch.ones(w.d_model, dtype=w.dtype, device=dev), w.norm_eps)
    st = DecodeState.empty(model, w.batch, ctx + 16)
    with torch.no_grad():
        memory_step(model, 0, st, h[:, :ctx], memory_codes(model, 0, st, h_norm=h_norm[:, :ctx]))
    st.length = ctx
    h1, hn1 = h[:, ctx:ctx + 1].contiguous(), h_norm[:, ctx:ctx + 1].contiguous()
    L_t = torch.full((), ctx, dtype=torch.int32, device=dev)

    def eager():
        return memory_step(model, 0, st, h1, memory_codes(model, 0, st, h_norm=hn1))

    def static():
        return static_memory_step(model, 0, st, h1, None, L_t, router_x=hn1)

    def run() -> dict:
        out = {}
        with torch.no_grad():
            static()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                static()
            for name, fn in (("eager", eager), ("graph", g.replay)):
                times = []
                for i in range(warmup + iters):
                    torch.cuda.synchronize()
                    t0 = time.perf_counter()
                    fn()
                    torch.cuda.synchronize()
                    if i >= warmup:
                        times.append((time.perf_counter() - t0) * 1e6)
                out[f"{name}_median_us"] = float(np.median(times))
        med = out["graph_median_us"]
        return {"workload": f"SB-shape memory layer cached decode step: {w.batch} sequences x 1 new token after {ctx} "
                            "cached positions (router + fused readout on the code cache + o-proj + conv over the "
                            "cached window)",
                "unit": "us per step", "iters": iters, **out, "tokens_per_s": w.batch / (med * 1e-6)}

    return run


def tree_verify_step(dev, iters: int, warmup: int):
    """Set up, and return the timing run of, the memory block of draft-tree verification at the SB
    layer shape: one sequence with 2048 cached positions takes the 16 nodes of a draft tree (the
    nodes' router codes, their n-gram rows along their ancestors, the fused readout over those rows,
    the output projection into the conv cache and the conv over each node's ancestor window).  Eager
    launches, device synchronisation per step; the cached length stays 2048."""
    import numpy as np
    import torch

    from drafting.tree import tree16
    from ffnmem.infer import DecodeState, memory_codes, memory_model, memory_step, static_tree_memory_step, \
        tree_memory_step
    from lngram_hip import ops, workloads

    w = workloads.SB.with_shape(1, 2048)
    ctx, parent = 2048, tree16().parent
    n = len(parent)
    mem = workloads.build_memory(w, seed=0, device=dev)
    model = memory_model(mem)
    h = workloads.make_hidden(w.with_shape(1, ctx + n), seed=1, device=dev)
    h_norm = ops.rmsnorm(h, torch.ones(w.d_model, dtype=w.dtype, device=dev), w.norm_eps)
    st = DecodeState.empty(model, 1, ctx + n)
    with torch.no_grad():
        memory_step(model, 0, st, h[:, :ctx], memory_codes(model, 0, st, h_norm=h_norm[:, :ctx]))
    st.length = ctx
    hn, hnn = h[:, ctx:].contiguous(), h_norm[:, ctx:].contiguous()
    L_t = torch.full((), ctx, dtype=torch.int32, device=dev)

    def eager():
        return tree_memory_step(model, 0, st, hn, memory_codes(model, 0, st, h_norm=hnn), parent)

    def static():
        return static_tree_memory_step(model, 0, st, hn, memory_codes(model, 0, st, h_norm=hnn), parent, L_t)

    def run() -> dict:
        out = {}
        with torch.no_grad():
            static()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                static()
            for name, fn in (("eager", eager), ("graph", g.replay)):
                times = []
                for i in range(warmup + iters):
                    torch.cuda.synchronize()
                    t0 = time.perf_counter()
                    fn()
                    torch.cuda.synchronize()
                    if i >= warmup:
                        times.append((time.perf_counter() - t0) * 1e6)
                out[f"{name}_median_us"] = float(np.median(times))
                out[f"{name}_p99_us"] = float(np.percentile(times, 99))
        return {"workload": f"SB-shape memory layer, draft-tree verification: 1 sequence, {n}-node tree after {ctx} "
                            "cached positions (node codes, ancestor-window rows, fused readout over them, o-proj "
                            "into the conv cache, conv over ancestor windows)",
                "unit": "us per tree", "iters": iters, **out}

    return run


def serving_step(dev, iters: int, warmup: int):
    """Set up, and return the timing run of, decoding from host RAM at the SB shape: 8 sequences with
    2048 cached positions each take one new token, the rows coming from a serving-layout copy of the
    tables in pinned host memory that the GPU reads directly: B1 (the step's exact rows) and B4 (the
    step's rows selected from candidate blocks prefetched by the previous step), against B0 (tables in
    HBM).  Also the serving permutation of the 205 MB table (HBM-bound) and the host-link rate of the
    candidate reads beside a plain pinned host-to-device copy."""
    import numpy as np
    import torch

    from ffnmem.infer import DecodeState, memory_decode, memory_model
    from lngram_hip import ops, workloads
    from serving.prefetch import CandidatePrefetcher, HostGather, HostTables

    w = workloads.SB
    ctx = 2048
    mem = workloads.build_memory(w, seed=0, device=dev)
    model = memory_model(mem)
    h = workloads.make_hidden(w.with_shape(w.batch, ctx + 1), seed=1, device=dev)
    h_norm = ops.rmsnorm(h, torch.ones(w.d_model, dtype=w.dtype, device=dev), w.norm_eps)
    st = DecodeState.empty(model, w.batch, ctx + warmup + iters + 1)
    with torch.no_grad():
        memory_decode(model, 0, st, h[:, :ctx], h_norm=h_norm[:, :ctx])
    st.length = ctx
    h1, hn1 = h[:, ctx:ctx + 1].contiguous(), h_norm[:, ctx:ctx + 1].contiguous()
    host = HostTables.from_model(model)
    lt = host[0]
    m = mem.module
    t3 = m.tables["ngram_3"].weight.detach()

    def run() -> dict:
        out = {}
        b1, b4 = HostGather(host, dev), CandidatePrefetcher(host, dev)
        with torch.no_grad():
            for name, prov in (("b0", None), ("b1", b1), ("b4", b4)):
                # a run of single-token steps from position 2048 on (each mode rewinds the state)
                st.length = ctx
                times = []
                for i in range(warmup + iters):
                    torch.cuda.synchronize()
                    t0 = time.perf_counter()
                    memory_decode(model, 0, st, h1, h_norm=hn1, row_provider=prov)
                    torch.cuda.synchronize()
                    st.length += 1
                    if i >= warmup:
                        times.append((time.perf_counter() - t0) * 1e6)
                out[f"{name}_median_us"] = float(np.median(times))
            out["b4_hit_rate"] = b4.stats.summary()["hit_rate"]
            # serving permutation of the 3-gram table (193 MB read + written), HBM-bound
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            dst = torch.empty_like(t3)
            ops.permute_table(t3, m.num_routes, 3, 4, dst)
            e0.record()
            for _ in range(5):
                ops.permute_table(t3, m.num_routes, 3, 4, dst)
            e1.record()
            torch.cuda.synchronize()
            perm_ms = e0.elapsed_time(e1) / 5
            perm_bytes = 2 * t3.numel() * t3.element_size()
            # host link: candidate blocks of 8 sequences read from host RAM by the GPU, beside a pinned copy
            hist = st.codes[0][:, ctx - 2:ctx].contiguous()
            cand = lt.candidates(hist, ctx)
            e0.record()
            for _ in range(10):
                lt.candidates(hist, ctx, cand)
            e1.record()
            torch.cuda.synchronize()
            cand_ms = e0.elapsed_time(e1) / 10
            src = torch.empty(64 << 20, dtype=torch.uint8, pin_memory=True)
            dst8 = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
            dst8.copy_(src, non_blocking=True)
            e0.record()
            for _ in range(10):
                dst8.copy_(src, non_blocking=True)
            e1.record()
            torch.cuda.synchronize()
            h2d_gbs = 10 * src.numel() / (e0.elapsed_time(e1) * 1e-3) / 1e9
        b4.close()
        cand_bytes = cand.numel() * cand.element_size()
        del dst, dst8, src, cand
        return {"workload": f"SB-shape memory layer decode from host RAM: {w.batch} sequences x 1 new token after {ctx} "
                            "cached positions; tables (205 MB, serving layout) in pinned host memory read by the GPU",
                "unit": "us per step", "iters": iters, **out,
                "permute_table": {"kernel": "k_permute_table", "table": "3-gram, 193 MB", "avg_ms": perm_ms,
                                  "achieved_GBs": perm_bytes / (perm_ms * 1e-3) / 1e9,
                                  "hbm_frac": perm_bytes / (perm_ms * 1e-3) / 1e9 / HBM_PEAK_GBS},
                "candidate_read": {"kernel": "k_serving_candidates", "bytes": cand_bytes, "avg_us": cand_ms * 1e3,
                                   "host_link_GBs": cand_bytes / (cand_ms * 1e-3) / 1e9,
                                   "pinned_h2d_copy_GBs": h2d_gbs}}

    return run


def sdc_forward(dev, steps: int, warmup: int):
    """Set up, and return the timing run of, the SD-C layer: 8 x 4096 tokens, 181 routes; one step =
    diagonal SSM scan of u [8, 4096, 256] fp32 (decays U[0.9, 0.999]; the states also rounded to
    bf16 in the same launch) + the token router over concat(RMSNorm(E[x_{t-1}]), RMSNorm(E[x_t]),
    s_t) from token ids (V 32768, bf16; the feature rows gathered inside the router GEMM from the
    tabled embedding norms, formed once per weight version before timing) + memory forward (router
    GEMM 2304 -> 724 + sign-pack, query RMSNorm + projection, fused gather + readout, output
    projection, causal conv)."""
    import torch

    from lngram_hip import workloads

    w = workloads.SDC
    mem = workloads.build_memory(w, seed=0, device=dev)
    g = torch.Generator().manual_seed(7)
    E = (torch.randn(w.vocab, w.d_model, generator=g) * 0.02).to(w.dtype).to(dev)
    tok = torch.randint(0, w.vocab, (w.batch, w.seq), generator=g).to(dev)
    a = (0.9 + 0.099 * torch.rand(w.ssm_dim, generator=g)).to(dev)
    u = torch.randn(w.batch, w.seq, w.ssm_dim, generator=g).to(dev)
    h = workloads.make_hidden(w, seed=1, device=dev)
    mem.router_features.tables(E)                          # once per weight version (cached)

    def step():
        from lngram_hip import ops
        _, sb = ops.ssm_scan(a, u, want_bf16=True)
        return mem.forward_ids(h, tok, E, sb)

    def run() -> dict:
        ms, kms = _time_steps(step, steps, warmup, "ssm_scan", "memory_readout_fused")
        return _sdc_result(w, ms, kms)

    return run


def _sdc_result(w, ms: float, kms: dict) -> dict:
    scan_ms, fused_ms = kms["ssm_scan"], kms["memory_readout_fused"]
    n = w.tokens
    scan_bytes = 2 * n * w.ssm_dim * 4                  # the layer's minimum: u read, fp32 states written
    scan_kernel_bytes = scan_bytes + n * w.ssm_dim * 2   # the kernel also writes the states' bf16 copy
    layer_bytes = n * w.algorithmic_bytes_per_token() + w.weight_bytes() + scan_bytes
    # rows (R x 2 orders x 256 B) + query + codes read, head output written (the query's RMSNorm
    # scale comes with the query: the projection forms it)
    fused_bytes = n * (w.routes * 2 * w.mem_dim * 2 + 2 * w.d_model * 2 + w.routes)
    return {"workload": "SD-C layer: 8 x 4096 tokens, R181, d1024 bf16, 256-channel SSM scan (fp32, bf16 copy) + "
                        "embed2_ssm token router (feature rows gathered in the router GEMM) + memory forward",
            "tokens_per_s": n / (ms * 1e-3), "ms_per_step": ms, "algorithmic_bytes": layer_bytes,
            "layer_hbm_frac": layer_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "scan": {"kernel": "k_ssm_scan", "avg_ms": scan_ms, "algorithmic_bytes": scan_kernel_bytes,
                     "achieved_GBs": scan_kernel_bytes / (scan_ms * 1e-3) / 1e9,
                     "hbm_frac": scan_kernel_bytes / (scan_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                     "note": "u read, fp32 states and their bf16 copy written"},
            "readout": {"kernel": "k_readout_fused", "avg_ms": fused_ms, "algorithmic_bytes": fused_bytes,
                        "achieved_GBs": fused_bytes / (fused_ms * 1e-3) / 1e9,
                        "hbm_frac": fused_bytes / (fused_ms * 1e-3) / 1e9 / HBM_PEAK_GBS}}


def scaled_gather(dev, steps: int, warmup: int):
    """Set up, and return the timing run of, the scaled-table stress: 16 x 4096 tokens, 184 routes,
    orders (2, 3), each route's order block grown 64x (51,249,152 rows x 128 bf16 = 13.1 GB,
    HBM-resident), uniformly random codes; one step = one gather + sum launch (one row per token,
    route and order; fp32 sums [16, 4096, 128])."""
    import torch

    B, T, R, orders, sl, md = 16, 4096, 184, (2, 3), 6, 128
    n2, n3 = R << (sl + 8), R << (sl + 12)
    table = torch.empty(n2 + n3, md, dtype=torch.bfloat16, device=dev)
    g = torch.Generator(device=dev).manual_seed(0)
    for s0 in range(0, n2 + n3, 1 << 24):
        blk = table[s0:s0 + (1 << 24)]
        blk.normal_(0.0, 0.02, generator=g)
    tabs = [table[:n2], table[n2:]]
    codes = torch.randint(0, 16, (B, T, R), device=dev, dtype=torch.uint8)
    state = {"tabs": tabs, "codes": codes}
    del table, tabs, codes

    def run() -> dict:
        r = _scaled_run(state["tabs"], state["codes"], B, T, R, orders, sl, md, steps, warmup)
        state.clear()
        torch.cuda.empty_cache()
        return r

    return run


def _scaled_run(tabs, codes, B, T, R, orders, sl, md, steps: int, warmup: int) -> dict:
    import torch

    from lngram_hip import ops

    for _ in range(warmup):
        ops.gather_sum_scaled(tabs, codes, orders, 4, sl, seed=2024)
    torch.cuda.synchronize()
    with ops.KernelTimer("gather_sum_scaled") as kt:
        for i in range(steps):
            ops.gather_sum_scaled(tabs, codes, orders, 4, sl, seed=2024 + i)
        torch.cuda.synchronize()
    ms = kt.mean_ms()
    rows = B * R * ((T - 1) + (T - 2))                      # t >= n-1 reads a row
    alg = rows * md * 2 + B * T * md * 4 + B * T * R       # rows + fp32 out + codes
    gbs = alg / (ms * 1e-3) / 1e9
    return {"workload": "scaled-table gather + sum: B16 x T4096, R184, orders (2,3), 64x table "
                        "(51,249,152 x 128 bf16 = 13.1 GB), uniform random codes",
            "kernel": "k_gather_sum_scaled", "tokens_per_s": B * T / (ms * 1e-3), "avg_ms": ms,
            "algorithmic_bytes": alg, "achieved_GBs": gbs, "hbm_frac": gbs / HBM_PEAK_GBS, "steps": steps,
            "traffic": measured_traffic("gather_sum_scaled_traffic.json"),
            "traffic_source": "profiles/gather_sum_scaled_traffic.json (committed counter summary)"}


def surrogate_backward(dev, steps: int, warmup: int):
    """Set up, and return the timing run of, the lookup surrogate's backward at the SB shape: 8 x 2048
    tokens, 184 routes, mem_dim 128, bf16 tables of orders 2 and 3, approximate mode; one step = the
    route-logit gradient of both orders (one ``k_surrogate_grad`` launch per order) from resident
    memory gradients, logits and codes, each window's looked-up row read from the table as the
    training lookup does (its saved rows are the table's rows); the same step with the saved rows
    streamed in (``hard_memory`` given) is timed beside it."""
    import torch

    from lngram_hip import ops

    B, T, R, D, bits = 8, 2048, 184, 128, 4
    g = torch.Generator(device=dev).manual_seed(11)
    codes = torch.randint(0, 16, (B, T, R), device=dev, dtype=torch.uint8, generator=g)
    q = torch.randn(B, T, R, bits, device=dev, generator=g)
    legs = []
    for order in (2, 3):
        table = torch.empty(R << (bits * order), D, dtype=torch.bfloat16, device=dev).normal_(0.0, 0.02, generator=g)
        grad = torch.empty(B, T, R, D, dtype=torch.bfloat16, device=dev).normal_(0.0, 1.0, generator=g)
        valid = torch.ones(B, T, dtype=torch.bool, device=dev)
        valid[:, :order - 1] = False
        hard = ops.route_tokens(codes, [table], [order], bits)
        legs.append((order, table, grad, valid, hard))

    def step(saved: bool):
        for order, table, grad, valid, hard in legs:
            ops.surrogate_grad(grad, hard if saved else None, q, codes, table, valid, order, bits, 0, 1.0, 1.0,
                               False)

    def timed(saved: bool):
        for _ in range(warmup):
            step(saved)
        torch.cuda.synchronize()
        with ops.KernelTimer("surrogate_grad") as kt:
            t0 = time.perf_counter()
            for _ in range(steps):
                step(saved)
            torch.cuda.synchronize()
            el = time.perf_counter() - t0
        return el / steps * 1e3, kt.durations_ms()

    def run() -> dict:
        saved_ms, saved_d = timed(True)
        ms, d = timed(False)
        per_order = {f"order_{o}_us": 1e3 * sum(d[i::2]) / len(d[i::2]) for i, o in enumerate((2, 3))}
        # per (token, route, order n): the memory-gradient row, the looked-up row and n*bits
        # counterfactual rows (256 B each), 16 B of logits, 16 B of gradient, the code
        alg = B * T * R * sum((2 + n * bits) * D * 2 + 2 * bits * 4 + 1 for n in (2, 3))
        kern_ms = sum(d) / len(d) * 2
        gbs = alg / (kern_ms * 1e-3) / 1e9
        # distinct bytes: the memory-gradient stream, logits, gradient and codes once, plus each order's
        # table once (the looked-up rows come from the table)
        distinct = sum(B * T * R * (D * 2 + 2 * bits * 4 + 1) + (R << (bits * n)) * D * 2 for n in (2, 3))
        legs.clear()
        torch.cuda.empty_cache()
        return {"workload": "lookup surrogate backward (approximate) at the SB shape: B8 x T2048, R184, mem_dim 128, "
                            "bf16 tables of orders 2 and 3; route-logit gradient of both orders",
                "kernel": "k_surrogate_grad", "ms_per_step": ms, "tokens_per_s": B * T / (ms * 1e-3), **per_order,
                "gathered_bytes": alg, "gathered_GBs": gbs, "distinct_bytes": distinct,
                "distinct_GBs": distinct / (kern_ms * 1e-3) / 1e9,
                "distinct_hbm_frac": distinct / (kern_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "steps": steps,
                "with_saved_rows": {"ms_per_step": saved_ms,
                                    **{f"order_{o}_us": 1e3 * sum(saved_d[i::2]) / len(saved_d[i::2])
                                       for i, o in enumerate((2, 3))}},
                "note": "gathered bytes: the rows the reference algorithm reads (the counterfactual rows of a window "
                        "lie in its route's block, so most come from L2); distinct bytes: what has to cross HBM"}

    return run


def copy_bandwidth(dev, mib: int = 2048, reps: int = 10) -> float:
    """Bytes read + written per second by a plain device-to-device copy of ``mib`` MiB (HIP
    events over ``reps`` copies): the bandwidth a streaming kernel reaches on this GPU, reported
    beside the nominal 8 TB/s peak that every fraction here is taken against."""
    import torch

    n = mib << 20
    src = torch.ones(n // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    gbs = 2 * n * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del src, dst
    torch.cuda.empty_cache()
    return gbs


def measured_traffic(name: str = "readout_fused_sb_traffic.json"):
    """HBM-side bytes per launch of a kernel at its workload, from the committed hardware-counter
    summary (FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by the factor a plain copy of known
    size reads for the same counter); None if the summary is absent."""
    f = ROOT / "profiles" / name
    if not f.exists():
        return None
    try:
        return int(json.loads(f.read_text())["traffic_bytes"])
    except (ValueError, KeyError):
        return None


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # the GPU reaches its steady clocks after some tens of milliseconds of load: 50 warmup
    # forwards (~20 ms), then 100 timed ones (~40 ms)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--draft-iters", type=int, default=200)
    ap.add_argument("--no-draft", action="store_true")
    ap.add_argument("--no-scaled", action="store_true")
    ap.add_argument("--no-sdc", action="store_true")
    ap.add_argument("--no-train", action="store_true", help="skip the surrogate-backward leg")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="run one plain device copy of MIB MiB before warmup (known-size kernel that scales "
                         "hardware byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the hot path is single-GPU; --gpus {args.gpus} is not supported)",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from lngram_hip import _lib, ops, workloads

    if not _lib.LIB_PATH.exists():
        import __graft_entry__

        __graft_entry__.build()
    dev = torch.device("cuda:0")
    w = workloads.SB
    log(f"building {w.name}")
    mem = workloads.build_memory(w, seed=0, device=dev)
    h = workloads.make_hidden(w, seed=1, device=dev)
    h_norm = ops.rmsnorm(h, torch.ones(w.d_model, dtype=w.dtype, device=dev), w.norm_eps)
    torch.cuda.synchronize()
    if args.copy_calibration > 0:
        n = args.copy_calibration << 20
        src = torch.ones(n // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy calibration: {n} bytes read, {n} bytes written")
        del src, dst

    # Every leg is set up first (host-side model builds take seconds, during which an idle GPU
    # lowers its clocks); then the GPU legs run back to back and the headline's forwards follow at
    # once.  The power-hungriest legs (the plain copy, the 13 GB random gather) go first and the
    # SD-C layer forward, the load most like the headline's, last: after a change of load the GPU's
    # clocks settle over a few milliseconds, and the headline's first forwards would otherwise run
    # in that transient (up to ~7 % slower).  The CPU baselines run after every GPU measurement.
    legs: dict = {}
    if not args.no_scaled:
        log("scaled-table gather: set-up")
        legs["scaled_gather"] = scaled_gather(dev, max(3, args.steps // 2), 5)
    if not args.no_draft:
        log("draft step: set-up")
        legs["draft_step_us"] = draft_step(dev, args.draft_iters, 20)
    if not args.no_draft:
        log("chain draft (the reference's drafter benchmark): set-up")
        legs["chain_draft"] = chain_draft(dev, args.draft_iters, 20)
    if not args.no_draft:
        log("cached decode step: set-up")
        legs["decode_step"] = decode_step(dev, args.draft_iters, 20)
    if not args.no_draft:
        log("draft-tree verification memory block: set-up")
        legs["tree_verify_step"] = tree_verify_step(dev, args.draft_iters // 2, 10)
    if not args.no_draft:
        log("host-RAM serving step: set-up")
        legs["serving_step"] = serving_step(dev, args.draft_iters // 2, 10)
    if not args.no_train:
        log("surrogate backward: set-up")
        legs["surrogate_backward"] = surrogate_backward(dev, max(3, args.steps // 4), 2)
    if not args.no_sdc:
        log("tiny and SD-C forwards: set-up")
        legs["tiny_forward"] = tiny_forward(dev, 50, 5)
        legs["sdc_forward"] = sdc_forward(dev, max(3, args.steps // 2), 5)
    torch.cuda.synchronize()
    copy_gbs = copy_bandwidth(dev)
    extra: dict = {}
    for name, run in legs.items():
        log(name)
        extra[name] = run()

    with torch.no_grad():
        for _ in range(args.warmup):
            mem(h, h_norm)
        torch.cuda.synchronize()
        log(f"warmup done ({args.warmup}), timing {args.steps} steps")
        # timing events bracket every 5th readout launch of the timed loop (an event pair costs
        # ~5 us of device time per bracketed step)
        with ops.KernelTimer("memory_readout_fused", every=EVENT_STRIDE) as kt:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(args.steps):
                mem(h, h_norm)
            torch.cuda.synchronize()
            el = time.perf_counter() - t0
        fused_ms = kt.mean_ms()
    ms = el / args.steps * 1e3
    tok_s = w.tokens / (el / args.steps)
    # fused kernel algorithmic bytes per launch: rows (R x 2 orders x 256 B) + query + codes read,
    # head output written (the query arrives scaled by its RMSNorm: the projection forms the scale)
    es = 2
    fused_bytes = w.tokens * (w.routes * 2 * w.mem_dim * es + 2 * w.d_model * es + w.routes)
    achieved = fused_bytes / (fused_ms * 1e-3) / 1e9
    layer_bytes = w.tokens * w.algorithmic_bytes_per_token() + w.weight_bytes()
    layer_gbs = layer_bytes / (el / args.steps) / 1e9
    traffic = measured_traffic()
    log(f"{ms:.3f} ms/step, {tok_s / 1e6:.2f} M tok/s, fused kernel {fused_ms * 1e3:.1f} us "
        f"({achieved:.0f} GB/s)")

    result = {
        "metric": METRIC,
        "value": tok_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) hidden states, N(0,0.02) weights/tables)",
        "config": {"workload": "SB-shape layer-1 memory forward, hidden-state router", "d_model": w.d_model,
                   "routes": w.routes, "mem_dim": w.mem_dim, "batch": w.batch, "seq_len": w.seq,
                   "table_params": w.routes * (256 + 4096) * w.mem_dim},
        "roofline": {"bound": "hbm", "kernel": "k_readout_fused", "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "algorithmic_bytes": fused_bytes, "avg_ms": fused_ms,
                     "timed_launches": f"HIP events around every {EVENT_STRIDE}th launch of the timed loop",
                     "traffic_source": "profiles/readout_fused_sb_traffic.json: rocprofv3 FETCH_SIZE + WRITE_SIZE "
                                       "per dispatch of this kernel at this workload, copy-calibrated; read from "
                                       "the committed summary, not measured in this run"},
        "layer_hbm_frac": layer_gbs / HBM_PEAK_GBS,
        "layer_algorithmic_bytes": layer_bytes,
        "copy_GBs": copy_gbs,
    }
    result.update(extra)
    if not args.no_cpu:
        if "draft_step_us" in result:
            log("draft step cpu baseline")
            result["draft_step_us"]["cpu_baseline"] = draft_cpu_baseline(args.cpu_seconds)
        if "scaled_gather" in result:
            log("scaled-table gather cpu baseline")
            result["scaled_gather"]["cpu_baseline"] = scaled_cpu_baseline(min(args.cpu_seconds, 8.0))
        if "sdc_forward" in result:
            log("SD-C cpu baseline")
            result["sdc_forward"]["cpu_baseline"] = sdc_cpu_baseline(min(args.cpu_seconds, 8.0))
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
