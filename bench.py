#!/usr/bin/env python3
"""Benchmark: a decode step through 40 routed-expert MoE layers on one MI355X, and the legs around it.

Workload of `value` (one "step"): T = 4 tokens through 40 MoE layers of H 4096 / I 2048, 384 routed experts
(top-8) plus 1 shared expert per layer, all EXL3 3.0 bpw and resident in HBM (40 x 385 experts, 146 GB). Routing
per layer is Zipf(1.1) over a seeded permutation (seed 2000 + layer); weights are seeded synthetic (1000 + layer);
the input is bf16 N(0, 1) and each layer's output is rescaled to unit RMS (bf16) before the next layer. Each layer
runs routing prep, the fused decode expert kernels (trellis decode + GEMV + SwiGLU + Hadamard transforms) and the
fixed-order combine; the 40-layer step is replayed as one HIP graph.

Prints one JSON line. `value` is MoE tok/s = T / step time. `roofline` is measured live on the dominant kernel
(the gate/up decode GEMV) with HIP events on its stream. The other objects of the line:
  decode_t1       the same 40-layer step at T = 1
  split_combine   split + combine latency of one decode call (T = 4, 709-slot map), graph-launched
  prefill         the 16,384-token prefill layer (skewed routing) on the fat-expert grouped GEMM: MFMA utilisation
  peaks           HBM copy / read rates and a dense fp16 / bf16 GEMM (hipBLASLt) measured in the same run
  dsv41           the served DSV41 expert shape (H 5120, I 2304, top-6) as a secondary point: the 40-layer decode
                  step (204 GB of experts) and the 16k prefill layer
  cache           the capacity-limited configuration: experts in pinned host memory, a 709-slot HBM cache, decode
                  T = 4 with 8,192-token prefill chunks staged through 8 slots x 8 experts
  cpu_baseline    the reference's own CPU expert tier (kernels/cpu_avx2/ft_core.h, compiled from its sources into
                  oracle/_ref) on this host's cores: one layer of the step and the decode layer at T = 1, auto and
                  EXACT modes, on every physical core of the GPU's NUMA node and on 22 threads, 50 warm-up + 300
                  timed jobs each (p50 / p90)
"""
import argparse
import ctypes
import gc
import glob
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "dsv41-flash-offload_amd"))

METRIC = "MoE tok/s (decode T=1/4, prefill 16k) + HBM GB/s & MFMA util vs peak"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0           # dense fp16 / bf16
CPU_JOB_SHAPES = ((1, 3), (1, 6), (2, 6), (4, 6), (4, 10))   # (tokens, experts) of the reference's tier jobs


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def trellis_bytes(K, N):
    return (K // 16) * (N // 16) * 96


def expert_bytes(H, I):
    """Trellis of gate, up and down plus the fp16 scales of one expert (9,474,048 B at 4096 / 2048)."""
    return 2 * trellis_bytes(H, I) + trellis_bytes(I, H) + (2 * H + 2 * I + I + H) * 2


# ------------------------------------------------------------------------------------------ CPU baseline

def _cpulist(s):
    out = []
    for part in s.strip().split(","):
        if part:
            a, _, b = part.partition("-")
            out += list(range(int(a), int(b or a) + 1))
    return out


def host_topology():
    """lscpu-style counts from sysfs: sockets, physical cores, threads per core, NUMA nodes, the NUMA node of the
    GPU (its PCI device's numa_node; -1 on a single-node host means node 0) and the CPUs this process may use."""
    allowed = sorted(os.sched_getaffinity(0))
    core_of = {}
    for c in allowed:
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            with open(base + "physical_package_id") as f:
                pkg = int(f.read())
            with open(base + "core_id") as f:
                core = int(f.read())
        except OSError:
            pkg, core = 0, c
        core_of[c] = (pkg, core)
    nodes = {}
    for d in sorted(glob.glob("/sys/devices/system/node/node[0-9]*")):
        with open(os.path.join(d, "cpulist")) as f:
            nodes[int(d.rsplit("node", 1)[1])] = _cpulist(f.read())
    gpu_node = -1
    for d in sorted(glob.glob("/sys/class/drm/card[0-9]*/device/numa_node")):
        try:
            with open(d) as f:
                gpu_node = int(f.read())
            break
        except (OSError, ValueError):
            pass
    node = gpu_node if gpu_node in nodes else (min(nodes) if nodes else 0)
    node_cpus = [c for c in nodes.get(node, allowed) if c in core_of]
    seen, phys = set(), []
    for c in node_cpus:                       # one hardware thread per physical core
        if core_of[c] not in seen:
            seen.add(core_of[c])
            phys.append(c)
    cores = len(set(core_of.values()))
    return {"cpus_allowed": len(allowed), "sockets": len({p for p, _ in core_of.values()}), "physical_cores": cores,
            "threads_per_core": round(len(allowed) / max(1, cores), 2), "numa_nodes": max(1, len(nodes)),
            "gpu_numa_node": node, "gpu_numa_node_raw": gpu_node, "node_physical_cpus": phys, "allowed": allowed}


def cpu_child(spec):
    """One reference CPU-tier pool (the pool starts once per process): times the requested tasks and prints one
    JSON line. Tasks: "config0" (one layer at T = 1: top-8 of 384 + the shared expert), "layer" (layer 0 of the
    decode step: T = 4, top-8 + shared), "jobs" (the reference's tier job shapes at the served DSV41 shape, random
    experts of a 64-expert layer, x ~ N(0, 0.35), weights 0.15, as experimental/b70-tier/repro/smt_bench.py),
    "prefill" (the 16,384-token skewed layer: one timed moe_forward over a stratified quarter of the experts,
    every 4th in descending route count, each with all of its routes; the time is scaled by all routes over the
    sampled routes)."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    from mi355moe import workload
    from mi355moe.store import synth_scales

    spec = json.loads(spec)
    ref = os.path.join(ROOT, "oracle", "_ref", "libftref.so")
    R = ctypes.CDLL(ref)
    R.ref_moe_forward.restype = ctypes.c_int
    P = lambda a: ctypes.c_void_p(a.ctypes.data)
    keep = []

    def add_layer(li, E, H, I, seed, experts):
        ptrs = np.zeros((E, 3), np.int64)
        for e in sorted(set(experts)):
            mats = []
            for m in O.synth_expert_trellis(seed, e, H, I):
                b = np.zeros(m.size + 2048, np.uint16)      # tail pad: the AVX2 decode reads past a tile's end
                b[: m.size] = m.ravel()
                mats.append(b)
            keep.append(mats)
            ptrs[e] = [mm.ctypes.data for mm in mats]
        sc = synth_scales(seed, E, H, I)
        arrs = [np.ascontiguousarray(a).view(np.uint16) for a in (sc["w13_suh"][:, 0], sc["w13_svh"][:, 0],
                                                                   sc["w13_suh"][:, 1], sc["w13_svh"][:, 1],
                                                                   sc["w2_suh"], sc["w2_svh"])]
        keep.append((ptrs, arrs))
        R.ref_add_layer(li, E, H, I, P(ptrs), *[P(a) for a in arrs])

    H, I, E, K = 4096, 2048, 384, 8
    r0 = workload.zipf_routing(1, K, E, seed=2000)
    r4 = workload.zipf_routing(4, K, E, seed=2000)
    tasks = spec["tasks"]
    if "config0" in tasks or "layer" in tasks:
        add_layer(0, E + 1, H, I, 1000, list(r0[0].ravel()) + list(r4[0].ravel()) + [E])
    DH, DI, DE = 5120, 2304, 64
    if "jobs" in tasks:
        add_layer(1, DE, DH, DI, 1000, range(DE))
    if "prefill" in tasks:
        TP = 16384
        pids, pw = workload.skewed_routing(TP, K, E, seed=2000)
        pcounts = np.bincount(pids.ravel(), minlength=E)
        samp = np.argsort(-pcounts, kind="stable")[::4]
        add_layer(2, E, H, I, 1000, samp)
    cpus = spec["cpus"]
    carr = (ctypes.c_int * len(cpus))(*cpus)
    R.ref_pool_start(int(spec["threads"]), carr, len(cpus))
    R.ref_set_limit(ctypes.c_float(10.0))

    def run(li, make, mode, warm, timed, budget_s):
        ts, md = [], -1
        t_end = time.perf_counter() + budget_s
        for it in range(warm + timed):
            x, tok, exp, wt, out = make(it)
            t0 = time.perf_counter()
            md = R.ref_moe_forward(li, P(x), x.shape[0], P(tok), P(exp), P(wt), tok.size, P(out), mode)
            dt = time.perf_counter() - t0
            if md < 0:
                raise RuntimeError("reference CPU tier refused the call")
            if it >= warm:
                ts.append(dt)
            if time.perf_counter() > t_end and len(ts) >= 20:
                break
        ts.sort()
        return ts, {0: "AFFINE", 1: "EXACT", 2: "I16"}.get(md, str(md))

    def fixed(ids, w, T, H):
        ids = np.concatenate([ids, np.full((T, 1), E)], 1)
        w = np.concatenate([w, np.ones((T, 1), np.float32)], 1)
        x = np.random.default_rng(7).normal(0, 1, (T, H)).astype(np.float16).astype(np.float32)
        tok = np.repeat(np.arange(T, dtype=np.int32), ids.shape[1])
        job = (x, tok, ids.ravel().astype(np.int32), w.ravel().astype(np.float32), np.zeros((T, H), np.float32))
        return job, len(np.unique(ids))

    res = []
    budget = float(spec.get("budget_s", 30.0))
    for name, (ids, w) in (("config0", r0), ("layer", r4)):
        if name not in tasks:
            continue
        T = ids.shape[0]
        job, nexp = fixed(ids, w, T, H)
        for mode in spec["modes"]:
            ts, md = run(0, lambda it: job, mode, 50, 300, budget)
            p50 = ts[len(ts) // 2]
            res.append({"task": name, "tokens": T, "experts": nexp, "mode": "auto" if mode < 0 else md,
                        "mode_used": md, "p50_ms": round(p50 * 1e3, 4), "p90_ms": round(ts[int(len(ts) * 0.9)] * 1e3, 4),
                        "timed_jobs": len(ts), "warmup_jobs": 50,
                        "gbs": round(nexp * expert_bytes(H, I) / p50 / 1e9, 2), "tok_s": round(T / p50, 2)})
    if "jobs" in tasks:
        rng = np.random.default_rng(0)
        for m, k in CPU_JOB_SHAPES:
            def make(it, m=m, k=k):
                sel = np.stack([rng.choice(DE, k, replace=False) for _ in range(m)])
                if m > 1:
                    sel[1:, : k // 3] = sel[0, : k // 3]          # some sharing, as in real decode
                x = (rng.normal(0, 0.35, (m, DH))).astype(np.float16).astype(np.float32)
                tok = np.repeat(np.arange(m, dtype=np.int32), k)
                return (x, tok, sel.ravel().astype(np.int32), np.full(m * k, 0.15, np.float32),
                        np.zeros((m, DH), np.float32))
            ts, md = run(1, make, -1, 50, 300, budget / 2)
            res.append({"task": f"job m{m}k{k}", "shape": "H 5120 / I 2304", "tokens": m, "experts_per_token": k,
                        "mode": "auto", "mode_used": md, "p50_ms": round(ts[len(ts) // 2] * 1e3, 4),
                        "p90_ms": round(ts[int(len(ts) * 0.9)] * 1e3, 4), "timed_jobs": len(ts), "warmup_jobs": 50})
    if "prefill" in tasks:
        mask = np.isin(pids, samp)
        tt, jj = np.nonzero(mask)
        xp = np.random.default_rng(7).normal(0, 1, (TP, H)).astype(np.float16).astype(np.float32)
        tok = tt.astype(np.int32)
        exp = pids[tt, jj].astype(np.int32)
        wt = pw[tt, jj].astype(np.float32)
        outp = np.zeros((TP, H), np.float32)
        # warm-up: the first 64 tokens' sampled picks (pool and workspaces up)
        wm = tok < 64
        w_tok, w_exp, w_wt = (np.ascontiguousarray(a[wm]) for a in (tok, exp, wt))   # held across the call
        R.ref_moe_forward(2, P(xp), 64, P(w_tok), P(w_exp), P(w_wt), int(w_tok.size), P(outp), -1)
        t0 = time.perf_counter()
        md = R.ref_moe_forward(2, P(xp), TP, P(tok), P(exp), P(wt), int(tok.size), P(outp), -1)
        dt = time.perf_counter() - t0
        if md < 0:
            raise RuntimeError("reference CPU tier refused the call")
        scale = pids.size / tok.size
        fat = pcounts > 32
        flops = 2.0 * pcounts[fat].sum() * 3 * H * I
        res.append({"task": "prefill16k", "tokens": TP, "mode": "auto", "mode_used": {0: "AFFINE", 1: "EXACT", 2: "I16"}[md],
                    "sampled_experts": int(samp.size), "sampled_routes": int(tok.size), "routes": int(pids.size),
                    "sample_s": round(dt, 3), "layer_s_scaled": round(dt * scale, 3),
                    "tok_s": round(TP / (dt * scale), 1), "tflops": round(flops / (dt * scale) / 1e12, 3)})
    print(json.dumps({"threads": spec["threads"], "cpus": cpus, "results": res}), flush=True)


def cpu_baseline(L=40, T=4):
    """The reference CPU tier on this host, in child processes started before this process touches the GPU: (i)
    every physical core of the GPU's NUMA node (config 0, the step's layer, the tier job shapes; auto and EXACT),
    (ii) 22 threads as the reference serves it (ct/ct_vllm.py:46,79), placed on this process's CPUs the way the
    reference's pool places them (cpus[w % ncpus]) when there are fewer than 22."""
    if not os.path.exists(os.path.join(ROOT, "oracle", "_ref", "libftref.so")):
        log("cpu baseline: oracle/_ref/libftref.so not built; skipped")
        return None
    topo = host_topology()
    sets = [{"label": "every physical core of the GPU's NUMA node", "threads": len(topo["node_physical_cpus"]),
             "cpus": topo["node_physical_cpus"], "tasks": ["config0", "layer", "jobs", "prefill"], "modes": [-1, 1],
             "budget_s": 20.0},
            {"label": "22 threads (the reference's DSV41_CT_THREADS)", "threads": 22, "cpus": topo["allowed"],
             "tasks": ["config0", "layer"], "modes": [-1], "budget_s": 8.0}]
    runs = []
    for s in sets:
        t0 = time.time()
        spec = {k: s[k] for k in ("threads", "cpus", "tasks", "modes", "budget_s")}
        p = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-child", json.dumps(spec)],
                           capture_output=True, text=True, timeout=240)
        if p.returncode != 0:
            log(f"cpu baseline child failed ({p.returncode}): {p.stderr[-2000:]}")
            continue
        r = json.loads(p.stdout.strip().splitlines()[-1])
        r["label"] = s["label"]
        r["oversubscribed"] = s["threads"] > len(s["cpus"])
        runs.append(r)
        log(f"cpu baseline: {s['label']}: {time.time() - t0:.1f}s {r['results']}")
    if not runs:
        return None
    main = next((x for x in runs[0]["results"] if x["task"] == "layer" and x["mode"] == "auto"), None)
    pre = next((x for x in runs[0]["results"] if x["task"] == "prefill16k"), None)
    topo_out = {k: topo[k] for k in ("cpus_allowed", "sockets", "physical_cores", "threads_per_core", "numa_nodes",
                                     "gpu_numa_node", "gpu_numa_node_raw")}
    return {"value": round(T / (L * main["p50_ms"] * 1e-3), 3), "unit": "tok/s", "cores": runs[0]["threads"],
            "kind": "reference",
            "sample": f"layer 0 of the step ({main['experts']} experts, T={T}) on the reference CPU tier "
                      f"(ft_core.h moe_forward, auto mode = {main['mode_used']}), {main['timed_jobs']} timed jobs "
                      f"after 50 warm-up, p50 {main['p50_ms']:.3f} ms (p90 {main['p90_ms']:.3f}), scaled to {L} layers",
            "topology": topo_out, "runs": runs,
            "prefill16k": None if pre is None else dict(pre, cores=runs[0]["threads"], kind="reference",
                                                          sample=f"one moe_forward over {pre['sampled_experts']} of 384 "
                                                                 f"experts (every 4th by route count, all their "
                                                                 f"routes: {pre['sampled_routes']} of {pre['routes']}), "
                                                                 f"time scaled by routes")}


# ------------------------------------------------------------------------------------------ GPU legs

def start_cache_child(args):
    """The capacity-limited cache leg runs in a child process of its own, started here before this process touches
    the GPU: it waits on its stdin until the parent's GPU legs are done, then runs the leg and prints its JSON line.
    A failure of the leg (an exception, a signal) then costs that leg only; the parent reports it and still prints
    its line."""
    cmd = [sys.executable, "-u", os.path.abspath(__file__), "--workload", "cache", "--cache-child",
           "--slots", str(args.slots), "--cache-steps", str(args.cache_steps), "--chunk-every", str(args.chunk_every),
           "--chunk-tokens", str(args.chunk_tokens), "--home-layers", str(args.home_layers),
           "--ec-warmup", str(args.ec_warmup), "--cache-warmup", str(args.cache_warmup),
           "--hyb-tokens", str(args.hyb_tokens)]
    if not args.cpu_tier:
        cmd.append("--no-cpu-tier")

    def die_with_parent():                          # PR_SET_PDEATHSIG: the leg ends if this process does
        import signal
        ctypes.CDLL(None, use_errno=True).prctl(1, signal.SIGKILL, 0, 0, 0)
    return subprocess.Popen(cmd, stdin=subprocess.PIPE, stdout=subprocess.PIPE, text=True, preexec_fn=die_with_parent)


def run_cache_child(p, timeout_s=900):
    """Releases the waiting cache-leg child and returns its "cache" object, or a record of how it failed."""
    t0 = time.time()
    try:
        out, _ = p.communicate(input="go\n", timeout=timeout_s)
    except subprocess.TimeoutExpired:
        p.kill()
        p.wait()
        return {"error": f"timed out after {timeout_s} s", "process": "child"}
    lines = [l for l in out.splitlines() if l.startswith("{")]
    if p.returncode != 0 or not lines:
        return {"error": f"child exited with status {p.returncode}", "process": "child",
                "wall_s": round(time.time() - t0, 1)}
    try:
        r = json.loads(lines[-1])["cache"]
    except (ValueError, KeyError, TypeError) as ex:
        return {"error": f"unreadable child output: {ex!r}", "process": "child"}
    r["process"] = "child"
    return r


def free_gpu():
    import torch
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def synth_stores(E, H, I, L, dev):
    import torch
    from mi355moe.store import ExpertStore
    t0 = time.time()
    stores = []
    for l in range(L):
        stores.append(ExpertStore(E + 1, H, I, device=dev, limit=10.0).synthesize(1000 + l))
        if l % 10 == 9 or l == L - 1:
            torch.cuda.synchronize()
            log(f"stores {H}/{I}: {l + 1}/{L} layers resident ({(l + 1) * (E + 1) * expert_bytes(H, I) / 1e9:.1f} GB) "
                f"{time.time() - t0:.1f}s")
    return stores


def decode_step(stores, E, H, I, K, T, L, steps, warmup, roofline):
    """The L-layer decode step at T tokens, replayed as one HIP graph; with `roofline`, the gate/up and down
    partial-sum kernels' own per-layer launches are captured in graphs of their own and timed between events."""
    import numpy as np
    import torch
    from mi355moe import workload
    from mi355moe.moe import DecodeRunner
    dev = stores[0].w13_suh.device
    routes = [workload.zipf_routing(T, K, E, seed=2000 + l) for l in range(L)]
    uniq = [len(np.unique(r[0])) for r in routes]
    runners = []
    for l in range(L):
        R = DecodeRunner(E, H, I, T, K, device=dev)
        R.set_routes(torch.from_numpy(routes[l][0]).to(dev), torch.from_numpy(routes[l][1]).to(dev))
        runners.append(R)
    x0 = torch.from_numpy(workload.activations(T, H, seed=7)).to(dev)
    outs = [torch.empty((T, H), dtype=torch.float32, device=dev) for _ in range(2)]

    def step():
        # layer l reads the previous output (fp32), rescales it to unit RMS, rounds it through bf16 to the fp16
        # expert input, and writes its own output
        src = x0
        for l in range(L):
            src = runners[l].layer(stores[l], x=src, out=outs[l % 2], rescale=True)
        return src

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        final = step()
    torch.cuda.synchronize()
    res = {}
    if roofline:
        # Kernel-level timings first (every runner's workspace holds its layer's routing records from the eager pass
        # above). Each is taken at the GPU's steady clocks: from idle, this load runs about 20 % slower for its first
        # 30 ms or so while the clocks ramp up, so a graph is replayed untimed for at least 60 ms before its timed
        # replays. As a side effect the step below is also timed at steady clocks.
        def kernel_graph(phase):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for l in range(L):
                    runners[l].experts(stores[l], x=outs[0], phases=phase)
            return g

        def time_graph(g, warm_ms=60.0, reps=20):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            spent = 0.0
            while spent < warm_ms:
                e0.record()
                for _ in range(5):
                    g.replay()
                e1.record()
                torch.cuda.synchronize()
                spent += e0.elapsed_time(e1)
            e0.record()
            for _ in range(reps):
                g.replay()
            e1.record()
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) / (reps * L)     # ms per launch

        g_gu, g_d = kernel_graph(2), kernel_graph(8)
        res["t_gu"], res["t_d"] = time_graph(g_gu), time_graph(g_d)

        # the same launches inside the step: the step's kernels launched eagerly, layer by layer in the step's order
        # (route prep with the rescale, gate/up partial sums, epilogue, down partial sums, down epilogue, combine),
        # with events recorded on the stream right before and after each gate/up launch
        def eager_step(evs):
            src = x0
            for l in range(L):
                R = runners[l]
                R.experts(stores[l], x=src, phases=1, rescale=True)
                if evs is not None:
                    evs[l][0].record()
                R.experts(stores[l], x=src, phases=2)
                if evs is not None:
                    evs[l][1].record()
                R.experts(stores[l], x=src, phases=4 | 8 | 16)
                src = R.combine(out=outs[l % 2])

        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(L)]
        eager_step(None)
        torch.cuda.synchronize()
        per = []
        for _ in range(3):
            eager_step(evs)
            torch.cuda.synchronize()
            per += [a.elapsed_time(b) for a, b in evs]
        res["t_gu_in_step"] = float(np.mean(per))
        bgu = 2 * trellis_bytes(H, I) + 2 * H * 2          # gate/up partial kernel: trellis + suh13 per expert
        res["bytes_gu"] = float(np.mean([(u + 1) * bgu for u in uniq]))
        res["bytes_d"] = float(np.mean([(u + 1) * trellis_bytes(I, H) for u in uniq]))
        del g_gu, g_d
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_start = time.perf_counter()
    ev0.record()
    for _ in range(steps):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    ms_step = ev0.elapsed_time(ev1) / steps
    out_rms = float(final.float().pow(2).mean().sqrt())
    step_bytes = float(sum((u + 1) * expert_bytes(H, I) for u in uniq))
    res.update({"ms_step": ms_step, "ms_wall": wall * 1e3 / steps, "uniq": uniq, "step_bytes": step_bytes,
                "out_rms": out_rms})
    log(f"decode {H}/{I} T={T} top-{K}: step {ms_step:.3f} ms (wall {res['ms_wall']:.3f} ms), "
        f"{step_bytes / (ms_step * 1e-3) / 1e9:.0f} GB/s, final output rms {out_rms:.4f}")
    del graph
    return res


def bench_prefill(store, E, H, I, k, reps, tokens=16384, cap=32):
    """The 16k-token prefill layer: skewed routing (64 hot experts take 60 % of the assignments), every routed
    expert above `cap` routes on the fat-expert grouped GEMM. Returns timings and MFMA utilisation."""
    import numpy as np
    import torch
    from mi355moe import _lib, moe, workload
    dev = store.w13_suh.device
    ids, w = workload.skewed_routing(tokens, k, E, seed=2000)
    counts = np.bincount(ids.ravel(), minlength=E)
    fat = counts > cap
    flops = float(2.0 * counts[fat].sum() * 3 * H * I)
    x = torch.from_numpy(workload.activations(tokens, H, seed=7)).to(dev).to(torch.bfloat16)
    idd, wd = torch.from_numpy(ids).to(dev), torch.from_numpy(w).to(dev)
    n = tokens * k
    ws, wsb = moe._prefill_ws(store, n, dev)
    out = torch.empty((tokens, H), dtype=torch.float32, device=dev)
    Y = torch.empty((n, H), dtype=torch.float32, device=dev)

    def layer():
        _lib.call("mm_moe_prefill", store.mm_layer(), x.data_ptr(), _lib.DTYPE_BF16, tokens, k, idd.data_ptr(),
                  wd.data_ptr(), cap, 0, out.data_ptr(), ws.data_ptr(), wsb, _lib.stream_ptr())

    def grouped():
        _lib.call("mm_grouped_gemm", store.mm_layer(), x.data_ptr(), _lib.DTYPE_BF16, tokens, k, idd.data_ptr(), cap,
                  Y.data_ptr(), ws.data_ptr(), wsb, _lib.stream_ptr())

    def timed(fn, warm_ms=60.0):
        # untimed calls for at least warm_ms first, so the timed ones run at the GPU's steady clocks
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        spent = 0.0
        while spent < warm_ms:
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            spent += e0.elapsed_time(e1)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps
    t_layer = timed(layer)
    t_grouped = timed(grouped)
    peak = MFMA_PEAK_TFLOPS * 1e12
    return {"workload": f"prefill {tokens} tokens through one MoE layer (H {H}, I {I}), top-{k} skewed routing (64 "
                        f"hot experts take 60 %), experts above {cap} routes on the grouped GEMM, bf16 input",
            "tokens": tokens, "fat_experts": int(fat.sum()), "fat_routes": int(counts[fat].sum()),
            "fat_flops": flops, "ms_layer": round(t_layer, 4), "ms_grouped_gemm": round(t_grouped, 4),
            "tok_s": round(tokens / (t_layer * 1e-3), 1),
            "mfma_util_layer": round(flops / (t_layer * 1e-3) / peak, 4),
            "mfma_util_grouped_gemm": round(flops / (t_grouped * 1e-3) / peak, 4),
            "mfma_peak_tflops": MFMA_PEAK_TFLOPS, "dtype": "fp16 MFMA, fp32 accumulation", "reps": reps}


def bench_router(dev, E, H, k, reps=20):
    """The router (logits x G^T in fp32 from bf16 x and fp32 G ~ N(0, 0.02), top-k, softmax of the picks) at the
    decode (T = 4) and prefill (T = 16,384) sizes: `ms` per call from `reps` calls replayed as one graph (GPU time),
    `ms_eager` from the same calls launched one by one (the host's launch cost included)."""
    import numpy as np
    import torch
    from mi355moe import _lib, workload
    G = torch.from_numpy(np.random.default_rng(5).normal(0, 0.02, (E, H)).astype(np.float32)).to(dev)
    out = {}
    for T in (4, 16384):
        x = torch.from_numpy(workload.activations(T, H, seed=7)).to(dev).to(torch.bfloat16)
        ids = torch.empty((T, k), dtype=torch.int64, device=dev)
        w = torch.empty((T, k), dtype=torch.float32, device=dev)
        logits = torch.empty((T, E), dtype=torch.float32, device=dev)

        def call():
            _lib.call("mm_router_topk", x.data_ptr(), T, H, G.data_ptr(), E, k, logits.data_ptr(), ids.data_ptr(),
                      w.data_ptr(), _lib.stream_ptr())
        call()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            call()
        e1.record()
        torch.cuda.synchronize()
        ms_eager = e0.elapsed_time(e1) / reps
        # the same calls captured in one graph: the GPU's time per call, without the host's launch cost
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(reps):
                call()
        g.replay()
        torch.cuda.synchronize()
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        del g
        out[f"t{T}"] = {"ms": round(ms, 4), "fp32_tflops": round(2.0 * T * E * H / (ms * 1e-3) / 1e12, 2),
                        "ms_eager": round(ms_eager, 4)}
    out["workload"] = f"router top-{k} of {E} experts, H {H}: bf16 x, fp32 gate, fp32 logits and softmax"
    return out


def bench_split(calls=10000, per_graph=100):
    """Split + weighted combine + host-partial combine of one decode call (T=4 x top-8 over 384 experts, Zipf(1.1)
    routing, a 709-slot cache map with about 40 % of the picked experts resident, the image's cost-model policy,
    synthetic expert rows Y ~ N(0, 1) [32, 4096]); the host partial is already answered (ctrl[1] set ahead), so
    the bounded wait returns at once. `per_graph` calls are captured in one HIP graph; each replay is timed with
    events, giving `calls` per-call latencies (replay time / per_graph)."""
    import numpy as np
    import torch
    from mi355moe import _lib, workload
    from mi355moe.hostmem import HostBuffer
    dev = torch.device("cuda", 0)
    T, K, E, H = 4, 8, 384, 4096
    n = T * K
    ids, w = workload.zipf_routing(T, K, E, seed=2000)
    slotof = workload.cache_map(ids, E, slots=709, frac_resident=0.4, seed=2000)
    z = np.random.default_rng(7).normal(0, 1, (T, H)).astype(np.float16)
    pol = np.array([0.58, 0.03, 0.11, 0.20, 0.35, 384, -1, 0, 0], np.float32)
    Yh = np.random.default_rng(8).normal(0, 1, (n, H)).astype(np.float32)
    hb = HostBuffer(128 + T * H * 2 + n * 12)
    ctrl = hb.array(np.int64, (16,), 0)
    ctrl[:] = 0
    ctrl[1] = 1 << 62                      # the host has answered every job
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    sel, wd, zd, sl = t(ids.ravel()), t(w.ravel()), t(z.view(np.uint16)), t(slotof)
    score, pold, Y = torch.zeros(E, dtype=torch.float32, device=dev), t(pol), t(Yh)
    seqc = torch.zeros(1, dtype=torch.int64, device=dev)
    so = torch.empty(n, dtype=torch.int64, device=dev)
    wo = torch.empty(n, dtype=torch.float32, device=dev)
    dflag = torch.zeros(1, dtype=torch.int64, device=dev)
    stats = torch.zeros(8, dtype=torch.int64, device=dev)
    counts = torch.zeros(E, dtype=torch.int32, device=dev)
    hout = torch.zeros(T * H, dtype=torch.float32, device=dev)
    out = torch.empty((T, H), dtype=torch.float32, device=dev)

    def call(stream):
        sp = stream.cuda_stream
        _lib.call("mm_split", sel.data_ptr(), wd.data_ptr(), zd.data_ptr(), n, T, H, E, sl.data_ptr(), score.data_ptr(),
                  pold.data_ptr(), hb.data_ptr(0), hb.data_ptr(128), hb.data_ptr(128 + T * H * 2), seqc.data_ptr(), 0,
                  so.data_ptr(), wo.data_ptr(), dflag.data_ptr(), stats.data_ptr(), counts.data_ptr(), None, None, None,
                  sp)
        _lib.call("mm_combine", out.data_ptr(), Y.data_ptr(), so.data_ptr(), wo.data_ptr(), T, K, H, E, 0, sp)
        _lib.call("mm_combine_host", out.data_ptr(), T * H, dflag.data_ptr(), hb.data_ptr(0), hout.data_ptr(),
                  stats.data_ptr(), 10 ** 9, sp)

    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        call(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(per_graph):
            call(torch.cuda.current_stream())
    g.replay()
    torch.cuda.synchronize()
    reps = max(1, calls // per_graph)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for a, b in evs:
        a.record()
        g.replay()
        b.record()
    torch.cuda.synchronize()
    per = np.array(sorted(a.elapsed_time(b) * 1e3 / per_graph for a, b in evs))
    st = stats.cpu().tolist()
    res = {"workload": "split + weighted combine + host-partial combine, T=4 x top-8 over 384 experts, 709-slot map",
           "calls": reps * per_graph, "p50_us": round(float(per[len(per) // 2]), 3),
           "p90_us": round(float(per[int(len(per) * 0.9)]), 3), "hits_per_call": round(st[0] / max(1, st[3]), 2),
           "misses_per_call": round(st[1] / max(1, st[3]), 2), "host_experts_per_call": round(st[2] / max(1, st[3]), 2)}
    # the oracle's split and combine on one host core (bounded sample: 2,000 calls)
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    ts = []
    for _ in range(2000):
        t0 = time.perf_counter()
        r = O.split(ids.ravel(), w.ravel(), z, E, slotof, np.zeros(E, np.float32), pol)
        wm = np.where(r["sel_out"] >= 0, r["w_out"], 0).reshape(T, K).astype(np.float32)
        O.combine(np.zeros((T, H), np.float32), Yh, wm)
        ts.append(time.perf_counter() - t0)
    ts.sort()
    res["cpu_baseline"] = {"p50_us": round(ts[len(ts) // 2] * 1e6, 2), "cores": 1, "kind": "port",
                           "sample": "2,000 calls of the oracle's split and combine (C restatement) on one core"}
    del g
    return res


def calibrate_peaks(dev):
    """Rates measured in the same run: a 2 GiB device-to-device copy (read + write bytes / time), a 4 GiB read
    (the library's read probe: 16-byte loads, every byte once) and a dense 8192^3 GEMM through torch.mm
    (hipBLASLt) in fp16 and bf16."""
    import torch
    from mi355moe import _lib

    def timed(fn, reps):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / reps
    nb = 2 << 30
    a = torch.empty(nb // 4, dtype=torch.float32, device=dev).fill_(1.0)
    b = torch.empty_like(a)
    t_copy = timed(lambda: b.copy_(a), 10)
    del a, b
    nr = 4 << 30
    r = torch.empty(nr, dtype=torch.uint8, device=dev).fill_(3)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    t_read = timed(lambda: _lib.call("mm_read_probe", r.data_ptr(), nr, sink.data_ptr(), 0, _lib.stream_ptr()), 10)
    del r
    res = {"hbm_copy_gbs": round(2 * nb / t_copy / 1e9, 1), "hbm_read_gbs": round(nr / t_read / 1e9, 1)}
    n = 8192
    for name, dt in (("fp16", torch.float16), ("bf16", torch.bfloat16)):
        A = torch.randn((n, n), dtype=dt, device=dev)
        B = torch.randn((n, n), dtype=dt, device=dev)
        C = torch.empty((n, n), dtype=dt, device=dev)
        t = timed(lambda: torch.mm(A, B, out=C), 20)
        res[f"gemm_{name}_tflops"] = round(2.0 * n ** 3 / t / 1e12, 1)
        del A, B, C
    res["method"] = ("2 GiB torch copy (read + write bytes) and 4 GiB mm_read_probe (read bytes), 10 reps each; "
                     "torch.mm 8192^3, 20 reps; HIP events")
    return res


def bench_dsv41(args, dev):
    """The served DSV41 expert shape (H 5120, I 2304, top-6; experimental/b70-tier/repro/rep_ct.py:11): the 40-layer
    decode step at T = 4 with 40 x 385 experts resident (204 GB) and the 16k prefill layer."""
    H, I, E, K, L = 5120, 2304, 384, 6, args.layers
    stores = synth_stores(E, H, I, L, dev)
    d = decode_step(stores, E, H, I, K, 4, L, args.steps, args.warmup, roofline=False)
    res = {"workload": f"decode step through {L} MoE layers, T=4, H {H}, I {I}, 384 routed experts top-{K} + 1 shared, "
                       f"EXL3 3.0 bpw, all experts HBM-resident ({L * (E + 1) * expert_bytes(H, I) / 1e9:.1f} GB)",
           "ms_per_step": round(d["ms_step"], 4), "tok_s": round(4 / (d["ms_step"] * 1e-3), 2),
           "bytes_per_step": d["step_bytes"], "hbm_gbs": round(d["step_bytes"] / (d["ms_step"] * 1e-3) / 1e9, 1),
           "frac_of_peak": round(d["step_bytes"] / (d["ms_step"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           "mean_distinct_experts_per_layer": round(sum(d["uniq"]) / len(d["uniq"]), 2)}
    if not args.no_prefill:
        res["prefill"] = bench_prefill(stores[0], E, H, I, K, args.prefill_reps)
        log(f"dsv41 prefill: {res['prefill']}")
    del stores
    return res


def bench_cache(args):
    """Capacity-limited expert cache: 40 layers whose routed experts live in pinned host memory, a 709-slot HBM
    cache (elastic, replanned every 16 decode steps), decode T=4 steps interleaved with 8,192-token prefill
    chunks (one chunk every `--chunk-every` decode steps) whose host-resident experts stream through 8 staging
    slots of 8 experts. Routing Zipf(1.1) per layer, the ranking reshuffled by 5 % every 64 steps."""
    import numpy as np
    import torch
    from mi355moe import _lib, cache, ct_vllm, exl3, tier, workload
    from mi355moe.hostmem import HostBuffer
    from mi355moe.store import ExpertStore

    dev = torch.device("cuda", 0)
    H, I, E, K, T, L = 4096, 2048, 384, 8, 4, args.layers
    TP, NH = args.chunk_tokens, max(1, min(args.home_layers, L))
    os.environ.update({"DSV41_CT_LAYERS": str(L), "DSV41_EC_SLOTS": str(args.slots), "DSV41_EC_EVERY": "16",
                       "DSV41_EC_ADMIT": "48", "DSV41_EC_DECAY": "0.9", "DSV41_EC_HYST": "1.0",
                       "DSV41_EC_WARMUP": str(args.ec_warmup), "DSV41_EC_ASYNC": "1",
                       "DSV41_EC_PREFILL_TOKENS": "512", "DSV41_EC_REWARM_AFTER": "4", "DSV41_EC_ELASTIC": "1",
                       "DSV41_EC_MARGIN_MB": "1500", "DSV41_CPU_TIER": "1" if args.cpu_tier else "0",
                       "DSV41_CT_HYB_MAX": str(args.hyb_tokens) if args.cpu_tier else "0"})
    exl3._EXL3_HOST_DMA_MODE, exl3._DMA_B, exl3._DMA_NS, exl3._DMA_MIN_TOKENS = 1, 8, 8, 513
    exl3.FAT_EXPERT_THRESHOLD = 32
    rows = cache.ExpertRows(H, I)
    t0 = time.time()
    bufs = [HostBuffer(E * rows.row_bytes) for _ in range(NH)]
    log(f"cache: {NH} pinned host homes ({NH * E * rows.row_bytes / 1e9:.1f} GB) {time.time() - t0:.1f}s")
    ct_vllm.reset()
    ct_vllm.install(exl3)
    method = exl3.Exl3MoEMethod()
    stores, shared = [], []
    for l in range(L):
        st = ExpertStore(E, H, I, device=dev, limit=10.0, host_home=cache.HostHome(E, H, I, buffer=bufs[l % NH]))
        st.synthesize(1000 + l, trellis=l < NH)
        method.process_weights_after_loading(st)
        stores.append(st)
        shared.append(ExpertStore(1, H, I, device=dev, limit=10.0).synthesize(5000 + l))
    torch.cuda.synchronize()
    c = ct_vllm.EC["cache"]
    assert c is not None and ct_vllm.S["started"]
    log(f"cache: {L} layers registered {time.time() - t0:.1f}s")
    policy = None
    if args.cpu_tier:
        policy = ct_vllm.calibrate()
        log(f"cache: host tier calibrated {policy}, self-test {ct_vllm.S['selftest']}")
    # pinned -> HBM copy-engine peak (one 2 GB transfer)
    nb = min(2 << 30, bufs[0].nbytes)
    dst = torch.empty(nb, dtype=torch.uint8, device=dev)
    cache.stage_copy([(dst.data_ptr(), bufs[0].ptr, nb)])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    cache.stage_copy([(dst.data_ptr(), bufs[0].ptr, nb)])
    e1.record()
    torch.cuda.synchronize()
    h2d_peak = nb / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del dst
    log(f"cache: pinned H2D copy peak {h2d_peak:.1f} GB/s")

    rng = np.random.default_rng(2000)
    perms = [np.random.default_rng(2000 + l).permutation(E) for l in range(L)]
    prank = None
    exl3._DMA_TIMING = []
    c.timing = []

    def run_layers(x, ids_w, tokens):
        xbf = torch.empty((tokens, H), dtype=torch.bfloat16, device=dev)
        xh = torch.empty((tokens, H), dtype=torch.float16, device=dev)
        src = x
        for l in range(L):
            ids, w = ids_w(l)
            out = exl3.apply_exl3_fused_moe(src, ids, w, stores[l], None, None, 10.0)
            so = torch.zeros((tokens, 1), dtype=torch.long, device=dev)
            out += exl3.apply_exl3_fused_moe(src, so, torch.ones((tokens, 1), device=dev), shared[l], None, None, 10.0)
            _lib.call("mm_prepare_input", out.data_ptr(), tokens, H, 1, xbf.data_ptr(), xh.data_ptr(), _lib.stream_ptr())
            src = xbf
        return src

    stats = {"decode_steps": 0, "decode_s": 0.0, "prefill_chunks": 0, "prefill_s": 0.0}

    def tier_busy():                      # the host tier's cumulative busy time (ns), 0 without the tier
        return tier.stats()["busy_ns"] if args.cpu_tier else 0
    busy0 = None
    x0 = torch.from_numpy(workload.activations(T, H, seed=7)).to(dev).to(torch.bfloat16)
    total_steps = args.cache_steps
    step = 0
    hit0 = None
    t_all = time.perf_counter()
    while step < total_steps:
        if step % 64 == 0 and step:
            perms = [workload.drift(p, rng) for p in perms]
        if args.chunk_every and step % args.chunk_every == args.chunk_every // 2:
            if prank is None:
                prank = workload.zipf_ids(TP, K, E, np.random.default_rng(3000), np.arange(E))
            ct_vllm.before_step(TP)
            xp = torch.from_numpy(np.random.default_rng(step).normal(0, 1, (TP, H)).astype(np.float32)).to(dev).to(torch.bfloat16)
            pr_ids = torch.from_numpy(prank[0]).to(dev)
            pr_w = torch.from_numpy(prank[1]).to(dev)
            perm_d = [torch.from_numpy(p).to(dev) for p in perms]
            torch.cuda.synchronize()
            ts = time.perf_counter()
            run_layers(xp, lambda l: (perm_d[l][pr_ids], pr_w), TP)
            torch.cuda.synchronize()
            if step >= args.cache_warmup:          # the same window as the timed decode steps
                stats["prefill_s"] += time.perf_counter() - ts
                stats["prefill_chunks"] += 1
            ct_vllm.ec_step()
            log(f"cache: prefill chunk at step {step}: {time.perf_counter() - ts:.2f}s {ct_vllm.ec_summary()}")
        routes = [workload.zipf_ids(T, K, E, rng, perms[l]) for l in range(L)]
        rd = [(torch.from_numpy(r[0]).to(dev), torch.from_numpy(r[1]).to(dev)) for r in routes]
        ct_vllm.before_step(T)
        torch.cuda.synchronize()
        ts = time.perf_counter()
        run_layers(x0, lambda l: rd[l], T)
        ct_vllm.ec_step()
        torch.cuda.synchronize()
        dt = time.perf_counter() - ts
        if step >= args.cache_warmup:
            stats["decode_s"] += dt
            stats["decode_steps"] += 1
            if hit0 is None:
                hit0 = ct_vllm.S["stats"].tolist()
                busy0 = tier_busy()
        step += 1
        if step % 32 == 0:
            log(f"cache: step {step}/{total_steps} decode {dt * 1e3:.1f} ms {ct_vllm.summary()}")
    total_s = time.perf_counter() - t_all
    st = ct_vllm.S["stats"].tolist()
    busy_ms = (tier_busy() - busy0) * 1e-6 if busy0 is not None else 0.0
    # a lone prefill step of hyb_tokens tokens (every layer's experts staged: the cache is released first), with
    # the host tier taking each layer's trailing staging batches (the hybrid tail) and without it
    hybrid = None
    if args.cpu_tier and args.hyb_tokens > 0:
        TH = args.hyb_tokens
        hr = workload.zipf_ids(TH, K, E, np.random.default_rng(4000), np.arange(E))
        xh = torch.from_numpy(np.random.default_rng(4001).normal(0, 1, (TH, H)).astype(np.float32)).to(dev).to(torch.bfloat16)
        hid, hw = torch.from_numpy(hr[0]).to(dev), torch.from_numpy(hr[1]).to(dev)
        perm_d = [torch.from_numpy(p).to(dev) for p in perms]
        hybrid = {"tokens": TH, "runs": []}
        for rep, use in enumerate((True, False, True, False)):
            ct_vllm.S["hyb_max"] = TH if use else 0
            ct_vllm.before_step(TH, solo=True)
            tail0 = sum(int(s_._exl3_dma.get("tail_skipped", 0)) for s_ in stores)
            torch.cuda.synchronize()
            ts = time.perf_counter()
            run_layers(xh, lambda l: (perm_d[l][hid], hw), TH)
            torch.cuda.synchronize()
            dt = time.perf_counter() - ts
            ct_vllm.ec_step()
            tail = sum(int(s_._exl3_dma.get("tail_skipped", 0)) for s_ in stores) - tail0
            hybrid["runs"].append({"host_tail": use, "s": round(dt, 3), "tok_s": round(TH / dt, 1),
                                   "tail_batches": tail})
            log(f"cache: {TH}-token chunk, host tail {use}: {dt:.3f}s, {tail} tail batches over {L} layers")
        ct_vllm.S["hyb_max"] = TH
        w_ = [r["s"] for r in hybrid["runs"] if r["host_tail"]]
        wo_ = [r["s"] for r in hybrid["runs"] if not r["host_tail"]]
        hybrid.update(s_with_tail=round(min(w_), 3), s_without_tail=round(min(wo_), 3),
                      speedup=round(min(wo_) / min(w_), 3), cost=dict(ct_vllm.S["hyb_cost"]),
                      summary=ct_vllm.summary()["hybrid"])
    if hit0 is None:                      # every step was a warm-up step
        hit0 = st
    hits, misses = st[0] - hit0[0], st[1] - hit0[1]
    copy_ms = sum(a.elapsed_time(b) for a, b, _ in exl3._DMA_TIMING) + sum(a.elapsed_time(b) for a, b, _ in c.timing)
    copy_bytes = sum(n for _, _, n in exl3._DMA_TIMING) + sum(n for _, _, n in c.timing)
    dec_tok_s = T * stats["decode_steps"] / max(stats["decode_s"], 1e-9)
    pre_tok_s = TP * stats["prefill_chunks"] / max(stats["prefill_s"], 1e-9)
    summ = ct_vllm.summary()
    res = {
        "workload": f"capacity-limited expert cache: {L} MoE layers (H 4096, I 2048, 384 routed experts top-8 in "
                    f"pinned host memory + 1 HBM shared expert), {args.slots}-slot HBM cache, decode T={T} with one "
                    f"{TP}-token prefill chunk every {args.chunk_every} steps, 8 staging slots x 8 experts"
                    + (", decode misses split between PCIe reads and the host tier" if args.cpu_tier else ""),
        "layers": L, "slots": args.slots, "chunk_tokens": TP, "chunk_every": args.chunk_every,
        "distinct_host_homes": NH, "steps": total_steps, "timed_decode_steps": stats["decode_steps"],
        "warmup_steps": args.cache_warmup,
        "decode_ms_per_step": round(stats["decode_s"] * 1e3 / max(1, stats["decode_steps"]), 3),
        "hit_rate": round(hits / max(1, hits + misses), 4), "hits": hits, "misses": misses,
        "h2d_gbs": round(copy_bytes / max(copy_ms * 1e-3, 1e-9) / 1e9, 2), "h2d_bytes": copy_bytes,
        "h2d_peak_gbs": round(h2d_peak, 2),
        "decode_tok_s": round(dec_tok_s, 3), "prefill_tok_s": round(pre_tok_s, 1),
        "moe_tok_s": round((T * stats["decode_steps"] + TP * stats["prefill_chunks"]) /
                           max(stats["decode_s"] + stats["prefill_s"], 1e-9), 2),
        "prefill_chunks": stats["prefill_chunks"], "prefill_s": round(stats["prefill_s"], 3),
        "cpu_tier": bool(args.cpu_tier), "host_experts": summ["cpu_experts"], "host_jobs": summ["host_jobs"],
        "host_timeouts": summ["timeouts"],
        "host_busy_ms_per_step": round(busy_ms / max(1, stats["decode_steps"]), 3),
        "policy": policy, "hybrid_prefill": hybrid,
        "ec": ct_vllm.ec_summary(), "wall_s": round(total_s, 1),
    }
    ct_vllm.uninstall(exl3)
    ct_vllm.reset()
    exl3._DMA_STATE.clear()
    exl3._DMA_LAST.clear()
    exl3._WS.clear()
    del stores, shared, bufs
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--tokens", type=int, default=4)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-split", action="store_true")
    ap.add_argument("--no-dsv41", action="store_true")
    ap.add_argument("--no-cache", action="store_true")
    ap.add_argument("--no-peaks", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="after the measurements, copy 1 GiB device to device 3 times (torch copy kernel of known "
                         "bytes: 1 GiB read + 1 GiB written per launch), to scale HBM byte counters")
    ap.add_argument("--prefill-reps", type=int, default=5)
    ap.add_argument("--workload", choices=("decode", "cache"), default="decode",
                    help="decode: the 40-layer HBM-resident decode step and every other leg; cache: the "
                         "capacity-limited expert cache alone")
    ap.add_argument("--slots", type=int, default=709)
    ap.add_argument("--cache-steps", type=int, default=480)
    ap.add_argument("--chunk-every", type=int, default=64)
    ap.add_argument("--chunk-tokens", type=int, default=8192)
    ap.add_argument("--home-layers", type=int, default=4)
    ap.add_argument("--ec-warmup", type=int, default=16)
    ap.add_argument("--cache-warmup", type=int, default=320,
                    help="untimed steps of the cache leg: the 709-slot cache fills in about 240 steps at 48 admits "
                         "per 16-step replan")
    ap.add_argument("--no-cpu-tier", dest="cpu_tier", action="store_false",
                    help="cache leg: every decode miss read over PCIe by the GPU (default: the host tier serves the "
                         "share of the misses the split's cost model gives it, as the reference serves this "
                         "configuration)")
    ap.add_argument("--hyb-tokens", type=int, default=2048,
                    help="cache leg: the lone prefill step timed with and without the host tier's tail batches "
                         "(DSV41_CT_HYB_MAX; 0 = not timed)")
    ap.add_argument("--cpu-child", default=None, help=argparse.SUPPRESS)
    ap.add_argument("--cache-child", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.cpu_child is not None:
        return cpu_child(args.cpu_child)
    if args.cache_child and sys.stdin.readline().strip() != "go":
        return                                      # the parent ended before releasing this leg
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: measures one MI355X only (got --gpus {args.gpus}, WORLD_SIZE {world}); the multi-GPU "
              "expert-parallel design is documented but not built, so N > 1 is not run.", flush=True)
        sys.exit(2)

    # the cache leg's process starts (and waits) and the CPU baseline runs, in child processes, before this process
    # touches the GPU
    cache_child = None
    if args.workload == "decode" and not args.no_cache and args.layers == 40:
        cache_child = start_cache_child(args)
    cpu = None
    if args.workload == "decode" and not args.no_cpu_baseline:
        log("cpu baseline: reference CPU tier")
        cpu = cpu_baseline(L=args.layers, T=args.tokens)

    import numpy as np
    import torch
    dev = torch.device("cuda", 0)
    if args.workload == "cache":
        r = bench_cache(args)
        out = {"metric": METRIC, "value": r["decode_tok_s"], "unit": "tok/s", "n_gpus": 1,
               "steps": r["timed_decode_steps"], "warmup": r["warmup_steps"], "ms_per_step": r["decode_ms_per_step"],
               "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
               "data": "synthetic: seeded EXL3 3-bpw trellis + fp16 scales, Zipf(1.1) routing with 5 % rank drift "
                       "every 64 steps, bf16 N(0,1) input",
               "config": {"workload": r["workload"]}, "cache": r}
        print(json.dumps(out), flush=True)
        return

    H, I, E, K_TOP, T, L = 4096, 2048, 384, 8, args.tokens, args.layers
    stores = synth_stores(E, H, I, L, dev)
    d4 = decode_step(stores, E, H, I, K_TOP, T, L, args.steps, args.warmup, roofline=True)
    ms_step = d4["ms_step"]
    gu_gbs = d4["bytes_gu"] / (d4["t_gu"] * 1e-3) / 1e9
    gu_step_gbs = d4["bytes_gu"] / (d4["t_gu_in_step"] * 1e-3) / 1e9
    d_gbs = d4["bytes_d"] / (d4["t_d"] * 1e-3) / 1e9
    step_gbs = d4["step_bytes"] / (ms_step * 1e-3) / 1e9
    log(f"gate/up kernel: in the step {d4['t_gu_in_step'] * 1e3:.1f} us avg, {gu_step_gbs:.0f} GB/s; own graph "
        f"{d4['t_gu'] * 1e3:.1f} us avg, {gu_gbs:.0f} GB/s; down kernel: {d4['t_d'] * 1e3:.1f} us avg, "
        f"{d_gbs:.0f} GB/s; step {step_gbs:.0f} GB/s")
    d1 = decode_step(stores, E, H, I, K_TOP, 1, L, args.steps, args.warmup, roofline=False)
    ms1 = d1["ms_step"]
    # the same steps with EXACT weights (every decoded weight rounded to fp16, as the oracle and the reference's
    # reconstructed GPU weights are) instead of the AFFINE codebook evaluation
    for st in stores:
        st.exact, st._c = True, None
    d4x = decode_step(stores, E, H, I, K_TOP, T, L, args.steps, args.warmup, roofline=True)
    d1x = decode_step(stores, E, H, I, K_TOP, 1, L, args.steps, args.warmup, roofline=False)
    for st in stores:
        st.exact, st._c = False, None
    exact = {"ms_per_step": round(d4x["ms_step"], 4), "tok_s": round(T / (d4x["ms_step"] * 1e-3), 2),
             "hbm_gbs": round(d4x["step_bytes"] / (d4x["ms_step"] * 1e-3) / 1e9, 1),
             "gate_up_kernel_us": round(float(d4x["t_gu_in_step"]) * 1e3, 2),
             "gate_up_kernel_gbs": round(d4x["bytes_gu"] / (d4x["t_gu_in_step"] * 1e-3) / 1e9, 1),
             "gate_up_kernel_own_graph_us": round(float(d4x["t_gu"]) * 1e3, 2),
             "t1_ms_per_step": round(d1x["ms_step"], 4), "t1_tok_s": round(1 / (d1x["ms_step"] * 1e-3), 2)}
    log(f"decode EXACT: {exact}")
    router = None
    if not args.no_prefill:
        router = bench_router(dev, E, H, K_TOP)
        log(f"router: {router}")
    prefill = None
    if not args.no_prefill:
        log("prefill: 16384-token layer")
        prefill = bench_prefill(stores[0], E, H, I, K_TOP, args.prefill_reps)
        log(f"prefill: {prefill}")
    del stores
    free_gpu()

    split_res = None
    if not args.no_split:
        log("split/combine latency (10,000 graph-launched calls)")
        split_res = bench_split()
        log(f"split/combine: {split_res}")
        free_gpu()

    peaks = None
    if not args.no_peaks:
        peaks = calibrate_peaks(dev)
        log(f"peaks: {peaks}")
        free_gpu()

    dsv = None
    if not args.no_dsv41 and L == 40:
        log("dsv41 shape: 40 layers of H 5120 / I 2304, top-6")
        dsv = bench_dsv41(args, dev)
        log(f"dsv41: {dsv}")
        free_gpu()

    cache_res = None
    if cache_child is not None:
        log(f"cache: capacity-limited configuration, {args.cache_steps} steps (child process)")
        free_gpu()
        cache_res = run_cache_child(cache_child)
        log(f"cache: {cache_res.get('error', 'done')}")

    res = {
        "metric": METRIC,
        "value": round(T / (ms_step * 1e-3), 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: seeded EXL3 3-bpw trellis + fp16 scales, Zipf(1.1) routing, bf16 N(0,1) input",
        "config": {"workload": f"decode step through {L} MoE layers, T={T} tokens, H=4096, I=2048, 384 routed experts "
                               "top-8 + 1 shared, EXL3 3.0 bpw, all experts HBM-resident",
                   "layers": L, "tokens": T, "hidden": H, "intermediate": I, "experts": E, "top_k": K_TOP,
                   "shared_experts": 1, "mean_distinct_experts_per_layer": round(float(np.mean(d4["uniq"])), 2)},
        "roofline": {"bound": "hbm", "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": traffic_bytes(L, T),
                     "kernel": "mm::k_partial<0> (gate/up decode GEMV partial sums)",
                     "avg_launch_us": round(float(d4["t_gu"]) * 1e3, 2),
                     "bytes_per_launch": round(float(d4["bytes_gu"]), 1),
                     "method": "the 40 gate/up launches of the step, captured in a graph of their own and replayed "
                               "between HIP events",
                     "in_step": {"avg_launch_us": round(float(d4["t_gu_in_step"]) * 1e3, 2),
                                 "achieved": round(gu_step_gbs, 1), "frac": round(gu_step_gbs / HBM_PEAK_GBS, 4),
                                 "method": "the step's kernels launched eagerly in the step's order, HIP events right "
                                           "before and after each gate/up launch (includes any dispatch gap)"}},
        "step_hbm": {"bytes_per_step": d4["step_bytes"], "achieved_gbs": round(step_gbs, 1),
                     "frac_of_peak": round(step_gbs / HBM_PEAK_GBS, 4),
                     "down_kernel_gbs": round(d_gbs, 1), "down_avg_launch_us": round(float(d4["t_d"]) * 1e3, 2)},
        "ms_per_step_wall": round(d4["ms_wall"], 4),
        "decode_t1": {"ms_per_step": round(ms1, 4), "tok_s": round(1 / (ms1 * 1e-3), 2),
                      "hbm_gbs": round(d1["step_bytes"] / (ms1 * 1e-3) / 1e9, 1)},
    }
    res["decode_exact"] = exact
    if router is not None:
        res["router"] = router
    if peaks is not None:
        res["peaks"] = peaks
        res["roofline"]["frac_of_measured_read"] = round(gu_gbs / peaks["hbm_read_gbs"], 4)
        res["step_hbm"]["frac_of_measured_read"] = round(step_gbs / peaks["hbm_read_gbs"], 4)
    if split_res is not None:
        res["split_combine"] = split_res
    if prefill is not None:
        if peaks is not None:
            gemm = peaks["gemm_fp16_tflops"] * 1e12
            prefill["mfma_util_layer_vs_measured_gemm"] = round(prefill["fat_flops"] / (prefill["ms_layer"] * 1e-3) / gemm, 4)
        res["prefill"] = prefill
    if dsv is not None:
        res["dsv41"] = dsv
    if cache_res is not None:
        res["cache"] = cache_res
    if cpu is not None:
        res["cpu_baseline"] = cpu
    print(json.dumps(res), flush=True)
    if args.copy_calibration:
        a = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        log("copy calibration: 3 x 1 GiB device copies done")


def traffic_bytes(L, T):
    """HBM bytes per launch of the gate/up decode kernel at this workload, from the committed rocprofv3 counter
    summary (FETCH_SIZE and WRITE_SIZE passes scaled by a calibration copy), or None for another workload."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if L != 40 or T != 4 or not os.path.exists(path):
        return None
    with open(path) as f:
        return float(json.load(f)["traffic_bytes_per_launch"])


if __name__ == "__main__":
    main()
