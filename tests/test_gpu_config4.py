"""The capacity-limited expert cache at its benchmark shape, checked step by step: 40 MoE layers of H 4096 / I 2048
with 384 routed experts each in pinned host memory (the 40 layers' home rows alias 4 pinned stores, as the
benchmark's cache leg does), a 709-slot HBM cache replanned every 16 decode steps with the image's parameters,
decode T = 4 through the tier's split / fused / combine entry, then one 8,192-token chunk through the staging path
(8 slots x 8 experts) and the rewarm after it."""
import numpy as np
import pytest

import oracle as O
from ec_oracle import ECOracle
from helpers import OracleLayer, within_tolerance

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _check_placement(c, stores, bufs, NH, rng):
    """Pointer tables and slotof of every layer equal the cache's live residency (pending newcomers still point
    home); sampled residents' slot bytes equal their home bytes."""
    E = c.E
    pending = set()
    if c.pending:
        for li, items in c.pending["items"].items():
            pending.update(li * E + int(it[0]) for it in items)
    for li, st in enumerate(stores):
        tabs = np.stack([st._exl3_ptrs[k].cpu().numpy() for k in ("gate_trellis", "up_trellis", "down_trellis")], 1)
        want = st.home.numpy().copy()
        slot = np.full(E, -1, np.int32)
        for e in range(E):
            i = li * E + e
            if i in c.where and i not in pending:
                want[e] = c.pool.addrs(c.where[i])
                slot[e] = c.where[i]
        assert np.array_equal(tabs, want), f"layer {li}: pointer tables differ from the residency"
        assert np.array_equal(st.slotof.cpu().numpy(), slot), f"layer {li}: slotof differs"
    res = list(c.where.items())
    rb = c.pool.rows.row_bytes
    for k in rng.choice(len(res), min(4, len(res)), replace=False):
        i, s = res[int(k)]
        li, e = divmod(i, E)
        home = bufs[li % NH].array(np.uint8)[e * rb:(e + 1) * rb]
        got = c.pool.t[s].cpu().numpy().view(np.uint8)
        assert np.array_equal(got, home), f"slot {s} of ({li}, {e}) differs from its home row"


def test_capacity_limited_cache_at_benchmark_shape(dev, monkeypatch):
    import torch
    from mi355moe import cache, ct_vllm, exl3, moe, workload
    from mi355moe.hostmem import HostBuffer
    from mi355moe.store import ExpertStore

    H, I, E, K, T, L, NH, SLOTS, TP = 4096, 2048, 384, 8, 4, 40, 4, 709, 8192
    env = {"DSV41_CT_LAYERS": str(L), "DSV41_EC_SLOTS": str(SLOTS), "DSV41_EC_EVERY": "16", "DSV41_EC_ADMIT": "48",
           "DSV41_EC_DECAY": "0.9", "DSV41_EC_HYST": "1.0", "DSV41_EC_WARMUP": "16", "DSV41_EC_ASYNC": "1",
           "DSV41_EC_PREFILL_TOKENS": "512", "DSV41_EC_REWARM_AFTER": "4", "DSV41_EC_ELASTIC": "1",
           "DSV41_EC_MARGIN_MB": "1500"}
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    saved = (exl3._EXL3_HOST_DMA_MODE, exl3._DMA_B, exl3._DMA_NS, exl3._DMA_MIN_TOKENS, exl3.FAT_EXPERT_THRESHOLD,
             dict(exl3._DMA_STATE))
    exl3._EXL3_HOST_DMA_MODE, exl3._DMA_B, exl3._DMA_NS, exl3._DMA_MIN_TOKENS = 1, 8, 8, 513
    exl3.FAT_EXPERT_THRESHOLD = 32
    exl3._DMA_STATE.clear()
    exl3._DMA_LAST.clear()
    ct_vllm.reset()
    try:
        rows = cache.ExpertRows(H, I)
        bufs = [HostBuffer(E * rows.row_bytes) for _ in range(NH)]
        ct_vllm.install(exl3)
        method = exl3.Exl3MoEMethod()
        stores = []
        for l in range(L):
            st = ExpertStore(E, H, I, device=dev, limit=10.0, host_home=cache.HostHome(E, H, I, buffer=bufs[l % NH]))
            st.synthesize(1000 + l, trellis=l < NH)         # layer l's trellis is layer (l % NH)'s
            method.process_weights_after_loading(st)
            stores.append(st)
        hbm0 = ExpertStore(E, H, I, device=dev, limit=10.0).synthesize(1000)   # an HBM copy of layer 0
        torch.cuda.synchronize()
        c = ct_vllm.EC["cache"]
        assert c is not None and ct_vllm.S["started"] and len(ct_vllm.S["layers"]) == L
        print("config-4 cache: 40 layers registered", flush=True)
        rng = np.random.default_rng(2000)
        chk = np.random.default_rng(1)
        perms = [np.random.default_rng(2000 + l).permutation(E) for l in range(L)]
        x = _t(workload.activations(T, H, seed=7), dev).to(torch.bfloat16)
        ec = None
        replans = 0

        def decode_step(step):
            nonlocal ec, replans
            if step % 64 == 0 and step:
                for l in range(L):
                    perms[l] = workload.drift(perms[l], rng)
            routes = [workload.zipf_ids(T, K, E, rng, perms[l]) for l in range(L)]
            ct_vllm.before_step(T)
            for l in range(L):
                ids, w = _t(routes[l][0], dev), _t(routes[l][1], dev)
                out = exl3.apply_exl3_fused_moe(x, ids, w, stores[l], None, None, 10.0)
                if l == 0 and step % 12 == 0:
                    ref = exl3.apply_exl3_fused_moe(x, ids, w, hbm0, None, None, 10.0)
                    torch.cuda.synchronize()
                    assert torch.equal(out, ref), f"step {step}: layer 0 differs from its HBM copy"
            replan = not c.released and (c.step_no + 1) % c.every == 0 and c.step_no + 1 >= c.warmup
            counts = torch.stack([s.counts for s in stores]).cpu().numpy().copy() if replan else None
            rel, rew = c.releases, c.rewarms
            ct_vllm.ec_step()
            torch.cuda.synchronize()
            if c.rewarms != rew:
                adm = ec.rewarm(c.N)
                assert [(i, s) for i, s in c.where.items()] == adm
                _check_placement(c, stores, bufs, NH, chk)
                print(f"step {step}: rewarm of {len(adm)} experts checked", flush=True)
            if replan:
                if ec is None:
                    assert c.N == SLOTS
                    ec = ECOracle(L, E, c.N, admit=48, decay=0.9, hyst=1.0)
                ec.step(counts)
                assert [(i, s) for i, s in c.where.items()] == ec.resident
                assert c.free == ec.free and np.array_equal(c.score.reshape(-1), np.array(ec.score))
                _check_placement(c, stores, bufs, NH, chk)
                replans += 1
                print(f"step {step}: replan {replans} checked, {len(c.where)} resident, {ct_vllm.summary()['hit_rate']}"
                      f" hit rate", flush=True)

        for step in range(48):
            decode_step(step)
        assert replans == 3 and c.admits == 144
        # one 8,192-token chunk through the staging path: the cache is released first (elastic)
        ctx = workload.zipf_ids(TP, K, E, np.random.default_rng(3000), perms[0])
        xp = _t(np.random.default_rng(3001).normal(0, 1, (TP, H)).astype(np.float32), dev).to(torch.bfloat16)
        ct_vllm.before_step(TP)
        assert c.released and all(int((s.slotof >= 0).sum()) == 0 for s in stores)
        ec.release()
        print("staged 8192-token chunk", flush=True)
        idp, wp = _t(ctx[0], dev), _t(ctx[1], dev)
        staged = exl3.apply_exl3_fused_moe(xp, idp, wp, stores[0], None, None, 10.0)
        torch.cuda.synchronize()
        D = stores[0]._exl3_dma
        assert D["batches"] == 48 and D["bytes"] == 384 * rows.row_bytes
        w16 = ctx[1].astype(np.float16).astype(np.float32)
        one = moe.moe_prefill(hbm0, xp, idp, _t(w16, dev), cap=0)
        torch.cuda.synchronize()
        a, b = staged.cpu().numpy(), one.cpu().numpy()
        # the same per-route rows, added to a token in staging-batch order instead of route order: fp32
        # reassociation only
        mx, mean = O.tolerance_metrics(a, b.astype(np.float64))
        print(f"staged vs one-pass prefill on the HBM copy: {mx:.2e} {mean:.2e}", flush=True)
        assert mx <= 1e-5 and mean <= 1e-6
        rws = [0, 4095, 8191]
        x16 = xp.half().cpu().numpy()[rws].astype(np.float32)
        ref = OracleLayer(hbm0, 1000, cache=False).forward(x16, ctx[0][rws], w16[rws])
        ok, m = within_tolerance(a[rws], ref)
        print(f"staged chunk vs oracle {m}", flush=True)
        assert ok, m
        ct_vllm.ec_step()                                   # the step after the chunk: still released
        for step in range(48, 53):                          # calm decode steps: rewarm after 4
            decode_step(step)
        assert c.rewarms == 1 and not c.released
    finally:
        ct_vllm.uninstall(exl3)
        ct_vllm.reset()
        (exl3._EXL3_HOST_DMA_MODE, exl3._DMA_B, exl3._DMA_NS, exl3._DMA_MIN_TOKENS,
         exl3.FAT_EXPERT_THRESHOLD) = saved[:5]
        exl3._DMA_STATE.clear()
        exl3._DMA_STATE.update(saved[5])


def _host_picks():
    """The picks of the last published host job: (layer, [(token, expert)]), read from the pinned mailbox."""
    from mi355moe import ct_vllm
    S = ct_vllm.S
    mail = S["mail"]
    ctrl = mail.array(np.int64, (16,), 0)
    picks = mail.array(np.int32, (S["maxpicks"], 3), S["picks"] - mail.ptr)
    n = int(ctrl[4])
    return int(ctrl[2]), [(int(t), int(e)) for t, e in picks[:n, :2]]


def test_capacity_limited_cache_with_host_tier_past_drift(dev, monkeypatch):
    """The capacity-limited cache with the host tier serving the split's share of the misses (the benchmark's
    default), for 80 decode steps: past the ranking drift at step 64 and the replan after it. Every replan equals
    the oracle planner and leaves the tables equal to the residency; layer 0's output at steps 20 and 70, whose
    host share the tier computed from the pinned home rows, matches the oracle (GPU picks with fp16 weights, host
    picks with fp32 weights)."""
    import torch
    from mi355moe import cache, ct_vllm, exl3, workload
    from mi355moe import tier as host_tier
    from mi355moe.hostmem import HostBuffer
    from mi355moe.store import ExpertStore

    H, I, E, K, T, L, NH, SLOTS = 4096, 2048, 384, 8, 4, 40, 4, 709
    env = {"DSV41_CT_LAYERS": str(L), "DSV41_EC_SLOTS": str(SLOTS), "DSV41_EC_EVERY": "16", "DSV41_EC_ADMIT": "48",
           "DSV41_EC_DECAY": "0.9", "DSV41_EC_HYST": "1.0", "DSV41_EC_WARMUP": "16", "DSV41_EC_ASYNC": "1",
           "DSV41_EC_PREFILL_TOKENS": "512", "DSV41_EC_REWARM_AFTER": "4", "DSV41_EC_ELASTIC": "1",
           "DSV41_EC_MARGIN_MB": "1500", "DSV41_CPU_TIER": "1", "DSV41_CT_FORCE_N": "6", "DSV41_CT_THREADS": "8"}
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    ct_vllm.reset()
    try:
        rows = cache.ExpertRows(H, I)
        bufs = [HostBuffer(E * rows.row_bytes) for _ in range(NH)]
        ct_vllm.install(exl3)
        method = exl3.Exl3MoEMethod()
        stores = []
        for l in range(L):
            st = ExpertStore(E, H, I, device=dev, limit=10.0, host_home=cache.HostHome(E, H, I, buffer=bufs[l % NH]))
            st.synthesize(1000 + l, trellis=l < NH)
            method.process_weights_after_loading(st)
            stores.append(st)
        hbm0 = ExpertStore(E, H, I, device=dev, limit=10.0).synthesize(1000)
        torch.cuda.synchronize()
        c = ct_vllm.EC["cache"]
        assert c is not None and ct_vllm.S["started"] and ct_vllm.S["cpu_tier"] and host_tier.serving()
        print(f"config-4 cache with the host tier: self-test {ct_vllm.S['selftest']}", flush=True)
        assert ct_vllm.S["selftest"]["max_rel_vs_gpu"] < 2e-2
        oracle = OracleLayer(hbm0, 1000, cache=False)
        rng = np.random.default_rng(2000)
        chk = np.random.default_rng(1)
        perms = [np.random.default_rng(2000 + l).permutation(E) for l in range(L)]
        x = _t(workload.activations(T, H, seed=7), dev).to(torch.bfloat16)
        x16 = x.half().cpu().numpy().astype(np.float32)
        ec = None
        replans = 0
        for step in range(80):
            if step % 64 == 0 and step:
                for l in range(L):
                    perms[l] = workload.drift(perms[l], rng)
            routes = [workload.zipf_ids(T, K, E, rng, perms[l]) for l in range(L)]
            ct_vllm.before_step(T)
            for l in range(L):
                ids, w = _t(routes[l][0], dev), _t(routes[l][1], dev)
                out = exl3.apply_exl3_fused_moe(x, ids, w, stores[l], None, None, 10.0)
                if l == 0 and step in (20, 70):
                    torch.cuda.synchronize()
                    li, hp = _host_picks()
                    assert li == 0 and hp, f"step {step}: no host share on layer 0"
                    host = np.zeros((T, K), bool)
                    rid, rw = routes[0]
                    for t, e in hp:
                        host[t] |= rid[t] == e
                    ref = oracle.forward(x16, rid, np.where(host, rw, rw.astype(np.float16).astype(np.float32)))
                    ok, m = within_tolerance(out.cpu().numpy(), ref)
                    print(f"step {step}: layer 0 with {len(hp)} host picks vs oracle {m}", flush=True)
                    assert ok, m
            replan = not c.released and (c.step_no + 1) % c.every == 0 and c.step_no + 1 >= c.warmup
            counts = torch.stack([s.counts for s in stores]).cpu().numpy().copy() if replan else None
            ct_vllm.ec_step()
            torch.cuda.synchronize()
            if replan:
                if ec is None:
                    ec = ECOracle(L, E, c.N, admit=48, decay=0.9, hyst=1.0)
                ec.step(counts)
                assert [(i, s) for i, s in c.where.items()] == ec.resident
                assert c.free == ec.free and np.array_equal(c.score.reshape(-1), np.array(ec.score))
                _check_placement(c, stores, bufs, NH, chk)
                replans += 1
                print(f"step {step}: replan {replans} checked, {len(c.where)} resident, "
                      f"{ct_vllm.summary()['hit_rate']} hit rate", flush=True)
        s = ct_vllm.summary()
        hs = host_tier.stats()
        print(f"summary {s}, tier {hs}", flush=True)
        assert replans == 5 and c.admits == 240
        assert s["timeouts"] == 0 and s["cpu_experts"] > 0 and hs["rejected"] == 0
    finally:
        ct_vllm.uninstall(exl3)
        ct_vllm.reset()
