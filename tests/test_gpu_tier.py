"""The hybrid decode tier end to end on the GPU: mm_split publishes the picks its cost model gives the host, the
host tier's worker computes them from the pinned home rows while the GPU computes the rest, and mm_combine_host
adds the host partial; with the worker stopped the bounded wait drops the partial."""
import numpy as np
import pytest

from helpers import OracleLayer, within_tolerance

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_hybrid_tier_split_worker_combine(dev, monkeypatch):
    import torch
    from mi355moe import ct_vllm, exl3
    from mi355moe import tier as host_tier
    from mi355moe.cache import HostHome
    from mi355moe.store import ExpertStore
    H, I, E, T, k, seed = 1024, 512, 32, 4, 6, 5050
    monkeypatch.setenv("DSV41_CPU_TIER", "1")
    monkeypatch.setenv("DSV41_CT_LAYERS", "1")
    monkeypatch.setenv("DSV41_CT_FORCE_N", "3")          # the first three misses (ascending id) to the host
    monkeypatch.setenv("DSV41_CT_THREADS", "4")
    monkeypatch.setenv("DSV41_CT_TIMEOUT_S", "0.05")
    ct_vllm.reset()
    try:
        st = ExpertStore(E, H, I, device=dev, host_home=HostHome(E, H, I)).synthesize(seed)
        torch.cuda.synchronize()
        ct_vllm.install(exl3)
        exl3.Exl3MoEMethod().process_weights_after_loading(st)
        assert ct_vllm.S["started"] and ct_vllm.S["cpu_tier"]
        print("selftest", ct_vllm.S["selftest"], flush=True)
        assert ct_vllm.S["selftest"]["max_rel_vs_gpu"] < 2e-2
        rng = np.random.default_rng(7)
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
        w = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
        x = _t(rng.normal(0, 1, (T, H)).astype(np.float32), dev).to(torch.bfloat16)
        idd, wd = _t(ids, dev), _t(w, dev)
        print("hybrid call", flush=True)
        out = exl3.apply_exl3_fused_moe(x, idd, wd, st, None, None, 10.0)
        torch.cuda.synchronize()
        s = ct_vllm.summary()
        host = sorted(np.unique(ids))[:3]
        assert s["cpu_experts"] == 3 and s["host_jobs"] == 1 and s["timeouts"] == 0
        assert host_tier.stats()["picks"] == int(np.isin(ids, host).sum())
        x16 = x.half().cpu().numpy().astype(np.float32)
        w16 = w.astype(np.float16).astype(np.float32)
        oracle = OracleLayer(st, seed)
        ref = oracle.forward(x16, ids, np.where(np.isin(ids, host), w, w16))
        ok, m = within_tolerance(out.cpu().numpy(), ref)
        print("hybrid vs oracle", m, flush=True)
        assert ok, m
        # the worker stopped: the 50 ms wait runs out, the host share is dropped, the GPU share stays
        host_tier.stop()
        print("timeout path", flush=True)
        out2 = exl3.apply_exl3_fused_moe(x, idd, wd, st, None, None, 10.0)
        torch.cuda.synchronize()
        s2 = ct_vllm.summary()
        assert s2["timeouts"] == 1
        ref2 = oracle.forward(x16, np.where(np.isin(ids, host), -1, ids), w16)
        ok, m = within_tolerance(out2.cpu().numpy(), ref2)
        assert ok, m
    finally:
        ct_vllm.uninstall(exl3)
        ct_vllm.reset()


def test_hybrid_prefill_tail_2048_tokens(dev, monkeypatch):
    """The hybrid prefill tail at full expert shape: a lone 2,048-token call on a layer of 128 host-resident
    experts (16 staging batches of 8): the cost model gives the host tier the last 3 batches (DSV41_HYB_MAX_BATCHES
    caps it), the split sends every pick of those 24 experts to the host, the staged prefill skips their batches,
    and the combine adds the host partial. Sampled tokens match the oracle (host picks with fp32 weights, GPU
    picks with fp16 weights); the whole output matches the all-staged call within the tolerance."""
    import torch
    from mi355moe import ct_vllm, exl3, workload
    from mi355moe import tier as host_tier
    from mi355moe.cache import HostHome
    from mi355moe.store import ExpertStore
    H, I, E, T, k, seed = 4096, 2048, 128, 2048, 8, 6060
    env = {"DSV41_CPU_TIER": "1", "DSV41_CT_LAYERS": "1", "DSV41_CT_HYB_MAX": "2048", "DSV41_CT_THREADS": "8",
           "DSV41_HYB_C0": "0", "DSV41_HYB_C1": "0", "DSV41_HYB_DMA": "1", "DSV41_HYB_TOK_US": "0",
           "DSV41_HYB_MAX_BATCHES": "3", "DSV41_CT_TIMEOUT_S": "20", "DSV41_CT_SELFTEST": "0"}
    for kk, v in env.items():
        monkeypatch.setenv(kk, v)
    saved = (exl3._EXL3_HOST_DMA_MODE, exl3._DMA_B, exl3._DMA_NS, exl3._DMA_MIN_TOKENS, dict(exl3._DMA_STATE),
             dict(exl3._DMA_LAST))
    exl3._EXL3_HOST_DMA_MODE, exl3._DMA_B, exl3._DMA_NS, exl3._DMA_MIN_TOKENS = 1, 8, 8, 513
    exl3._DMA_STATE.clear()
    exl3._DMA_LAST.clear()
    ct_vllm.reset()
    try:
        st = ExpertStore(E, H, I, device=dev, host_home=HostHome(E, H, I)).synthesize(seed)
        torch.cuda.synchronize()
        ct_vllm.install(exl3)
        exl3.Exl3MoEMethod().process_weights_after_loading(st)
        assert ct_vllm.S["started"] and ct_vllm.S["cpu_tier"] and host_tier.serving()
        kc, tail = ct_vllm._hyb_tail(st, T, k)
        assert kc == 3 and tail == list(range(E - 24, E)), (kc, tail)
        rng = np.random.default_rng(7)
        ids, w = workload.zipf_ids(T, k, E, rng, rng.permutation(E))
        x = _t(rng.normal(0, 1, (T, H)).astype(np.float32), dev).to(torch.bfloat16)
        idd, wd = _t(ids, dev), _t(w, dev)
        ct_vllm.before_step(T, solo=True)
        print("hybrid 2048-token call", flush=True)
        out = exl3.apply_exl3_fused_moe(x, idd, wd, st, None, None, 10.0)
        torch.cuda.synchronize()
        s = ct_vllm.summary()
        hs = host_tier.stats()
        print(f"hybrid summary {s['hybrid']}, tier {hs}", flush=True)
        on_host = np.isin(ids, tail)
        assert s["hybrid"]["calls"] == 1 and s["hybrid"]["timeouts"] == 0
        assert s["hybrid"]["host_experts"] == len(set(ids[on_host].tolist()))
        assert hs["picks"] == int(on_host.sum()) and hs["rejected"] == 0 and hs["stale"] == 0
        assert st._exl3_dma["tail_skipped"] == 3
        a = out.cpu().numpy()
        # the same call with every batch staged (no host tail)
        ct_vllm.S["hyb_max"] = 0
        full = exl3.apply_exl3_fused_moe(x, idd, wd, st, None, None, 10.0)
        torch.cuda.synchronize()
        ok, m = within_tolerance(a, full.cpu().numpy().astype(np.float64))
        print(f"hybrid vs all-staged {m}", flush=True)
        assert ok, m
        rows = [0, 5, 1023, 2047]
        x16 = x.half().cpu().numpy()[rows].astype(np.float32)
        w16 = w.astype(np.float16).astype(np.float32)
        ref = OracleLayer(st, seed, cache=False).forward(x16, ids[rows], np.where(on_host, w, w16)[rows])
        ok, m = within_tolerance(a[rows], ref)
        print(f"hybrid sampled tokens vs oracle {m}", flush=True)
        assert ok, m
    finally:
        ct_vllm.uninstall(exl3)
        ct_vllm.reset()
        exl3._EXL3_HOST_DMA_MODE, exl3._DMA_B, exl3._DMA_NS, exl3._DMA_MIN_TOKENS = saved[:4]
        exl3._DMA_STATE.clear()
        exl3._DMA_STATE.update(saved[4])
        exl3._DMA_LAST.clear()
        exl3._DMA_LAST.update(saved[5])
