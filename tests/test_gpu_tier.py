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
