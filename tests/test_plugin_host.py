"""Host-side logic of the plugin surface without a GPU: install / uninstall wrapping, run_batch's staged inners."""
import types


def test_install_wraps_and_uninstall_restores():
    from mi355moe import ct_vllm

    calls = []

    class Method:
        def process_weights_after_loading(self, layer):
            calls.append(("pwal", layer))

    def fused(*a):
        return "orig"

    X = types.SimpleNamespace(apply_exl3_fused_moe=fused, Exl3MoEMethod=Method)
    ct_vllm.reset()
    try:
        ct_vllm.install(X)
        assert X.apply_exl3_fused_moe is ct_vllm._fused
        lay = types.SimpleNamespace(host_home=None)
        X.Exl3MoEMethod().process_weights_after_loading(lay)
        assert calls == [("pwal", lay)] and ct_vllm.S["layers"] == []      # no host experts: not a tier layer
        # a call on a layer outside the tier falls through to the original entry
        assert ct_vllm._fused(types.SimpleNamespace(shape=(4, 8)), None, None, lay, None, None, None) == "orig"
        ct_vllm.install(X)                                               # idempotent
        ct_vllm.uninstall(X)
        assert X.apply_exl3_fused_moe is fused
        assert X.Exl3MoEMethod.process_weights_after_loading is not None
        X.Exl3MoEMethod().process_weights_after_loading(lay)
        assert len(calls) == 2
    finally:
        ct_vllm.reset()


def test_run_batch_builds_staged_inners():
    """Busy experts of the batch point at their slot rows; everything else is skipped; inners is not modified."""
    from mi355moe import dma_gemm

    class Lin:
        def __init__(self, e, key):
            self.e, self.key, self.trellis = e, key, ("home", e, key)

    class Pool:
        n = 6

        def addrs(self, r):
            return (1000 + r, 2000 + r, 3000 + r)

    E = 10
    inners = [{k: Lin(e, k) for k in ("gate", "up", "down")} for e in range(E)]
    D = {"batches": [(0, 3), (3, 6), (6, 9)], "cold": [9, 1, 4, 0, 7, 2, 3, 5, 8]}
    st = {"slots": Pool(), "free": [None, None]}
    counts = [50, 3, 40, 0, 99, 0, 0, 33, 0, 0]
    got = {}

    def apply_fat(x, ts, ws, cnt, staged, limit, cap, out, use_kernel, skip):
        got.update(staged=staged, cap=cap, skip=skip, use_kernel=use_kernel)

    dma_gemm.run_batch(D, st, 1, inners, counts, 32, "x", "ts", "ws", 10.0, "out", apply_fat, True)
    # batch 1 = experts [0, 7, 2] in slot 1 (rows 3 .. 5); busy: 0 (50), 7 (33), 2 (40)
    assert got["skip"] == set(range(E)) - {0, 7, 2} and got["cap"] == 32
    for row, e in enumerate([0, 7, 2]):
        assert [got["staged"][e][k].trellis for k in ("gate", "up", "down")] == [1003 + row, 2003 + row, 3003 + row]
    assert got["staged"][4] is inners[4] and inners[0]["gate"].trellis == ("home", 0, "gate")
    got.clear()
    dma_gemm.run_batch(D, st, 2, inners, counts, 32, "x", "ts", "ws", 10.0, "out", apply_fat, True)
    assert got == {}                     # no busy expert in batch 2: nothing runs


def test_step_hook_releases_before_prefill_steps_and_steps_after(monkeypatch):
    """install() wraps GPUModelRunner.execute_model of the engine's model-runner module (ct/ct_vllm.py:459-488): a
    step with more scheduled tokens than the cache's prefill size releases the cache before it runs, every step is
    followed by ec_step, hook errors never reach the engine, and uninstall() restores the method."""
    import sys
    from mi355moe import ct_vllm

    log = []

    class Runner:
        def execute_model(self, scheduler_output, extra=None):
            log.append(("exec", scheduler_output.total_num_scheduled_tokens))
            return "result"

    mod = types.ModuleType("vllm.v1.worker.gpu_model_runner")
    mod.GPUModelRunner = Runner
    monkeypatch.setitem(sys.modules, "vllm.v1.worker.gpu_model_runner", mod)

    class Cache:
        prefill_tokens, elastic, last_ntok = 512, True, 0

        def release(self):
            log.append(("release",))

        def step(self):
            log.append(("ec_step",))

    X = types.SimpleNamespace(apply_exl3_fused_moe=lambda *a: None,
                              Exl3MoEMethod=type("M", (), {"process_weights_after_loading": lambda self, l: None}))
    ct_vllm.reset()
    try:
        ct_vllm.install(X)
        assert ct_vllm.S["step_hooks"] == ["vllm.v1.worker.gpu_model_runner"]
        ct_vllm.EC["cache"] = Cache()
        ct_vllm.S["started"] = True
        r = Runner().execute_model(types.SimpleNamespace(total_num_scheduled_tokens=8192))
        assert r == "result" and log == [("release",), ("exec", 8192), ("ec_step",)]
        log.clear()
        Runner().execute_model(scheduler_output=types.SimpleNamespace(total_num_scheduled_tokens=4))
        assert log == [("exec", 4), ("ec_step",)]
        # a failing hook part is counted, the step still runs
        ct_vllm.EC["cache"] = types.SimpleNamespace(prefill_tokens=1, elastic=True, last_ntok=0)   # no release()
        log.clear()
        assert Runner().execute_model(types.SimpleNamespace(total_num_scheduled_tokens=100)) == "result"
        assert log == [("exec", 100)] and ct_vllm.S["hook_errors"] == 2
        ct_vllm.uninstall(X)
        assert not getattr(Runner.execute_model, "_mi355moe_step_hook", False)
    finally:
        ct_vllm.EC["cache"] = None
        ct_vllm.reset()


def test_hybrid_tail_cost_model_known_answers():
    """_hyb_tail with the reference's default constants (ct/ct_vllm.py:163-178: C0 0.24, C1 0.085, DMA 0.54,
    6 us per token, at most 24 batches): 384 cold experts in 48 batches of 8, NS = 8 slots, top-8. Hand-computed:
    T = 2048: rows 42.67, host 0.24 + 0.085 x 41.67 = 3.782 ms per expert, n = (384 x 0.54 - 12.288) / 4.322 =
    45.1 experts -> 5 batches; T = 600: rows 12.5, host 1.2175, n = (207.36 - 3.6) / 1.7575 = 115.9 -> 14 batches;
    T = 513 with a cap of 10 -> 10; a cold set of 70 experts (9 batches): T = 2048 gives (37.8 - 12.288) / 4.322 =
    5.9 experts -> 0 batches, T = 600 gives (37.8 - 3.6) / 1.7575 = 19.5 -> 2, capped at 9 - 8 = 1."""
    import numpy as np
    from mi355moe import ct_vllm, exl3
    saved = (exl3._DMA_B, exl3._DMA_NS)
    exl3._DMA_B, exl3._DMA_NS = 8, 8
    ct_vllm.reset()
    try:
        ct_vllm.S["hyb_cost"] = {"c0": 0.24, "c1": 0.085, "dma": 0.54, "tok_us": 6.0, "max_batches": 24}
        lay = types.SimpleNamespace(E=384, slot_host=np.full(384, -1, np.int32), _exl3_dma={})
        kc, tail = ct_vllm._hyb_tail(lay, 2048, 8)
        assert kc == 5 and tail == list(range(384 - 40, 384))
        assert ct_vllm._hyb_tail(lay, 600, 8)[0] == 14
        ct_vllm.S["hyb_cost"]["max_batches"] = 10
        assert ct_vllm._hyb_tail(lay, 513, 8)[0] == 10
        lay.slot_host[70:] = 0                       # only experts 0 .. 69 are cold: 9 batches
        assert ct_vllm._hyb_tail(lay, 2048, 8) == (0, [])
        kc, tail = ct_vllm._hyb_tail(lay, 600, 8)
        assert kc == 1 and tail == list(range(64, 70))
        lay.slot_host[:] = 0                         # nothing staged: no tail
        assert ct_vllm._hyb_tail(lay, 2048, 8) == (0, [])
    finally:
        exl3._DMA_B, exl3._DMA_NS = saved
        ct_vllm.reset()
