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
