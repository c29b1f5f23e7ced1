"""The reference's expert-tier hook surface (ct/ct_vllm.py) over this library.

  install(X)                  wraps X.apply_exl3_fused_moe with the split/combine entry and
                              X.Exl3MoEMethod.process_weights_after_loading with register (ct_vllm.py:446-456)
  register(layer)             a layer with host-resident experts joins the tier: its slot table (_ct) is set up
                              (ct_vllm.py:89-117)
  _fused(x2d, ids, weights, layer, inners, expert_map, limit)
                              decode-sized calls: mm_split classifies the picks against the slot table (hits /
                              misses per distinct expert, routed counts for the cache), the fused MoE runs, and
                              mm_combine_host adds a host partial when one was published (ct_vllm.py:175-223)
  _ec_point, ec_step, ec_release, ec_rewarm, ec_summary, summary
                              the slot table and the elastic expert cache (ct_vllm.py:236-443), on
                              cache.ExpertCache
  before_step(ntok)           the engine-step hook's part before a step (ct_vllm.py:459-475): release the cache
                              before prefill-sized steps; the hook calls ec_step after every step
  install_step_hook(modules)  wraps GPUModelRunner.execute_model of the engine's model-runner modules with
                              before_step / ec_step (ct_vllm.py:459-488); install(X) calls it

  calibrate(), set_policy(...)  the split's cost-model constants measured on this machine (per-expert time of a
                              zero-copy miss on the GPU and of an expert on the host tier), or set by hand

With DSV41_CPU_TIER=1 the host tier (mi355moe.tier, the library's mm_tier_*) serves the picks the split sends
to the host: the split's cost model (ct/ft_tier_cu_v.cu:35-62) chooses how many of the call's misses the host
cores compute from their pinned home rows while the GPU reads the rest zero-copy over PCIe and computes its
share; the combine then adds the host partial (bounded wait, DSV41_CT_TIMEOUT_S). Without it the policy's
force_n is 0 and every routed expert runs on the GPU.

Hybrid prefill tail (ct/ct_vllm.py:163-225; DSV41_CT_HYB_MAX, 0 = off): a lone step of maxbsz < T <= HYB_MAX
tokens on a layer with staged experts gives the host tier the trailing staging batches (_hyb_tail's cost model:
host time per expert against copy time per expert), so the copy engine streams fewer experts while the host
cores compute the tail: the split marks the tail experts as misses (a slot table with -1 for them only) and
sends every one of their picks to the host, the staged prefill skips those batches, and the combine adds the
host partial.
"""
import importlib
import json
import os

import numpy as np
import torch

from . import _lib, cache, exl3
from . import tier as _tier
from .hostmem import HostBuffer

S = {"layers": [], "started": False, "init": False, "selftest": None, "cpu_tier": False}
EC = {"cache": None}
_ORIG = {}


def _f(k, d):
    return float(os.environ.get(k, d))


def _init(layer):
    dev = layer._exl3_ptrs["gate_trellis"].device
    H = layer.H
    maxbsz = int(os.environ.get("DSV41_CT_MAXBSZ", "32"))
    hyb = int(os.environ.get("DSV41_CT_HYB_MAX", "0"))        # hybrid DMA + host-tail range (maxbsz, hyb]; 0 = off
    buf = max(maxbsz, hyb)
    S.update(H=H, I=layer.I, dev=dev, maxbsz=maxbsz, maxpicks=8 * buf, hyb_max=hyb, buf=buf)
    # host mailbox (ct_vllm.py:58-65), pinned and device-mapped: ctrl int64 [16] | hx fp16 [buf * H] |
    # picks int32 [maxpicks * 3] | hout fp32 [buf * H] (the host worker's partial, read by mm_combine_host)
    o_hx, o_pk = 128, 128 + buf * H * 2
    o_out = (o_pk + S["maxpicks"] * 12 + 255) // 256 * 256
    S["mail"] = HostBuffer(o_out + buf * H * 4)
    S["mail"].array(np.uint8)[:] = 0
    S["ctrl"] = S["mail"].data_ptr(0)
    S["hx"] = S["mail"].data_ptr(o_hx)
    S["picks"] = S["mail"].data_ptr(o_pk)
    S["hout"] = S["mail"].data_ptr(o_out)
    S["dflag"] = torch.zeros(1, dtype=torch.int64, device=dev)
    S["seqc"] = torch.zeros(1, dtype=torch.int64, device=dev)
    S["stats"] = torch.zeros(8, dtype=torch.int64, device=dev)
    # cost-model policy (ct_vllm.py:69-71): without the host tier force_n = 0 sends nothing to the host
    S["cpu_tier"] = os.environ.get("DSV41_CPU_TIER", "0") == "1"
    force = _f("DSV41_CT_FORCE_N", -1) if S["cpu_tier"] else 0.0
    S["pol"] = torch.tensor([_f("DSV41_CT_TZC", 0.58), _f("DSV41_CT_THIT", 0.03), _f("DSV41_CT_A", 0.11),
                             _f("DSV41_CT_B", 0.16), _f("DSV41_CT_TOK", 0.2), _f("DSV41_CT_MAXN", 64), force, 0.0, 0.0],
                            dtype=torch.float32, device=dev)
    # hybrid: every miss to the host (force_n = all), and the x rows copied by the copy engine (ct_vllm.py:75-78);
    # the "misses" are exactly the tail experts (the tail's slot table)
    S["pol_hyb"] = torch.tensor([0.54, 0.0, 0.0, 0.0, 0.0, 4096.0, 4096.0, 0.0, 1.0], dtype=torch.float32, device=dev)
    S["stats_hyb"] = torch.zeros(8, dtype=torch.int64, device=dev)
    S["hyb_n"] = 0
    S["hyb_cost"] = {"c0": _f("DSV41_HYB_C0", 0.24), "c1": _f("DSV41_HYB_C1", 0.085), "dma": _f("DSV41_HYB_DMA", 0.54),
                     "tok_us": _f("DSV41_HYB_TOK_US", 6.0), "max_batches": int(_f("DSV41_HYB_MAX_BATCHES", 24))}
    S["timeout_ns"] = int(_f("DSV41_CT_TIMEOUT_S", 2) * 1e9)
    S["sel"] = torch.empty(S["maxpicks"], dtype=torch.long, device=dev)
    S["w"] = torch.empty(S["maxpicks"], dtype=torch.float32, device=dev)
    S["nlayers"] = int(os.environ.get("DSV41_CT_LAYERS", "40"))
    if S["cpu_tier"]:
        _tier.init(H, layer.I, S["nlayers"], mailbox={"ctrl": S["ctrl"], "hx": S["hx"], "picks": S["picks"],
                                                        "hout": S["hout"], "maxtok": buf,
                                                        "maxpicks": S["maxpicks"], "owner": S["mail"]})
        S["limit"] = _f("DSV41_CT_LIMIT", 10.0)
        _tier.set_limit(S["limit"] if S["limit"] > 0 else 0.0)
    S["init"] = True


def register(layer, nlayers=None):
    """Join the tier (layers whose experts have a pinned host home). The tier starts once `nlayers` layers
    (DSV41_CT_LAYERS, 40) are registered."""
    if layer.host_home is None:
        return
    if not S["init"]:
        _init(layer)
    if nlayers is not None:
        S["nlayers"] = int(nlayers)
    li = len(S["layers"])
    if li >= S["nlayers"]:
        return
    dev = S["dev"]
    layer._ct = {"li": li, "E": layer.E, "slotof": layer.slotof,
                 "score": torch.zeros(layer.E, dtype=torch.float32, device=dev), "counts": layer.counts,
                 "home": layer.home}
    if S["cpu_tier"]:
        _tier.add_layer(li, layer)          # home rows read in place, host copies of the scales (ct_vllm.py:97-110)
    S["layers"].append(layer)
    if len(S["layers"]) == S["nlayers"]:
        start()


def selftest(layers=None):
    """The host tier against the GPU path on the same cold experts (ct_vllm.py:123-140): x ~ N(0, 0.35^2) fp16, six
    random host-resident experts with weight 0.25, 1 and 3 tokens, up to three layers; returns the largest relative
    L2 difference of the weighted sums."""
    res = []
    g = torch.Generator(device="cpu").manual_seed(0)
    layers = S["layers"] if layers is None else layers
    orig = _ORIG.get("fused", exl3.apply_exl3_fused_moe)
    for layer in layers[:: max(1, len(layers) // 3)][:3]:
        cold = [e for e in range(layer.E) if int(layer.slotof[e]) < 0]
        for mt in (1, 3):
            x = (torch.randn(mt, S["H"], generator=g) * 0.35).half()
            exps = [cold[int(i)] for i in torch.randperm(len(cold), generator=g)[:6]]
            sel = torch.tensor([exps] * mt, dtype=torch.int32)
            w = torch.full((mt, 6), 0.25, dtype=torch.float32)
            cpu = torch.from_numpy(_tier.forward(layer._ct["li"], x.float().numpy(), sel.numpy(), w.numpy()))
            gpu = orig(x.to(S["dev"]), sel.long().to(S["dev"]), w.to(S["dev"]), layer, None, None,
                       S["limit"] if S["limit"] > 0 else None).float().cpu()
            res.append(float((cpu - gpu).norm() / gpu.norm().clamp_min(1e-12)))
    return {"max_rel_vs_gpu": round(max(res), 6), "n": len(res)}


def set_policy(tzc=None, thit=None, a=None, b=None, tok=None, maxn=None, force_n=None):
    """Set cost-model constants of the split's policy vector (ms per zero-copy miss, per resident hit, per host job,
    per host expert, extra-token factor, most host experts per call, forced host count or -1)."""
    p = S["pol"].cpu()
    for j, v in enumerate((tzc, thit, a, b, tok, maxn, force_n)):
        if v is not None:
            p[j] = float(v)
    S["pol"].copy_(p)


def calibrate(layer=None, experts=8):
    """Measure the policy's constants on this machine for one tier layer: a zero-copy miss (the GPU path on
    `experts` host-resident experts, one token), an HBM hit (the same experts from HBM copies is not needed: a hit
    streams the expert at HBM rate, taken as 1/400 of the miss), and the host tier on one and on `experts`
    experts (job overhead and per-expert time). Returns the constants set."""
    import time
    layer = S["layers"][0] if layer is None else layer
    orig = _ORIG.get("fused", exl3.apply_exl3_fused_moe)
    cold = [e for e in range(layer.E) if int(layer.slotof[e]) < 0][:experts]
    x = (torch.randn(1, S["H"]) * 0.35).half()
    xd = x.to(S["dev"])

    # each time is the median of 11 calls after 3 warm-up calls, so a call that the host's scheduler delays does
    # not set the policy

    def gpu_t(ids):
        idd = torch.tensor([ids], dtype=torch.long, device=S["dev"])
        wd = torch.full((1, len(ids)), 1.0 / len(ids), device=S["dev"])
        ts = []
        for r in range(14):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            orig(xd, idd, wd, layer, None, None, 10.0)
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts[3:])) * 1e3

    def cpu_t(ids):
        sel = np.array([ids], np.int32)
        ww = np.full((1, len(ids)), 1.0 / len(ids), np.float32)
        xf = x.float().numpy()
        ts = []
        for r in range(14):
            t0 = time.perf_counter()
            _tier.forward(layer._ct["li"], xf, sel, ww)
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts[3:])) * 1e3

    def cpu_rows_t(rows):
        # `rows` tokens, each routed to every one of the experts: ms per expert
        sel = np.tile(np.array(cold, np.int32), (rows, 1))
        ww = np.full(sel.shape, 1.0 / len(cold), np.float32)
        xf = (torch.randn(rows, S["H"]) * 0.35).half().float().numpy()
        ts = []
        for r in range(5):
            t0 = time.perf_counter()
            _tier.forward(layer._ct["li"], xf, sel, ww)
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts[1:])) * 1e3 / len(cold)

    def cpu_tok_t(T):
        # the per-token part of a job (every output row written) with no picks: ms per token
        sel = np.full((T, 1), -1, np.int32)
        xf = np.zeros((T, S["H"]), np.float32)
        ts = []
        for r in range(5):
            t0 = time.perf_counter()
            _tier.forward(layer._ct["li"], xf, sel, np.zeros((T, 1), np.float32))
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts[1:])) * 1e3 / T

    zc = gpu_t(cold) / len(cold)
    serving = _tier.serving()
    if serving:                     # synchronous host forwards need the mailbox worker stopped
        _tier.stop()
    try:
        c1, cn = cpu_t(cold[:1]), cpu_t(cold)
        hyb = S.get("hyb_max", 0) > 0
        if hyb:
            r1, rr = cpu_rows_t(1), cpu_rows_t(32)
            tok = cpu_tok_t(2048)
    finally:
        if serving:
            _tier.start()
    b = max((cn - c1) / max(1, len(cold) - 1), 1e-3)
    a = max(c1 - b, 0.0)
    set_policy(tzc=zc, thit=zc / 400.0, a=a, b=b)
    res = {"tzc": zc, "thit": zc / 400.0, "a": a, "b": b}
    if hyb:
        # copy time of one expert row through the staging copy stream (pinned home -> HBM)
        rows_b = cache.ExpertRows(S["H"], S["I"]).row_bytes
        dst = torch.empty(len(cold) * rows_b, dtype=torch.uint8, device=S["dev"])
        cs = _lib.copy_stream(S["dev"], _lib.COPY_STAGING)
        copies = [(dst.data_ptr() + i * rows_b, layer.host_home.row(e), rows_b) for i, e in enumerate(cold)]
        cache.stage_copy(copies, cs)
        cs.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(cs)
        cache.stage_copy(copies, cs)
        e1.record(cs)
        cs.synchronize()
        dma = e0.elapsed_time(e1) / len(cold)
        del dst
        S["hyb_cost"].update(c0=r1, c1=max((rr - r1) / 31.0, 0.0), dma=dma, tok_us=tok * 1e3)
        res["hybrid"] = dict(S["hyb_cost"])
    return res


def start(**ec_args):
    if S["started"]:
        return
    EC["cache"] = cache.ExpertCache(S["layers"], **ec_args)
    if S["cpu_tier"]:
        if os.environ.get("DSV41_CT_SELFTEST", "1") == "1":
            try:
                S["selftest"] = selftest()
            except Exception as exc:    # the diagnostic never blocks serving (ct_vllm.py:146-152)
                S["selftest"] = {"error": repr(exc)}
        _tier.start()
    S["started"] = True


def _hyb_tail(layer, T, k):
    """Trailing staging batches the host tier takes for a T-token step (ct_vllm.py:163-178): the host time of
    n experts, n (C0 + C1 (rows - 1)) ms at rows = k T / E routes per expert, against the copy time of the rest,
    DMA ms per expert, after a per-token input cost TOK_US; at most MAX_BATCHES, and at least the NS batches the
    copy engine starts with stay staged. Returns (batches, the tail's experts)."""
    if getattr(layer, "_exl3_dma", None) is None:
        return 0, []
    batches = exl3._dma_batches(layer)
    nb = len(batches)
    if nb == 0:
        return 0, []
    c = S["hyb_cost"]
    staged = sum(len(b) for b in batches)
    rows = k * T / layer.E
    c_cpu = c["c0"] + c["c1"] * max(0.0, rows - 1)
    fixed = c["tok_us"] * T / 1000.0
    n_cpu = max(0.0, (staged * c["dma"] - fixed) / (c["dma"] + c_cpu))
    kc = int(n_cpu // exl3._DMA_B)
    kc = max(0, min(kc, nb - exl3._DMA_NS, c["max_batches"]))
    return kc, [e for b in batches[nb - kc:] for e in b]


def _hybrid(x2d, ids, weights, layer, inners, limit, kc, tail):
    """One hybrid step (ct_vllm.py:186-213): the tail's experts to the host tier, the rest staged."""
    ct = layer._ct
    T = x2d.shape[0]
    dev = S["dev"]
    orig = _ORIG.get("fused", exl3.apply_exl3_fused_moe)
    key = (kc, tuple(tail))
    fake = ct.setdefault("hyb_slot", {}).get(key)
    if fake is None:
        f = np.zeros(ct["E"], np.int32)
        f[tail] = -1
        fake = torch.from_numpy(f).to(dev)
        ct["hyb_slot"] = {key: fake}            # the tail changes with the cache's residency: keep the latest
    n = ids.numel()
    so, wo = S["sel"][:n], S["w"][:n]
    z = x2d if (x2d.dtype == torch.half and x2d.is_contiguous()) else x2d.half().contiguous()
    # the x rows to the mailbox on the copy engine, on this stream, before the split publishes (pol[8] = 1)
    cache.stage_copy([(S["hx"], z.data_ptr(), z.numel() * 2)], torch.cuda.current_stream(dev))
    cnt = ct.get("hyb_cnt")
    if cnt is None:
        cnt = ct["hyb_cnt"] = torch.zeros(ct["E"], dtype=torch.int32, device=dev)
    idc = ids.contiguous().long()
    wc = weights.contiguous().float()
    _lib.call("mm_split", idc.data_ptr(), wc.data_ptr(), z.data_ptr(), n, T, S["H"], ct["E"], fake.data_ptr(),
              ct["score"].data_ptr(), S["pol_hyb"].data_ptr(), S["ctrl"], S["hx"], S["picks"], S["seqc"].data_ptr(),
              ct["li"], so.data_ptr(), wo.data_ptr(), S["dflag"].data_ptr(), S["stats_hyb"].data_ptr(),
              cnt.data_ptr(), None, None, None, _lib.stream_ptr())
    layer._hyb_tail = kc
    try:
        out = orig(x2d, so.view(ids.shape), wo.view(weights.shape).to(weights.dtype), layer, inners, None, limit)
    finally:
        layer._hyb_tail = 0
    _lib.call("mm_combine_host", out.data_ptr(), out.numel(), S["dflag"].data_ptr(), S["ctrl"], S["hout"],
              S["stats_hyb"].data_ptr(), S["timeout_ns"], _lib.stream_ptr())
    S["hyb_n"] += 1
    S["hyb_last"] = {"tokens": T, "batches": kc, "experts": len(tail)}
    return out


def _fused(x2d, ids, weights, layer, inners, expert_map, limit):
    """Split / fused MoE / combine for decode-sized calls of tier layers, the hybrid tail for lone prefill steps
    up to DSV41_CT_HYB_MAX tokens; everything else goes to the plugin's own entry unchanged
    (ct_vllm.py:181-223)."""
    ct = getattr(layer, "_ct", None)
    T = x2d.shape[0]
    orig = _ORIG.get("fused", exl3.apply_exl3_fused_moe)
    if (ct is not None and S["started"] and S["cpu_tier"] and expert_map is None and S.get("hyb_max", 0)
            and S["maxbsz"] < T <= S["hyb_max"] and S.get("solo", True) and ids.numel() <= S["maxpicks"]
            and inners is None and not torch.cuda.is_current_stream_capturing()):
        kc, tail = _hyb_tail(layer, T, ids.reshape(T, -1).shape[1])
        if kc > 0:
            return _hybrid(x2d, ids, weights, layer, inners, limit, kc, tail)
    if ct is None or not S["started"] or T > S["maxbsz"] or expert_map is not None or ids.numel() > S["maxpicks"]:
        return orig(x2d, ids, weights, layer, inners, expert_map, limit)
    n = ids.numel()
    so, wo = S["sel"][:n], S["w"][:n]
    z = x2d if (x2d.dtype == torch.half and x2d.is_contiguous()) else x2d.half().contiguous()
    idc = ids.contiguous().long()
    wc = weights.contiguous().float()
    _lib.call("mm_split", idc.data_ptr(), wc.data_ptr(), z.data_ptr(), n, T, S["H"], ct["E"], ct["slotof"].data_ptr(),
              ct["score"].data_ptr(), S["pol"].data_ptr(), S["ctrl"], S["hx"], S["picks"], S["seqc"].data_ptr(),
              ct["li"], so.data_ptr(), wo.data_ptr(), S["dflag"].data_ptr(), S["stats"].data_ptr(),
              ct["counts"].data_ptr(), None, None, None, _lib.stream_ptr())
    out = orig(x2d, so.view(ids.shape), wo.view(weights.shape).to(weights.dtype), layer, inners, expert_map, limit)
    if out.dtype != torch.float32 or not out.is_contiguous():
        raise RuntimeError("mi355moe ct_vllm: expected the fp32 contiguous routed accumulator")
    _lib.call("mm_combine_host", out.data_ptr(), out.numel(), S["dflag"].data_ptr(), S["ctrl"], S["hout"],
              S["stats"].data_ptr(), S["timeout_ns"], _lib.stream_ptr())
    return out


# ------------------------------------------------------------------------------------------ slot table / cache

def _ec_point(layer, items):
    """items: [(e, gate_ptr, up_ptr, down_ptr, slot_or_-1)] -> stream-ordered pointer-table + slotof update."""
    cache.point(layer, items)


def ec_step():
    c = EC["cache"]
    if c is None or not S["started"]:
        return
    c.step()


def ec_release():
    c = EC["cache"]
    if c is not None:
        c.release()


def ec_rewarm():
    c = EC["cache"]
    if c is not None:
        c.rewarm()


def ec_summary():
    c = EC["cache"]
    return c.summary() if c is not None else None


def summary():
    if not S["started"]:
        return None
    st = S["stats"].tolist()
    calls = max(1, st[3])
    h = _tier.stats() if S["cpu_tier"] else {"jobs": 0, "busy_ns": 0}
    hy = S["stats_hyb"].tolist()
    hyb = {"calls": hy[3], "host_experts": hy[2], "timeouts": hy[6], "last": S.get("hyb_last")} if hy[3] else None
    return {"calls": st[3], "hits": st[0], "misses": st[1], "cpu_experts": st[2], "cpu_per_call": round(st[2] / calls, 3),
            "hybrid": hyb,
            "gpu_wait_ms": round(st[4] / 1e6 / max(1, st[5]), 4), "timeouts": st[6], "host_jobs": h["jobs"],
            "host_busy_ms": round(h["busy_ns"] / 1e6 / max(1, h["jobs"]), 4), "selftest": S["selftest"],
            "hit_rate": round(st[0] / max(1, st[0] + st[1]), 4), "ec": ec_summary()}


def before_step(ntok, solo=None):
    """Before an engine step of `ntok` scheduled tokens: release the cache before prefill-sized steps (elastic
    cache); `solo` (one request in the step, when known) gates the hybrid prefill tail, which the reference runs
    for a lone request only (ct_vllm.py:525). ec_step() follows the step."""
    if solo is not None:
        S["solo"] = bool(solo)
    c = EC["cache"]
    if c is None:
        return
    c.last_ntok = int(ntok)
    if ntok > c.prefill_tokens and c.elastic:
        c.release()


RUNNER_MODULES = ("vllm.v1.worker.gpu.model_runner", "vllm.v1.worker.gpu_model_runner")


def install_step_hook(modules=RUNNER_MODULES):
    """Wrap GPUModelRunner.execute_model of each importable module in `modules` (the engine's model runners,
    ct/ct_vllm.py:459-488): before the step, before_step(total scheduled tokens) (the elastic cache's release
    before prefill-sized steps); after it, ec_step(). Errors inside the hook are counted (S["hook_errors"]) and
    never reach the engine. Returns the module names hooked; modules that do not import are skipped."""
    hooked = []
    for name in modules:
        try:
            mod = importlib.import_module(name)
        except Exception:
            continue
        cls = getattr(mod, "GPUModelRunner", None)
        if cls is None or getattr(cls.execute_model, "_mi355moe_step_hook", False):
            continue
        orig = cls.execute_model

        def execute_model(self, *a, _o=orig, **k):
            try:
                so = a[0] if a else k.get("scheduler_output")
                reqs = getattr(so, "num_scheduled_tokens", None)
                before_step(int(getattr(so, "total_num_scheduled_tokens", 0) or 0),
                            solo=(len(reqs) <= 1) if isinstance(reqs, dict) else None)
            except Exception:
                S["hook_errors"] = S.get("hook_errors", 0) + 1
            r = _o(self, *a, **k)
            try:
                ec_step()
            except Exception:
                S["hook_errors"] = S.get("hook_errors", 0) + 1
            return r
        execute_model._mi355moe_step_hook = True
        cls.execute_model = execute_model
        _ORIG.setdefault("runners", []).append((cls, orig))
        hooked.append(name)
    return hooked


def install(X, runner_modules=RUNNER_MODULES):
    """Wrap the plugin module X (exl3 here, or any module with the same two names) and the engine's step
    (install_step_hook over runner_modules)."""
    if "fused" in _ORIG:
        return
    _ORIG["fused"] = X.apply_exl3_fused_moe
    X.apply_exl3_fused_moe = _fused
    orig_pwal = X.Exl3MoEMethod.process_weights_after_loading

    def pwal(self, layer, _o=orig_pwal):
        _o(self, layer)
        register(layer)
    X.Exl3MoEMethod.process_weights_after_loading = pwal
    _ORIG["pwal"] = orig_pwal
    S["step_hooks"] = install_step_hook(runner_modules)


def uninstall(X):
    if "fused" not in _ORIG:
        return
    X.apply_exl3_fused_moe = _ORIG.pop("fused")
    X.Exl3MoEMethod.process_weights_after_loading = _ORIG.pop("pwal")
    for cls, orig in _ORIG.pop("runners", []):
        cls.execute_model = orig


def reset():
    """Forget every registered layer, the cache and the host tier (tests, benchmarks). The tier is shut down
    before the mailbox it reads is released."""
    if _tier.running():
        _tier.shutdown()
    S.clear()
    S.update({"layers": [], "started": False, "init": False, "selftest": None, "cpu_tier": False})
    EC["cache"] = None


def dumps():
    return json.dumps(summary())
