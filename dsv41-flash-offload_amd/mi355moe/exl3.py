"""The vllm_exl3 MoE entry points the reference patches (patches/vllm-exl3-host-dma.patch), over this library.

  apply_exl3_fused_moe(x2d, ids, weights, layer, inners, expert_map, limit) -> contiguous fp32 [T, H]
      the fused-MoE call (patch:241-449): routes of experts with more than FAT_EXPERT_THRESHOLD rows go to the
      fat-expert grouped GEMM, the rest to the decode path; with host-resident experts and at least
      _DMA_MIN_TOKENS tokens, the experts not in HBM are streamed through staging slots (EXL3_HOST_DMA).
  apply_exl3_batched_fat(xh, token_sorted, weight_sorted, counts_host, inners, limit, cap, out, use_kernel, skip)
      the fat-expert entry on expert-sorted routes (patch:182-201), accumulating into out.
  Exl3MoEMethod.process_weights_after_loading(layer)
      load-time hook; registers a layer with host-resident experts for the staging path (patch:27-56).

`layer` is an ExpertStore. `inners` is the per-expert list of {"gate", "up", "down"} matrices (Exl3Linear:
a trellis address plus the layer the scales come from), as layer_inners() builds it; None means the layer's own
pointer tables. Routing weights are used in fp16, as the plugin's flat_weight = weights.half() (patch:215) is.
"""
import os

import numpy as np
import torch

from . import _lib, cache, moe

SWIGLU_LIMIT_DEFAULT = 10.0


def _ienv(name, default):
    v = os.environ.get(name, "")
    try:
        return int(v) if v != "" else int(default)
    except ValueError:
        return int(default)


# default: the reference image's value (docker/entrypoint.sh:69); the plugin's own default is 256
FAT_EXPERT_THRESHOLD = max(0, _ienv("VLLM_EXL3_FAT_THRESHOLD", 32))
_EXL3_HOST_DMA_MODE = _ienv("EXL3_HOST_DMA", 0)
_DMA_B = _ienv("EXL3_HOST_DMA_BATCH", 16)
_DMA_NS = _ienv("EXL3_HOST_DMA_SLOTS", 3)
_DMA_MIN_TOKENS = _ienv("EXL3_HOST_DMA_MIN_TOKENS", 65)

# cross-layer prefetch (runtime/patch_dma_prefetch.py:17-36): after a layer's last staged batch, the next layer's
# first NS batches are queued on the copy engine, each behind the last reader of its slot
_DMA_PREFETCH = os.environ.get("EXL3_DMA_STOCK_PREFETCH", "1") == "1"
_DMA_STATE = {}         # device index -> {"slots": SlotPool [NS * B rows], "copy": Stream, "free": [Event | None] * NS}
_DMA_LAST = {}          # device index -> the last layer registered for staging (links each layer to the next)
_WS = {}                # device index -> reusable workspace tensor of the staged path
_DMA_TIMING = None      # a list to collect (start event, end event, bytes) of every staged copy, or None


class Exl3Linear:
    """One expert matrix: `trellis` (a tensor, or a device / host address) of expert `e`'s `key` matrix of
    `layer` (whose stacked parameters hold the scales)."""

    def __init__(self, layer, e, key, trellis):
        self.layer, self.e, self.key, self.trellis = layer, e, key, trellis

    def address(self):
        t = self.trellis
        return int(t.data_ptr()) if hasattr(t, "data_ptr") else int(t)


def layer_inners(layer):
    """Per-expert {"gate", "up", "down"} matrices at the layer's current pointer-table addresses."""
    hp = torch.stack([layer._exl3_ptrs[k] for k in ("gate_trellis", "up_trellis", "down_trellis")], 1).cpu().tolist()
    return [{k: Exl3Linear(layer, e, k, hp[e][j]) for j, k in enumerate(("gate", "up", "down"))}
            for e in range(layer.E)]


def _view(layer, limit, inners=None):
    """The layer with SwiGLU clamp `limit` (None or <= 0: no clamp) and, if `inners` is given, pointer tables
    built from its trellis addresses."""
    lim = float(limit) if (limit is not None and limit > 0) else 0.0
    if inners is None and lim == layer.limit:
        return layer
    if inners is not None:
        dev = layer._exl3_ptrs["gate_trellis"].device
        a = np.array([[inners[e][k].address() for e in range(layer.E)] for k in ("gate", "up", "down")], np.int64)
        t = torch.from_numpy(a).pin_memory().to(dev, non_blocking=True)
        v = layer.with_tables(t[0], t[1], t[2])
    else:
        v = layer.with_tables(*(layer._exl3_ptrs[k] for k in ("gate_trellis", "up_trellis", "down_trellis")))
    v.limit = lim
    return v


def _fat_ws(dev, n, T, E, H, I):
    need = _lib.load().mm_fat_batched_workspace(n, T, E, H, I)
    key = dev.index if dev.index is not None else 0
    ws = _WS.get(key)
    if ws is None or ws.numel() < need:
        ws = _WS[key] = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    return ws, need


def apply_exl3_batched_fat(xh, token_sorted, weight_sorted, counts_host, inners, limit, cap, out, use_kernel=True,
                           skip=None, layer=None):
    """Fat experts on expert-sorted routes (patch:182-201): for every expert e with counts_host[e] > cap that is
    not in `skip`, out[t] += w * expert_e(xh[t]) over its rows token_sorted / weight_sorted[offset_e ..
    offset_e + counts_host[e]). One grouped-GEMM path (use_kernel is accepted for the signature; there is no
    reconstruct fallback). `layer` defaults to the layer of `inners`."""
    if layer is None:
        if inners is None:
            raise ValueError("apply_exl3_batched_fat: need inners or layer")
        layer = inners[0]["gate"].layer
    L = _view(layer, limit, inners)
    dev = xh.device
    T, E = xh.shape[0], layer.E
    n = int(token_sorted.numel())
    if n == 0:
        return out
    counts = torch.as_tensor(np.asarray(counts_host, dtype=np.int64)[:E].astype(np.int32)) if not torch.is_tensor(
        counts_host) else counts_host[:E].to(torch.int32)
    counts = counts.to(dev, non_blocking=True).contiguous()
    sk = None
    if skip:
        m = np.zeros(E, np.uint8)
        m[[e for e in skip if 0 <= e < E]] = 1
        sk = torch.from_numpy(m).pin_memory().to(dev, non_blocking=True)
    tok = token_sorted.reshape(-1).to(torch.int64).contiguous()
    wsd = weight_sorted.reshape(-1).to(torch.float16).contiguous()
    x = xh.contiguous()
    ws, need = _fat_ws(dev, n, T, E, layer.H, layer.I)
    _lib.call("mm_fat_batched", L.mm_layer(), x.data_ptr(), moe.x_dtype_of(x), T, n, tok.data_ptr(), wsd.data_ptr(),
              counts.data_ptr(), None if sk is None else sk.data_ptr(), int(cap), out.data_ptr(), ws.data_ptr(), need,
              _lib.stream_ptr())
    return out


# ------------------------------------------------------------------------------------------ host DMA staging

def _dma_register(layer, dev=None):
    """Load time (patch:27-48): the device's staging slots (NS x B expert rows, once per device) for a layer whose
    experts have a pinned host home."""
    if layer.host_home is None:
        return False
    dev = layer._exl3_ptrs["gate_trellis"].device if dev is None else dev
    key = dev.index if dev.index is not None else 0
    st = _DMA_STATE.get(key)
    if st is None:
        st = _DMA_STATE[key] = {"slots": cache.SlotPool(_DMA_NS * _DMA_B, layer.H, layer.I, dev), "copy": None,
                                "free": [None] * _DMA_NS, "shape": (layer.H, layer.I), "owner": [None] * _DMA_NS}
    if st["shape"] != (layer.H, layer.I):
        return False
    layer._exl3_dma = {"tables": None, "copied": 0, "bytes": 0, "batches": 0, "pre": {}, "next": None,
                       "prefetched": 0}
    prev = _DMA_LAST.get(key)
    if prev is not None and getattr(prev, "_exl3_dma", None) is not None:
        prev._exl3_dma["next"] = layer
    _DMA_LAST[key] = layer
    return True


def _dma_batches(layer):
    """Staging batches of a layer: its host-resident experts that are not in an HBM slot (ascending id, from the
    host mirror of the slot table), B per batch. Known before the layer's routing, as the reference's are (every
    cold expert of the host plan, patch:31-52), so the previous layer can queue the first copies."""
    cold = [e for e in range(layer.E) if layer.slot_host[e] < 0]
    return [cold[i:i + _DMA_B] for i in range(0, len(cold), _DMA_B)]


def _dma_tables(layer):
    """The layer's staged pointer tables (a copy of its tables whose staged experts are repointed per batch)."""
    D = layer._exl3_dma
    if D["tables"] is None:
        D["tables"] = {k: layer._exl3_ptrs[k].clone() for k in ("gate_trellis", "up_trellis", "down_trellis")}
    return D["tables"]


def _dma_issue(layer, sl, experts, dev):
    """Copy the listed experts' home rows into staging slot `sl` rows 0 .. len - 1 on the copy stream, after the
    slot's last reader (patch:100-124). Returns the copy's event."""
    key = dev.index if dev.index is not None else 0
    st = _DMA_STATE[key]
    cs = st["copy"] = _lib.copy_stream(dev, _lib.COPY_STAGING)
    if st["free"][sl] is not None:
        cs.wait_event(st["free"][sl])
    pool = st["slots"]
    rb = pool.rows.row_bytes
    st["owner"][sl] = (id(layer), tuple(experts))       # what the slot holds once the copy has run
    cl = [(pool.row(sl * _DMA_B + r), layer.host_home.row(e), rb) for r, e in enumerate(experts)]
    D = layer._exl3_dma
    timing = _DMA_TIMING
    if timing is not None:
        t0 = torch.cuda.Event(enable_timing=True)
        t0.record(cs)
    D["copied"] += cache.stage_copy(cl, cs)
    D["bytes"] += rb * len(cl)
    ev = torch.cuda.Event(enable_timing=timing is not None)
    ev.record(cs)
    if timing is not None:
        timing.append((t0, ev, rb * len(cl)))
    return ev


def _dma_prefill(x2d, ids, w16, layer, limit, dev):
    """Prefill with host-resident experts: the experts in HBM (slot or home) in one grouped-GEMM pass on the
    layer's tables, then the host-resident experts in batches of B through NS staging slots: the copy of batch
    j + NS overlaps the compute of batch j (patch_dma_stock.py:41-52 with the busy-expert GEMM of
    runtime/dma_gemm.py). Unrouted experts of a batch are copied and skipped. The first NS batches may already be
    in flight, queued by the previous layer; after the last batch the next layer's first NS batches are queued.
    No host synchronisation."""
    T, E = x2d.shape[0], layer.E
    k = ids.shape[1]
    n = T * k
    key = dev.index if dev.index is not None else 0
    st = _DMA_STATE[key]
    D = layer._exl3_dma
    main = torch.cuda.current_stream(dev)
    routes = moe.permute(ids, w16, k, E)
    out = torch.zeros((T, layer.H), dtype=torch.float32, device=dev)
    tok = routes["token_sorted"][:n].to(torch.int64)
    wsd = routes["weight_sorted"][:n].to(torch.float16)
    counts_d = routes["counts"][:E]
    ws, need = _fat_ws(dev, n, T, E, layer.H, layer.I)
    batches = _dma_batches(layer)
    # a hybrid step's trailing batches belong to the host tier (its routes arrive masked): neither copied nor
    # computed here (runtime/patch_dma_prefetch.py:21)
    tail = int(getattr(layer, "_hyb_tail", 0) or 0)
    if tail > 0:
        batches = batches[:max(0, len(batches) - tail)]
        D["tail_skipped"] = D.get("tail_skipped", 0) + tail
    skip_e = {e for b in _dma_batches(layer)[len(batches):] for e in b} if tail > 0 else set()
    staged_e = {e for b in batches for e in b}
    masks = np.ones((len(batches) + 1, E), np.uint8)
    masks[0, [e for e in range(E) if e not in staged_e and e not in skip_e]] = 0   # row 0: the HBM-resident experts
    items = np.zeros((max(len(batches), 1), _DMA_B, 5), np.int64)
    items[:, :, 0] = -1
    pool = st["slots"]
    for j, b in enumerate(batches):
        masks[j + 1, b] = 0
        sl = j % _DMA_NS
        for r, e in enumerate(b):
            g, u, d = pool.addrs(sl * _DMA_B + r)
            items[j, r] = (e, g, u, d, sl * _DMA_B + r)
    masks_d = torch.from_numpy(masks).pin_memory().to(dev, non_blocking=True)
    items_d = torch.from_numpy(items).pin_memory().to(dev, non_blocking=True)
    L = _view(layer, limit)
    x = x2d.contiguous()
    xdt = moe.x_dtype_of(x)

    def run(view, mask_row):
        _lib.call("mm_fat_batched", view.mm_layer(), x.data_ptr(), xdt, T, n, tok.data_ptr(), wsd.data_ptr(),
                  counts_d.data_ptr(), masks_d[mask_row].data_ptr(), 0, out.data_ptr(), ws.data_ptr(), need,
                  _lib.stream_ptr(main))

    pre, D["pre"] = D.get("pre") or {}, {}
    events = {}
    for j in range(min(_DMA_NS, len(batches))):
        p = pre.get(j)
        if p is not None and p[0] == batches[j] and st["owner"][j % _DMA_NS] == (id(layer), tuple(batches[j])):
            events[j] = p[1]                    # copied while the previous layer finished, slot not reused since
            D["prefetched"] += 1
        else:
            events[j] = _dma_issue(layer, j % _DMA_NS, batches[j], dev)
    if len(staged_e) + len(skip_e) < E:
        run(L, 0)
    if batches:
        tabs = _dma_tables(layer)
        staged = layer.with_tables(tabs["gate_trellis"], tabs["up_trellis"], tabs["down_trellis"])
        staged.limit = L.limit
        for j in range(len(batches)):
            main.wait_event(events.pop(j))
            _lib.call("mm_slot_point", tabs["gate_trellis"].data_ptr(), tabs["up_trellis"].data_ptr(),
                      tabs["down_trellis"].data_ptr(), None, E, items_d[j].data_ptr(), _DMA_B, _lib.stream_ptr(main))
            run(staged, j + 1)
            done = torch.cuda.Event()
            done.record(main)
            st["free"][j % _DMA_NS] = done
            if j + _DMA_NS < len(batches):
                events[j + _DMA_NS] = _dma_issue(layer, (j + _DMA_NS) % _DMA_NS, batches[j + _DMA_NS], dev)
        D["batches"] += len(batches)
    nxt = D.get("next")
    if _DMA_PREFETCH and nxt is not None and getattr(nxt, "_exl3_dma", None) is not None:
        nb = _dma_batches(nxt)
        nxt._exl3_dma["pre"] = {j: (nb[j], _dma_issue(nxt, j % _DMA_NS, nb[j], dev))
                                for j in range(min(_DMA_NS, len(nb)))}
    return out


# ------------------------------------------------------------------------------------------ fused MoE

def apply_exl3_fused_moe(x2d, ids, weights, layer, inners=None, expert_map=None, limit=None):
    """Routed MoE of one layer: contiguous fp32 [T, H] = sum_j fp16(w[t, j]) * expert_{ids[t, j]}(x_t) over the
    routes with a valid local expert (ids mapped through expert_map when given; -1 and out-of-range ids
    contribute nothing)."""
    T = x2d.shape[0]
    dev = x2d.device
    ids = ids.reshape(T, -1)
    if expert_map is not None:
        ids = expert_map.to(dev)[ids.long().clamp(min=0)].masked_fill(ids < 0, -1)
    ids = ids.long().contiguous()
    w16 = weights.reshape(T, -1).to(torch.float16).float().contiguous()
    k = ids.shape[1]
    n = T * k
    if T == 0:
        return torch.zeros((0, layer.H), dtype=torch.float32, device=dev)
    L = _view(layer, limit, inners)
    if (_EXL3_HOST_DMA_MODE > 0 and layer.host_home is not None and getattr(layer, "_exl3_dma", None) is not None
            and T >= _DMA_MIN_TOKENS and inners is None and not torch.cuda.is_current_stream_capturing()):
        return _dma_prefill(x2d, ids, w16, layer, limit, dev)
    # at most FAT_EXPERT_THRESHOLD tokens: every route on the decode path (the reference's fat_possible test);
    # above it the experts with more than FAT_EXPERT_THRESHOLD routes go to the fat-expert GEMM. Both are decided on
    # the device, so no call synchronises the host and every call can be captured in a graph.
    return moe.moe_forward(L, x2d, ids, w16, fat_threshold=FAT_EXPERT_THRESHOLD)


class Exl3MoEMethod:
    """The plugin's MoE method object; process_weights_after_loading registers layers with host-resident experts
    for the staging path."""

    def process_weights_after_loading(self, layer):
        if layer.host_home is not None and _EXL3_HOST_DMA_MODE > 0:
            _dma_register(layer)
