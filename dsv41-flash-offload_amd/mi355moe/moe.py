"""Routed-expert MoE layer on MI355X: routing prep, decode expert path and fixed-order combine.

Every computation runs in libmi355moe.so; this module allocates buffers and launches on the current stream.
"""
import torch

from . import _lib

# Default fat-expert threshold of moe_forward: experts with more routes than this in a call go to the fat-expert
# grouped GEMM (the reference image's VLLM_EXL3_FAT_THRESHOLD, docker/entrypoint.sh:69).
FAT_THRESHOLD = 32
# Routes per call the decode path routes in-kernel (more go through the permutation).
GEMV_ROUTE_MAX = 1024


def _i(t):
    return _lib.ptr(t)


def permute(ids, w, topk, E, stream=None):
    """Routing prep (patches/vllm-exl3-host-dma.patch:204-236,296-312), stable by (expert, route index).
    Returns dict of device tensors: counts [E+1], offsets [E+2], order, token_sorted, weight_sorted, inv_order,
    active [E], nactive [1]."""
    ids = ids.reshape(-1).contiguous().long()
    n = ids.numel()
    dev = ids.device
    w = None if w is None else w.reshape(-1).contiguous().float()
    o = {
        "counts": torch.empty(E + 1, dtype=torch.int32, device=dev),
        "offsets": torch.empty(E + 2, dtype=torch.int32, device=dev),
        "order": torch.empty(max(n, 1), dtype=torch.int32, device=dev),
        "token_sorted": torch.empty(max(n, 1), dtype=torch.int32, device=dev),
        "weight_sorted": torch.empty(max(n, 1), dtype=torch.float32, device=dev),
        "inv_order": torch.empty(max(n, 1), dtype=torch.int32, device=dev),
        "active": torch.empty(E, dtype=torch.int32, device=dev),
        "nactive": torch.empty(1, dtype=torch.int32, device=dev),
    }
    wsb = _lib.load().mm_permute_workspace(n, E)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    _lib.call("mm_permute", _i(ids), _i(w), n, topk, E, _i(o["counts"]), _i(o["offsets"]), _i(o["order"]),
              _i(o["token_sorted"]), _i(o["weight_sorted"]), _i(o["inv_order"]), _i(o["active"]), _i(o["nactive"]),
              _i(ws), wsb, _lib.stream_ptr(stream))
    return o


def x_dtype_of(x):
    """MM_DTYPE_* code of a layer input tensor."""
    import torch
    codes = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}
    if x.dtype not in codes:
        raise TypeError(f"mi355moe: layer input must be fp16, bf16 or fp32 (got {x.dtype})")
    return codes[x.dtype]


def expert_gemv(store, x, ids, T, n, topk, max_rows, routes=None, rescale=False, phases=31, stream=None):
    """Per-route expert outputs Y fp32 [n, H] (flat route order) on the decode path. x [T, H] is fp16 (used as
    is), bf16 or fp32 (through bf16). Routes are found in-kernel from ids, or taken from a permutation
    (`routes`, from permute())."""
    dev = x.device
    E, H, I = store.E, store.H, store.I
    wsb = _lib.load().mm_gemv_workspace(n, E, H, I)
    ws = torch.zeros(wsb, dtype=torch.uint8, device=dev)
    Y = torch.zeros((n, H), dtype=torch.float32, device=dev)
    ids = ids.reshape(-1).contiguous().long()
    x = x.contiguous()
    r = routes or {}
    _lib.call("mm_expert_gemv", store.mm_layer(), _i(x), x_dtype_of(x), 1 if rescale else 0, T, n, topk, _i(ids),
              _i(r.get("offsets")), _i(r.get("order")), _i(r.get("active")), _i(r.get("nactive")), int(max_rows),
              _i(Y), _i(ws), wsb, phases, _lib.stream_ptr(stream))
    return Y


def combine(Y, ids, w, T, k, H, E, out=None, stream=None):
    ids = ids.reshape(-1).contiguous().long()
    w = w.reshape(-1).contiguous().float()
    acc = out is not None
    if out is None:
        out = torch.empty((T, H), dtype=torch.float32, device=Y.device)
    _lib.call("mm_combine", _i(out), _i(Y), _i(ids), _i(w), T, k, H, E, 1 if acc else 0, _lib.stream_ptr(stream))
    return out


def _with_shared(ids, w, T, shared_expert):
    ids = ids.reshape(T, -1).long()
    w = w.reshape(T, -1).float()
    if shared_expert is not None:
        ids = torch.cat([ids, torch.full((T, 1), int(shared_expert), dtype=torch.long, device=ids.device)], 1)
        w = torch.cat([w, torch.ones((T, 1), dtype=torch.float32, device=w.device)], 1)
    return ids.contiguous(), w.contiguous()


def decode_routes(store, x, ids, w, cap, out=None, rescale=False, stream=None):
    """out fp32 [T, H] (+)= sum_j w[t, j] * expert_{ids[t, j]}(x_t) over the routes whose expert has at most `cap`
    routes in the call (the decode path; experts above the cap contribute nothing). ids int64 [T, k], w fp32
    [T, k]. No host synchronisation: routing is found in-kernel for up to GEMV_ROUTE_MAX routes (k <= 16), else
    through the permutation."""
    T, k = ids.shape
    n = T * k
    dev = x.device
    x = x.contiguous()
    cap = max(1, int(cap))
    if n <= GEMV_ROUTE_MAX and k <= 16 and out is None:
        out = torch.empty((T, store.H), dtype=torch.float32, device=dev)
        wsb = _lib.load().mm_gemv_workspace(n, store.E, store.H, store.I)
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
        _lib.call("mm_moe_decode", store.mm_layer(), _i(x), x_dtype_of(x), 1 if rescale else 0, T, k, _i(ids), _i(w),
                  cap, _i(out), _i(ws), wsb, _lib.stream_ptr(stream))
        return out
    routes = permute(ids, w, k, store.E, stream) if n > GEMV_ROUTE_MAX else None
    # rows of routes above the cap stay zero and add nothing in the combine
    Y = expert_gemv(store, x, ids, T, n, k, cap, routes, rescale=rescale, stream=stream)
    return combine(Y, ids, w, T, k, store.H, store.E, out=out, stream=stream)


def moe_forward(store, x, ids, w, shared_expert=None, fat_threshold=FAT_THRESHOLD, stream=None):
    """out fp32 [T, H] = sum_j w[t, j] * expert_{ids[t, j]}(x_t) (+ expert `shared_expert` with weight 1).

    Routes with ids outside [0, E) contribute nothing. As the reference's fused-MoE call does
    (patches/vllm-exl3-host-dma.patch:241-290), a call of at most `fat_threshold` tokens runs every route on the
    decode path; a larger call sends the experts with more than `fat_threshold` routes to the fat-expert grouped
    GEMM and the rest to the decode path. The split is made on the device (no host synchronisation), so every
    call can be captured in a HIP graph."""
    T = x.shape[0]
    ids, w = _with_shared(ids, w, T, shared_expert)
    k = ids.shape[1]
    n = T * k
    thr = max(0, int(fat_threshold))
    if T <= thr:
        return decode_routes(store, x, ids, w, n, stream=stream)
    if thr == 0 or k > 16:
        return moe_prefill(store, x, ids, w, cap=thr, stream=stream)
    return fused_moe(store, x, ids, w, thr, stream=stream)


def fused_moe(store, x, ids, w, cap, stream=None):
    """mm_fused_moe: out fp32 [T, H] over ids [T, k] / w [T, k], experts with more than `cap` routes on the
    grouped GEMM and the others on the decode path, split on the device."""
    T, k = ids.shape
    x = x.contiguous()
    ids = ids.contiguous().long()
    w = w.contiguous().float()
    wsb = _lib.load().mm_fused_moe_workspace(T, k, store.E, store.H, store.I, int(cap))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=x.device)
    out = torch.empty((T, store.H), dtype=torch.float32, device=x.device)
    _lib.call("mm_fused_moe", store.mm_layer(), _i(x), x_dtype_of(x), T, k, _i(ids), _i(w), int(cap), _i(out), _i(ws),
              wsb, _lib.stream_ptr(stream))
    return out


def _prefill_ws(store, n, dev):
    wsb = _lib.load().mm_prefill_workspace(n, store.E, store.H, store.I)
    return torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev), wsb


def grouped_gemm(store, x, ids, cap=0, stream=None):
    """Fat-expert path: per-route expert outputs Y fp32 [n, H] (flat route order) of every route whose expert has
    more than `cap` routes (other rows stay zero). Weights decoded as fp16, multiplied on MFMA."""
    T = x.shape[0]
    ids = ids.reshape(T, -1).contiguous().long()
    k = ids.shape[1]
    n = T * k
    x = x.contiguous()
    ws, wsb = _prefill_ws(store, n, x.device)
    Y = torch.zeros((n, store.H), dtype=torch.float32, device=x.device)
    _lib.call("mm_grouped_gemm", store.mm_layer(), _i(x), x_dtype_of(x), T, k, _i(ids), int(cap), _i(Y), _i(ws), wsb,
              _lib.stream_ptr(stream))
    return Y


def moe_prefill(store, x, ids, w, cap=0, out=None, shared_expert=None, stream=None):
    """Prefill MoE layer on the fat-expert path: out fp32 [T, H] (+)= sum_j w[t, j] * expert_{ids[t, j]}(x_t)
    over the routes whose expert has more than `cap` routes. With `out` given the sum is added to it (the
    reference's apply_exl3_batched_fat accumulation, patches/vllm-exl3-host-dma.patch:182-201)."""
    T = x.shape[0]
    ids, w = _with_shared(ids, w, T, shared_expert)
    k = ids.shape[1]
    x = x.contiguous()
    ws, wsb = _prefill_ws(store, T * k, x.device)
    acc = out is not None
    if out is None:
        out = torch.empty((T, store.H), dtype=torch.float32, device=x.device)
    _lib.call("mm_moe_prefill", store.mm_layer(), _i(x), x_dtype_of(x), T, k, _i(ids), _i(w), int(cap), 1 if acc else 0,
              _i(out), _i(ws), wsb, _lib.stream_ptr(stream))
    return out


class DecodeRunner:
    """Fixed-shape decode MoE layer with every buffer preallocated: no allocation and no host sync per call,
    so a sequence of layers can be captured in one HIP graph."""

    def __init__(self, E, H, I, T, k, device="cuda", shared=True, max_rows=None):
        self.E, self.H, self.I, self.T, self.k0 = E, H, I, T, k
        self.shared = shared
        self.Eall = E + (1 if shared else 0)
        self.k = k + (1 if shared else 0)
        self.n = T * self.k
        # the decode path's cap on routes per expert: every route by default
        self.max_rows = self.n if max_rows is None else max_rows
        dev = torch.device(device)
        self.ids = torch.zeros((T, self.k), dtype=torch.long, device=dev)
        self.w = torch.zeros((T, self.k), dtype=torch.float32, device=dev)
        if shared:
            self.ids[:, -1] = E
            self.w[:, -1] = 1.0
        n, Ea = self.n, self.Eall
        self.counts = torch.empty(Ea + 1, dtype=torch.int32, device=dev)
        self.offsets = torch.empty(Ea + 2, dtype=torch.int32, device=dev)
        self.order = torch.empty(n, dtype=torch.int32, device=dev)
        self.active = torch.empty(Ea, dtype=torch.int32, device=dev)
        self.nactive = torch.empty(1, dtype=torch.int32, device=dev)
        self.pws_bytes = _lib.load().mm_permute_workspace(n, Ea)
        self.pws = torch.empty(max(self.pws_bytes, 1), dtype=torch.uint8, device=dev)
        self.gws_bytes = _lib.load().mm_gemv_workspace(n, Ea, H, I)
        self.gws = torch.zeros(self.gws_bytes, dtype=torch.uint8, device=dev)
        self.Y = torch.zeros((n, H), dtype=torch.float32, device=dev)
        self.x16 = torch.empty((T, H), dtype=torch.float16, device=dev)
        self.out = torch.empty((T, H), dtype=torch.float32, device=dev)

    def set_routes(self, ids, w):
        self.ids[:, : self.k0].copy_(ids)
        self.w[:, : self.k0].copy_(w)

    def route(self, ids=None, w=None, stream=None):
        ids = self.ids if ids is None else ids
        w = self.w if w is None else w
        _lib.call("mm_permute", _i(ids), _i(w), self.n, self.k, self.Eall, _i(self.counts), _i(self.offsets),
                  _i(self.order), None, None, None, _i(self.active), _i(self.nactive), _i(self.pws), self.pws_bytes,
                  _lib.stream_ptr(stream))

    def experts(self, store, x=None, ids=None, phases=31, use_permutation=False, rescale=False, stream=None):
        """The expert kernels (phases: mask of 1 route prep, 2 gate/up partial sums, 4 gate/up epilogue, 8 down
        partial sums, 16 down epilogue -> Y); routes found in-kernel from ids (or from route()'s permutation)."""
        x = self.x16 if x is None else x
        ids = self.ids if ids is None else ids
        p = use_permutation
        _lib.call("mm_expert_gemv", store.mm_layer(), _i(x), x_dtype_of(x), 1 if rescale else 0, self.T, self.n,
                  self.k, _i(ids), _i(self.offsets) if p else None, _i(self.order) if p else None,
                  _i(self.active) if p else None, _i(self.nactive) if p else None, self.max_rows, _i(self.Y),
                  _i(self.gws), self.gws_bytes, phases, _lib.stream_ptr(stream))

    def combine(self, ids=None, w=None, out=None, stream=None):
        ids = self.ids if ids is None else ids
        w = self.w if w is None else w
        out = self.out if out is None else out
        _lib.call("mm_combine", _i(out), _i(self.Y), _i(ids), _i(w), self.T, self.k, self.H, self.Eall, 0,
                  _lib.stream_ptr(stream))
        return out

    def layer(self, store, x=None, ids=None, w=None, out=None, rescale=False, stream=None):
        """One decode MoE layer through mm_moe_decode (5 launches: route prep, gate/up partial sums + epilogue,
        down partial sums, down epilogue fused with the weighted combine). x is fp16, bf16 or fp32; a chain of
        layers passes the previous out (fp32), with rescale for the unit-RMS step between layers."""
        x = self.x16 if x is None else x
        ids = self.ids if ids is None else ids
        w = self.w if w is None else w
        out = self.out if out is None else out
        _lib.call("mm_moe_decode", store.mm_layer(), _i(x), x_dtype_of(x), 1 if rescale else 0, self.T, self.k,
                  _i(ids), _i(w), self.max_rows, _i(out), _i(self.gws), self.gws_bytes, _lib.stream_ptr(stream))
        return out

    def run(self, store, x=None, ids=None, w=None, out=None, use_permutation=False, rescale=False, stream=None):
        """One layer as separate steps: expert MLP (in-kernel routing, or the permutation with use_permutation)
        -> Y -> combine. ids/w default to the runner's buffers."""
        if use_permutation:
            self.route(ids, w, stream)
        self.experts(store, x, ids, 31, use_permutation, rescale, stream)
        return self.combine(ids, w, out, stream)
