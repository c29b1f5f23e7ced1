"""Expert placement: host-pinned home copies, slot-table repoints, copy-engine staging and the elastic expert cache.

The kernels read each expert's trellis through the layer's pointer tables (`_exl3_ptrs`, int64 [E] per matrix,
device memory), so where an expert lives -- its HBM home, a cache slot, a staging slot, or its pinned host home
read over PCIe -- is decided by three table entries. A move is stream-ordered: mm_slot_point writes the entries
and `slotof` on the compute stream, so kernels enqueued before it read the old placement and kernels after it the
new one; the home copy stays valid throughout, so a stale pointer is slower but never wrong (the reference's
invariant, ct/ct_vllm.py:234-236).

ExpertCache restates the reference's VRAM mirror cache (ct/ct_vllm.py:236-436): scores decayed by DECAY plus
the routed counts of the last interval, the top N (layer, expert) pairs wanted, at most ADMIT newcomers per
replan in descending score, victims in ascending score taken only when the newcomer's score exceeds HYST x the
victim's, free slots popped from the end of the list, copies on a side stream with the newcomers going live at
the next replan (ASYNC), release before prefill-sized steps and rewarm after REWARM_AFTER calm steps. Ties in
score are broken toward the lower flat index (layer * E + expert) where the reference leaves them to torch.topk
and set iteration order.
"""
import ctypes
import os

import numpy as np
import torch

from . import _lib
from .hostmem import HostBuffer
from .store import trellis_words


def _env(name, default, cast=float):
    v = os.environ.get(name)
    return cast(v) if v not in (None, "") else cast(default)


# ------------------------------------------------------------------------------------------ primitives

def point(layer, items, stream=None):
    """Stream-ordered repoint of `layer`'s pointer tables and slotof (the reference's _ec_point,
    ct/ct_vllm.py:268-279). items: [(e, gate_addr, up_addr, down_addr, slot_or_-1)]."""
    if not items:
        return
    dev = layer._exl3_ptrs["gate_trellis"].device
    s = stream if stream is not None else torch.cuda.current_stream(dev)
    a = torch.tensor([[int(v) for v in it] for it in items], dtype=torch.int64).pin_memory()
    with torch.cuda.stream(s):                       # the item copy and the repoint on the same stream
        d = a.to(dev, non_blocking=True)
    p = layer._exl3_ptrs
    _lib.call("mm_slot_point", p["gate_trellis"].data_ptr(), p["up_trellis"].data_ptr(), p["down_trellis"].data_ptr(),
              layer.slotof.data_ptr(), int(layer.E), d.data_ptr(), len(items), _lib.stream_ptr(s))
    d.record_stream(s)
    mirror = getattr(layer, "slot_host", None)
    if mirror is not None:
        for it in items:                              # in order: the last item of an expert wins, as on the device
            if 0 <= int(it[0]) < layer.E:
                mirror[int(it[0])] = int(it[4])


def stage_copy(copies, stream=None):
    """Copy-engine transfers [(dst_addr, src_addr, nbytes)] on `stream` (adjacent copies merged). Returns the
    number of transfers enqueued."""
    if not copies:
        return 0
    n = len(copies)
    arr = np.asarray(copies, dtype=np.uint64).reshape(n, 3)
    dst, src, nb = (np.ascontiguousarray(arr[:, j]) for j in range(3))
    P = ctypes.c_void_p
    return _lib.call_count("mm_stage_copy", P(dst.ctypes.data), P(src.ctypes.data), P(nb.ctypes.data), n,
                           _lib.stream_ptr(stream))


class ExpertRows:
    """Expert trellis rows laid out [gate | up | down] per expert (one contiguous row each), so one expert moves
    in one transfer: the layout of the pinned host home, of the cache pool and of the staging slots."""

    def __init__(self, H, I):
        self.H, self.I = H, I
        self.n_mat = trellis_words(H, I)             # int16 words of one gate / up / down matrix
        self.row_words = 3 * self.n_mat
        self.row_bytes = 2 * self.row_words

    def addrs(self, base):
        """(gate, up, down) addresses of the row at `base`."""
        b = self.n_mat * 2
        return base, base + b, base + 2 * b


class HostHome:
    """Pinned (hipHostMalloc, device-mapped) home copies of one layer's experts, [E] rows of ExpertRows. Kernels
    read a row in place over PCIe when the pointer tables name it; cache and staging slots are filled from it by
    the copy engines. Several layers may share one buffer (`buffer`, `offset`)."""

    def __init__(self, E, H, I, buffer=None, offset=0):
        self.E = E
        self.rows = ExpertRows(H, I)
        need = E * self.rows.row_bytes
        if buffer is None:
            buffer = HostBuffer(need)
        if offset + need > buffer.nbytes:
            raise ValueError("HostHome: buffer too small")
        self.buffer = buffer
        self.base = buffer.ptr + offset

    def row(self, e):
        return self.base + int(e) * self.rows.row_bytes

    def pointers(self):
        """int64 [E, 3] (CPU) home addresses of each expert's gate / up / down trellis."""
        e = np.arange(self.E, dtype=np.int64)
        b = self.base + e * self.rows.row_bytes
        m = self.rows.n_mat * 2
        return torch.from_numpy(np.stack([b, b + m, b + 2 * m], axis=1))


class SlotPool:
    """Device rows of ExpertRows (one expert each): the cache pool or a set of staging slots."""

    def __init__(self, n, H, I, device):
        self.rows = ExpertRows(H, I)
        self.n = n
        self.t = torch.empty((max(n, 1), self.rows.row_words), dtype=torch.int16, device=device)

    def row(self, s):
        return self.t[s].data_ptr()

    def addrs(self, s):
        return self.rows.addrs(self.row(s))


# ------------------------------------------------------------------------------------------ expert cache

class ExpertCache:
    """The reference's elastic VRAM mirror cache over `layers` (ExpertStore objects whose experts have pinned
    host homes). Parameters default to the reference's environment variables (DSV41_EC_*), with the image's
    values where it sets them (docker/entrypoint.sh:76-81)."""

    def __init__(self, layers, slots=None, every=None, admit=None, decay=None, hyst=None, warmup=None,
                 async_copy=None, prefill_tokens=None, rewarm_after=None, margin_mb=None, elastic=None):
        self.layers = list(layers)
        self.L = len(self.layers)
        self.E = self.layers[0].E if self.layers else 0
        self.slots = _env("DSV41_EC_SLOTS", 0, int) if slots is None else int(slots)
        self.every = _env("DSV41_EC_EVERY", 16, int) if every is None else int(every)
        self.admit = _env("DSV41_EC_ADMIT", 48, int) if admit is None else int(admit)
        self.decay = _env("DSV41_EC_DECAY", 0.9) if decay is None else float(decay)
        self.hyst = _env("DSV41_EC_HYST", 1.0) if hyst is None else float(hyst)
        self.warmup = _env("DSV41_EC_WARMUP", 64, int) if warmup is None else int(warmup)
        self.async_copy = (_env("DSV41_EC_ASYNC", 1, int) == 1) if async_copy is None else bool(async_copy)
        self.prefill_tokens = _env("DSV41_EC_PREFILL_TOKENS", 512, int) if prefill_tokens is None else int(prefill_tokens)
        self.rewarm_after = _env("DSV41_EC_REWARM_AFTER", 4, int) if rewarm_after is None else int(rewarm_after)
        self.margin_mb = _env("DSV41_EC_MARGIN_MB", 1500) if margin_mb is None else float(margin_mb)
        self.elastic = (_env("DSV41_EC_ELASTIC", 1, int) == 1) if elastic is None else bool(elastic)
        self.N = 0
        self.step_no = 0
        self.owner = []
        self.where = {}             # flat index -> slot, in residency order
        self.free = []
        self.score = np.zeros((self.L, self.E), dtype=np.float64)
        self.admits = self.evicts = self.replans = self.releases = self.rewarms = self.errors = 0
        self.copies_issued = 0
        self.bytes_staged = 0
        self.pool = None
        self.pending = None
        self.keep = []
        self.released = False
        self.calm = 0
        self.last_ntok = 0
        self.side = None
        self.timing = None          # a list to collect (start event, end event, bytes) of every copy, or None

    # ---------------------------------------------------------------------------------- planning (host only)
    def plan(self, counts):
        """One replan on counts [L, E] (routed counts since the last replan). Updates scores and residency and
        returns (evicted, admitted): lists of (flat index, slot) in the order they happen, or None when the
        counts are all zero (no decay then, as in the reference)."""
        c = np.asarray(counts, dtype=np.float64).reshape(self.L, self.E)
        if float(c.sum()) == 0:
            return None
        self.score *= self.decay
        self.score += c
        flat = self.score.reshape(-1)
        n = min(self.N, flat.size)
        # top n by score, ties toward the lower flat index (stable sort of -score)
        top = np.argsort(-flat, kind="stable")[:n]
        want = set(int(i) for i in top if flat[i] > 0)
        have = self.where
        cand = np.array(sorted(i for i in want if i not in have), dtype=np.int64)
        if cand.size == 0:
            return [], []
        cand = cand[np.argsort(-flat[cand], kind="stable")][: self.admit]
        victims = sorted((i for i in have if i not in want), key=lambda i: float(flat[i]))
        evicted, admitted = [], []
        vi = 0
        for i in (int(v) for v in cand):
            if self.free:
                s = self.free.pop()
            elif vi < len(victims) and float(flat[i]) > self.hyst * float(flat[victims[vi]]):
                v = victims[vi]
                vi += 1
                s = have.pop(v)
                self.evicts += 1
                evicted.append((v, s))
            else:
                break
            have[i] = s
            self.owner[s] = i
            self.admits += 1
            admitted.append((i, s))
        self.replans += 1
        return evicted, admitted

    # ---------------------------------------------------------------------------------- device side
    def _per_expert_bytes(self):
        l0 = self.layers[0]
        return ExpertRows(l0.H, l0.I).row_bytes

    def alloc(self):
        """Allocate the slot pool (the reference's _ec_alloc, ct/ct_vllm.py:243-265): `slots` rows, or as many as
        free device memory minus the margin allows."""
        if not self.layers:
            self.N = -1
            return
        l0 = self.layers[0]
        dev = l0._exl3_ptrs["gate_trellis"].device
        per = self._per_expert_bytes()
        if self.elastic:
            torch.cuda.empty_cache()
        free, _ = torch.cuda.mem_get_info(dev)
        n = int((free - int(self.margin_mb * 2 ** 20)) // per)
        n = min(n, self.slots) if self.slots > 0 else n
        n = min(n, self.L * self.E)
        if n <= 0:
            self.N = -1
            return
        self.pool = SlotPool(n, l0.H, l0.I, dev)
        self.N = n
        self.owner = [None] * n
        self.free = list(range(n))

    def _home_items(self, li, e):
        hp = self.layers[li].home[e].tolist()
        return (e, hp[0], hp[1], hp[2], -1)

    def _slot_items(self, e, s):
        g, u, d = self.pool.addrs(s)
        return (e, g, u, d, s)

    def _copy_list(self, pairs):
        rb = self.pool.rows.row_bytes
        out = []
        for li, e, s in pairs:
            src = self.layers[li].host_home.row(e)
            out.append((self.pool.row(s), src, rb))
        return out

    def _timed_copy(self, cl, stream):
        if not cl:
            return
        nbytes = sum(c[2] for c in cl)
        if self.timing is not None:
            t0 = torch.cuda.Event(enable_timing=True)
            t0.record(stream)
        self.copies_issued += stage_copy(cl, stream)
        self.bytes_staged += nbytes
        if self.timing is not None:
            t1 = torch.cuda.Event(enable_timing=True)
            t1.record(stream)
            self.timing.append((t0, t1, nbytes))

    def step(self, counts=None, stream=None):
        """The reference's ec_step (ct/ct_vllm.py:283-391), called between engine steps: every `every` steps,
        read the layers' routed counts (one device sync), replan, repoint victims home, copy newcomers into
        their slots on the side stream and point them at the slots (now, or at the next replan with async
        copies). `counts` [L, E] may be given instead of reading the layers' `counts` tensors."""
        self.step_no += 1
        if self.N < 0:
            return
        if self.released:
            if self.last_ntok <= self.prefill_tokens:
                self.calm += 1
            else:
                self.calm = 0
            if self.calm >= self.rewarm_after:
                self.calm = 0
                self.rewarm(stream)
            return
        if self.N == 0:
            if self.step_no < self.warmup:
                return
            self.alloc()
            if self.N <= 0:
                return
        if self.step_no % self.every:
            return
        main = stream if stream is not None else torch.cuda.current_stream()
        if self.pending:
            main.wait_event(self.pending["event"])
            for li, ad in self.pending["items"].items():
                point(self.layers[li], ad, main)
            self.pending = None
        if counts is None:
            c = torch.stack([l.counts for l in self.layers]).cpu().numpy()
            for l in self.layers:
                l.counts.zero_()
        else:
            c = counts
        res = self.plan(c)
        if not res:
            return
        evicted, admitted = res
        E = self.E
        per_layer = {}
        for v, s in evicted:
            li, e = divmod(v, E)
            per_layer.setdefault(li, ([], []))[0].append(self._home_items(li, e))
        copies = []
        for i, s in admitted:
            li, e = divmod(i, E)
            copies.append((li, e, s))
            per_layer.setdefault(li, ([], []))[1].append(self._slot_items(e, s))
        for li, (ev, _) in per_layer.items():            # victims back to their home copies (compute stream)
            point(self.layers[li], ev, main)
        if self.async_copy:
            side = _lib.copy_stream(main.device, _lib.COPY_CACHE, main)
            if self.side is not None and side is not self.side:
                side.wait_stream(self.side)               # copies on an earlier copy stream stay ordered
            self.side = side
            self.side.wait_stream(main)                   # slots are free once every earlier reader ran
            cs = self.side
        else:
            cs = main
        cl = self._copy_list(copies)
        self._timed_copy(cl, cs)
        if self.async_copy:
            ev = torch.cuda.Event()
            ev.record(cs)
            self.pending = {"event": ev, "items": {li: ad for li, (_, ad) in per_layer.items() if ad}}
        else:
            for li, (_, ad) in per_layer.items():
                point(self.layers[li], ad, main)

    def release(self, stream=None):
        """Hand the pool back before a prefill-sized step (ct/ct_vllm.py:394-416): residents repointed home
        (stream ordered), the resident set kept for the rewarm, the pool freed."""
        if self.N <= 0:
            return
        main = stream if stream is not None else torch.cuda.current_stream()
        if self.side is not None:
            main.wait_stream(self.side)
        self.pending = None
        per = {}
        for i in list(self.where):
            li, e = divmod(i, self.E)
            per.setdefault(li, []).append(self._home_items(li, e))
        for li, items in per.items():
            point(self.layers[li], items, main)
        self.keep = list(self.where)
        self.where = {}
        self.owner = []
        self.free = []
        self.pool = None
        self.N = 0
        self.releases += 1
        self.released = True
        self.calm = 0
        main.synchronize()          # the repoints ran before the pool's memory goes back
        torch.cuda.empty_cache()

    def rewarm(self, stream=None):
        """Re-allocate the pool and re-admit the kept set in descending score (ct/ct_vllm.py:419-436)."""
        torch.cuda.empty_cache()
        self.alloc()
        self.released = False
        if self.N <= 0:
            return
        main = stream if stream is not None else torch.cuda.current_stream()
        flat = self.score.reshape(-1)
        keep = sorted(self.keep, key=lambda i: -float(flat[i]))[: self.N]
        per = {}
        copies = []
        for i in keep:
            s = self.free.pop()
            li, e = divmod(i, self.E)
            self.where[i] = s
            self.owner[s] = i
            copies.append((li, e, s))
            per.setdefault(li, []).append(self._slot_items(e, s))
        cl = self._copy_list(copies)
        self._timed_copy(cl, main)
        for li, items in per.items():
            point(self.layers[li], items, main)
        self.rewarms += 1

    def summary(self):
        """The reference's ec_summary fields (ct/ct_vllm.py:430-433)."""
        return {"slots": self.N, "resident": len(self.where), "admits": self.admits, "evicts": self.evicts,
                "replans": self.replans, "steps": self.step_no, "errors": self.errors, "releases": self.releases,
                "rewarms": self.rewarms}
