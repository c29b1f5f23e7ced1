"""The host expert tier (mm_tier_* in libmi355moe.so): routed experts computed on the host cores from their pinned
home rows, for the picks the decode split sends to the host (the reference's tier_* extension,
kernels/cpu_avx2/ft_tier_ext.cpp:36-231, driven from ct/ct_vllm.py:56-87,143-152).

  init(H, I, nlayers, mailbox=None)   workers and the mailbox (ctrl / hx / picks / hout addresses, its capacity
                                      maxtok / maxpicks and the buffer that owns it, or None for forward() only);
                                      threads, CPUs and mode from DSV41_CT_THREADS, DSV41_CT_CPUS and DSV41_CT_MODE
                                      as in the reference
  add_layer(li, layer)                a layer with a pinned host home (ExpertStore): its home rows and host copies
                                      of its scales
  start() / stop() / shutdown()       the serving thread
  forward(li, x, sel, w, mode)        synchronous forward (tests, the tier's self-check and calibration); mode 0
                                      AFFINE, 1 EXACT, 2 I16, -1 automatic (I16 when no expert has more than two
                                      rows, else AFFINE)
  stats()                             jobs, picks, tokens, empty jobs, busy ns, rejected and stale jobs

Host memory the workers read (the mailbox, the layers' pinned expert homes) is held while the tier is up: the
tier keeps a reference to each owning buffer and marks it held (HostBuffer.hold), so it can be neither collected
nor freed before shutdown(). The library's own exit handler stops the threads at process exit in any case.
"""
import atexit
import ctypes
import os

import numpy as np

from . import _lib

_T = {"up": False, "running": False, "layers": {}, "cpus": [], "threads": 0, "held": []}

STATS = ("jobs", "picks", "tokens", "empty", "busy_ns", "rejected", "stale")


def _hold(owner):
    if owner is not None and hasattr(owner, "hold"):
        owner.hold()
    if owner is not None:
        _T["held"].append(owner)


def _release_all():
    for o in _T["held"]:
        if hasattr(o, "release"):
            o.release()
    _T["held"] = []


def _cpus_from_env():
    """DSV41_CT_CPUS ("a-b,c"), else every CPU this process may use except the first two, which are left to the
    serving process's own threads (the reference's default "2-23" leaves CPUs 0 and 1 likewise, ct_vllm.py:44-49)."""
    v = os.environ.get("DSV41_CT_CPUS", "")
    if v:
        out = []
        for part in v.split(","):
            a, _, b = part.partition("-")
            out += list(range(int(a), int(b or a) + 1))
        return out
    avail = sorted(os.sched_getaffinity(0))
    return avail[2:] if len(avail) > 2 else (avail[1:] or avail)


def _p(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def init(H, I, nlayers, mailbox=None, threads=None, cpus=None, mode=None):
    if _T["up"]:
        return
    cpus = list(cpus) if cpus is not None else _cpus_from_env()
    if threads is None:
        threads = int(os.environ.get("DSV41_CT_THREADS", "0") or 0) or min(22, len(cpus))
    mode = int(os.environ.get("DSV41_CT_MODE", "-1")) if mode is None else int(mode)
    carr = (ctypes.c_int * max(1, len(cpus)))(*cpus)
    mb = mailbox or {}
    _lib.call("mm_tier_init", int(threads), carr, len(cpus), mb.get("ctrl"), mb.get("hx"), mb.get("picks"),
              mb.get("hout"), int(mb.get("maxtok", 0)), int(mb.get("maxpicks", 0)), mode, int(H), int(I), int(nlayers))
    _T.update(up=True, cpus=cpus, threads=int(threads), H=int(H), I=int(I), mode=mode, mailbox=bool(mailbox),
              held=[])
    _hold(mb.get("owner"))
    if not _T.get("atexit"):
        # the worker and the pool threads must be gone before the interpreter frees the pinned mailbox and homes
        atexit.register(_at_exit)
        _T["atexit"] = True


def _at_exit():
    if _T["up"]:
        shutdown()


def set_limit(limit):
    _lib.call("mm_tier_set_limit", ctypes.c_float(float(limit)))


def set_mode(mode):
    _lib.call("mm_tier_set_mode", int(mode))


def add_layer(li, layer=None, ptrs=None, scales=None):
    """Register layer li: an ExpertStore with a pinned host home, or explicit `ptrs` (int64 [E, 3] host
    addresses) and `scales` (dict of fp16 arrays suh_g, svh_g, suh_u, svh_u, suh_d, svh_d, [E, .])."""
    if layer is not None:
        home = getattr(layer, "host_home", None)
        if home is not None:
            _hold(getattr(home, "buffer", home))      # the workers read the pinned home rows in place
        ptrs = layer.home.numpy() if hasattr(layer.home, "numpy") else np.asarray(layer.home)
        s13, v13 = layer.w13_suh.cpu().numpy(), layer.w13_svh.cpu().numpy()
        scales = {"suh_g": s13[:, 0], "svh_g": v13[:, 0], "suh_u": s13[:, 1], "svh_u": v13[:, 1],
                  "suh_d": layer.w2_suh.cpu().numpy(), "svh_d": layer.w2_svh.cpu().numpy()}
    ptrs = np.ascontiguousarray(ptrs, dtype=np.int64)
    keep = [ptrs] + [np.ascontiguousarray(scales[k], dtype=np.float16) for k in
                     ("suh_g", "svh_g", "suh_u", "svh_u", "suh_d", "svh_d")]
    _lib.call("mm_tier_add_layer", int(li), int(ptrs.shape[0]), *[_p(a) for a in keep])
    _T["layers"][int(li)] = keep          # the tier reads these arrays in place


def start(cpu0=None):
    if cpu0 is None:
        cpu0 = _T["cpus"][0] if _T["cpus"] else -1
    _lib.call("mm_tier_start", int(cpu0))
    _T["running"] = True


def stop():
    _lib.call("mm_tier_stop")
    _T["running"] = False


def shutdown():
    _lib.call("mm_tier_shutdown")
    _T.update(up=False, running=False, layers={})
    _release_all()


def running():
    """The tier is initialised (workers up)."""
    return _T["up"]


def serving():
    """The mailbox worker is running (synchronous forward() calls are refused meanwhile)."""
    return _T["running"]


def forward(li, x, sel, w, mode=-1):
    """x fp32 [m, H] (fp16-valued), sel int32 [m, k] (-1 skips), w fp32 [m, k] -> out fp32 [m, H]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    sel = np.ascontiguousarray(sel, dtype=np.int32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    m, k = sel.shape
    out = np.empty((m, x.shape[1]), np.float32)
    _lib.call("mm_tier_forward", int(li), _p(x), m, _p(sel), _p(w), k, _p(out), int(mode))
    return out


def stats():
    a = np.zeros(len(STATS), np.int64)
    _lib.call("mm_tier_stats", _p(a))
    return {k: int(v) for k, v in zip(STATS, a)}
