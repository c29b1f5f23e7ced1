"""CPU ORACLE for the routed-expert MoE path -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import this module,
and only as the expected result that GPU outputs are compared against. The product library never routes
through it.

What each function restates (paths relative to the reference checkout) and how it is pinned:

  h2f / f2h        fp16 conversion                       pinned: numpy float16 over all 65,536 patterns + fp32 sweep
  perm             ft_core.h:48-61                       pinned: closed form (bijection, row/col structure) + golden
  state            ft_core.h:63-73                       pinned: golden dense weights from the compiled reference
  weight_h         ft_core.h:75-83                       pinned: golden (all states reachable via dense tiles) + closed form
  dense            ft_core.h:977-992                     pinned: golden from compiled reference dense_weights
  had128           ft_core.h:89-94                       pinned: Sylvester Hadamard matrix product (numpy) + golden expert
  prep/out_block   ft_core.h:96-110                      pinned: golden expert outputs (compiled ref_expert)
  act              ft_core.h:123-133                     pinned: golden expert outputs with limit 10
  linear/expert    ft_core.h:994-1011                    pinned: golden expert outputs (compiled ref_expert)
  router           build definition (vLLM router absent) pinned: torch.topk/softmax on CPU (library routines)
  split            ct/ft_tier_cu_v.cu:16-101             pinned: brute-force argmin over k + set invariants
  permute          patch:204-236,296-312                 pinned: numpy stable argsort + bincount
  combine          ct/ft_tier_cu_v.cu:103-127            pinned: closed form (numpy einsum in float64)
  prepare_input    build's decode-chain step (no ref.)   pinned: fixed-order sum against an fma emulation, ties
  synth_u16        build's synthetic generator           pinned: golden checksum + GPU fill agreement
  ec (ec_oracle)   ct/ct_vllm.py:243-427                 pinned: invariants (see tests/test_ec.py)
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

f32p = ctypes.POINTER(ctypes.c_float)
u16p = ctypes.POINTER(ctypes.c_uint16)
i32p = ctypes.POINTER(ctypes.c_int32)
i64p = ctypes.POINTER(ctypes.c_int64)


def build():
    subprocess.run(["make", "-s", "-C", _HERE, "libmmoracle.so"], check=True)


def lib():
    global _LIB
    if _LIB is None:
        # MM_ORACLE_LIB names another build of the same source (the sanitizer build of asan_check.sh)
        path = os.environ.get("MM_ORACLE_LIB") or os.path.join(_HERE, "libmmoracle.so")
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        L.mmo_h2f.restype = ctypes.c_float
        L.mmo_h2f.argtypes = [ctypes.c_uint16]
        L.mmo_f2h.restype = ctypes.c_uint16
        L.mmo_f2h.argtypes = [ctypes.c_float]
        L.mmo_state.restype = ctypes.c_uint16
        L.mmo_weight_h.restype = ctypes.c_uint16
        L.mmo_weight_h.argtypes = [ctypes.c_uint16]
        L.mmo_bytesum.restype = ctypes.c_int
        L.mmo_bytesum.argtypes = [ctypes.c_uint16]
        L.mmo_act.restype = ctypes.c_float
        L.mmo_act.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_float]
        L.mmo_expert_seed.restype = ctypes.c_uint64
        L.mmo_expert_seed.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        L.mmo_synth_u16.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p]
        L.mmo_row_scale.restype = ctypes.c_float
        L.mmo_row_scale.argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.mmo_row_sumsq.restype = ctypes.c_float
        L.mmo_row_sumsq.argtypes = [ctypes.c_void_p, ctypes.c_int]
        _LIB = L
    return _LIB


def _p(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else ctypes.c_void_p(0)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ---------------------------------------------------------------------------------------------- format
def f2h_bits(x):
    x = _c(x, np.float32).ravel()
    L = lib()
    return np.array([L.mmo_f2h(float(v)) for v in x], dtype=np.uint16)


def perm():
    out = np.zeros(256, dtype=np.int32)
    lib().mmo_perm(_p(out))
    return out


def state(tile, i):
    tile = _c(tile, np.uint16)
    assert tile.size == 48
    return lib().mmo_state(_p(tile), ctypes.c_int(i))


def weight_table():
    """fp16 weight of every 16-bit state (65,536 entries), as float32."""
    L = lib()
    bits = np.array([L.mmo_weight_h(s) for s in range(65536)], dtype=np.uint16)
    return bits.view(np.float16).astype(np.float32)


def dense(trellis, K, N):
    """Dense K x N fp32 weights (fp16 values) of tiles [K/16][N/16][48]."""
    t = _c(trellis, np.uint16)
    assert t.size == K * N * 3 // 16
    W = np.empty((K, N), dtype=np.float32)
    lib().mmo_dense(_p(t), K, N, _p(W))
    return W


def had128(v):
    v = _c(v, np.float32).copy()
    lib().mmo_had128(_p(v))
    return v


def prep_block(x, suh):
    x = _c(x, np.float32)
    suh = _c(suh, np.float16).view(np.uint16)
    out = np.empty(128, dtype=np.float32)
    lib().mmo_prep_block(_p(x), _p(suh), _p(out))
    return out


def out_block(y, svh):
    y = _c(y, np.float32).copy()
    svh = _c(svh, np.float16).view(np.uint16)
    lib().mmo_out_block(_p(y), _p(svh))
    return y


def act(g, u, limit):
    return lib().mmo_act(float(g), float(u), float(limit))


# ---------------------------------------------------------------------------------------------- expert
def _h(a):
    return _c(a, np.float16).view(np.uint16)


def linear(W, suh, svh, x):
    """x [ntok, K] fp16-valued -> y [ntok, N] (double accumulation, reference rounding points)."""
    K, N = W.shape
    x = _c(np.atleast_2d(x), np.float32)
    y = np.empty((x.shape[0], N), dtype=np.float32)
    lib().mmo_linear_dense(_p(_c(W, np.float32)), _p(_h(suh)), _p(_h(svh)), K, N, x.shape[0], _p(x), _p(y))
    return y


class DenseExpert:
    """An expert decoded once to dense fp32 weights, reusable for many token rows."""

    def __init__(self, tg, tu, td, suh_g, svh_g, suh_u, svh_u, suh_d, svh_d, H, I):
        self.H, self.I = H, I
        self.Wg, self.Wu, self.Wd = dense(tg, H, I), dense(tu, H, I), dense(td, I, H)
        self.s = [_h(v) for v in (suh_g, svh_g, suh_u, svh_u, suh_d, svh_d)]

    def __call__(self, x, limit):
        x = _c(np.atleast_2d(x), np.float32)
        y = np.empty((x.shape[0], self.H), dtype=np.float32)
        lib().mmo_expert_dense(_p(self.Wg), _p(self.Wu), _p(self.Wd), *[_p(v) for v in self.s], self.H, self.I,
                               ctypes.c_float(limit), x.shape[0], _p(x), _p(y))
        return y


# ---------------------------------------------------------------------------------------------- synth
def expert_seed(layer_seed, e):
    return lib().mmo_expert_seed(int(layer_seed), int(e))


def synth_u16(seed, start, n):
    out = np.empty(int(n), dtype=np.uint16)
    lib().mmo_synth_u16(ctypes.c_uint64(int(seed)), ctypes.c_uint64(int(start)), ctypes.c_uint64(int(n)), _p(out))
    return out


def synth_expert_trellis(layer_seed, e, H, I):
    """(gate [H/16,I/16,48], up [H/16,I/16,48], down [I/16,H/16,48]) uint16 of expert e."""
    n1 = (H // 16) * (I // 16) * 48
    w = synth_u16(expert_seed(layer_seed, e), 0, 3 * n1)
    return (w[:n1].reshape(H // 16, I // 16, 48), w[n1:2 * n1].reshape(H // 16, I // 16, 48),
            w[2 * n1:].reshape(I // 16, H // 16, 48))


# ---------------------------------------------------------------------------------------------- routing
def router(x, G, k):
    x = _c(x, np.float32)
    G = _c(G, np.float32)
    T, H = x.shape
    E = G.shape[0]
    logits = np.empty((T, E), dtype=np.float32)
    ids = np.empty((T, k), dtype=np.int64)
    w = np.empty((T, k), dtype=np.float32)
    lib().mmo_router(_p(x), _p(G), T, H, E, k, _p(logits), _p(ids), _p(w))
    return ids, w, logits


def split(sel, w, z, E, slotof, score, pol, seqc=0, li=0, stats=None, counts=None, H=None):
    """Returns a dict with every output of the split (device and host side)."""
    sel = _c(sel, np.int64).ravel()
    w = _c(w, np.float32).ravel()
    z = _c(z, np.float16)
    bsz, Hz = z.shape
    n = sel.size
    out = {
        "ctrl": np.zeros(16, np.int64), "hx": np.zeros(bsz * Hz, np.uint16), "hpicks": np.zeros(max(1, n) * 3, np.int32),
        "seqc": np.array([seqc], np.int64), "sel_out": np.zeros(n, np.int64), "w_out": np.zeros(n, np.float32),
        "dflag": np.zeros(1, np.int64), "stats": np.zeros(8, np.int64) if stats is None else _c(stats, np.int64).copy(),
        "counts": np.zeros(E, np.int32) if counts is None else _c(counts, np.int32).copy(),
        "hits": np.full(max(1, E), -1, np.int32), "misses": np.full(max(1, E), -1, np.int32), "nhnm": np.zeros(2, np.int32),
    }
    lib().mmo_split(_p(sel), _p(w), _p(z.view(np.uint16)), n, bsz, Hz, E, _p(_c(slotof, np.int32)), _p(_c(score, np.float32)),
                    _p(_c(pol, np.float32)), _p(out["ctrl"]), _p(out["hx"]), _p(out["hpicks"]), _p(out["seqc"]), li,
                    _p(out["sel_out"]), _p(out["w_out"]), _p(out["dflag"]), _p(out["stats"]), _p(out["counts"]),
                    _p(out["hits"]), _p(out["misses"]), _p(out["nhnm"]))
    nh, nm = int(out["nhnm"][0]), int(out["nhnm"][1])
    out["hits"], out["misses"] = out["hits"][:nh], out["misses"][:nm]
    out["npk"] = int(out["ctrl"][4]) if out["dflag"][0] else 0
    return out


def permute(ids, w, topk, E):
    ids = _c(ids, np.int64).ravel()
    n = ids.size
    w = None if w is None else _c(w, np.float32).ravel()
    counts = np.zeros(E + 1, np.int32)
    offsets = np.zeros(E + 2, np.int32)
    order = np.zeros(max(1, n), np.int32)
    tok = np.zeros(max(1, n), np.int32)
    ws = np.zeros(max(1, n), np.float32)
    lib().mmo_permute(_p(ids), _p(w), n, topk, E, _p(counts), _p(offsets), _p(order), _p(tok), _p(ws))
    return counts, offsets, order[:n], tok[:n], ws[:n]


def combine(out, Y, w, hout=None):
    out = _c(out, np.float32).copy()
    T, H = out.shape
    w = _c(w, np.float32)
    k = w.shape[1]
    Y = _c(Y, np.float32)
    assert Y.shape == (T * k, H)
    lib().mmo_combine(_p(out), _p(Y), _p(w), T, k, H, _p(None if hout is None else _c(hout, np.float32)),
                      0 if hout is None else 1)
    return out


# ---------------------------------------------------------------------------------------------- metrics
def bf16_rne(x):
    """float32 -> nearest bfloat16 value (ties to even), as float32."""
    u = _c(x, np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return u.view(np.float32)


def prepare_input(x, rescale=True, bits=False):
    """The decode-chain workload's step between layers (a definition of this build's benchmark, not of the
    reference): each fp32 row scaled to unit RMS, rounded to bf16 (RNE), then to fp16; the scale's sum of
    squares in the fixed fp32 order of mmo_prepare_input. Returns the fp16 values as float32 [T, H], or with
    bits=True the (bf16, fp16) bit patterns as uint16."""
    x = _c(np.atleast_2d(x), np.float32)
    T, H = x.shape
    xb = np.empty((T, H), np.uint16)
    xh = np.empty((T, H), np.uint16)
    lib().mmo_prepare_input(_p(x), T, H, 1 if rescale else 0, _p(xb), _p(xh))
    if bits:
        return xb, xh
    return xh.view(np.float16).astype(np.float32)


def row_scale(row):
    """The unit-RMS scale of one fp32 row, 1 / sqrt(sum(x^2) / H), its sum in mmo_prepare_input's order."""
    row = _c(row, np.float32)
    return float(lib().mmo_row_scale(_p(row), row.size))


def row_sumsq(row):
    """The fp32 sum of squares of one row in mmo_prepare_input's order."""
    row = _c(row, np.float32)
    return float(lib().mmo_row_sumsq(_p(row), row.size))


def tolerance_metrics(a, b):
    """(max|a-b| / RMS(b), sum|a-b| / sum|b|) in float64 over the whole output."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    d = np.abs(a - b)
    rms = float(np.sqrt(np.mean(b * b)))
    return float(d.max() / max(rms, 1e-30)), float(d.sum() / max(np.abs(b).sum(), 1e-30))
