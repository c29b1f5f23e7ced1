"""EXL3 checkpoint loading and the host plan: routed experts of real checkpoints into the layer stores.

Checkpoint keys follow the served pack (experimental/b70-tier/repro/rep_ct.py:50-57,
experimental/b70-tier/worker/bt_worker.py:251-270):
    layers.{L}.ffn.experts.{e}.{w1|w3|w2}.{trellis|suh|svh}
w1 = gate and w3 = up (trellis int16 [H/16, I/16, 48], suh fp16 [H], svh fp16 [I]); w2 = down (trellis
[I/16, H/16, 48], suh [I], svh [H]). Keys may carry a prefix (`model.`, `language_model.model.`). A checkpoint is a
directory with model.safetensors.index.json, one .safetensors file, or a list of them. Only the "mul1" codebook is
supported (the served pack's, pack/prepare_pack.py:47); a checkpoint that flags "mcg" is refused.

The host plan (pack/prepare_pack.py:85-86) is JSON {layer name: [expert ids kept in host memory]}; a layer name is
matched exactly or by suffix, either way round, as the plugin does (patches/vllm-exl3-host-dma.patch:530-543).
load_layer puts the plan's experts of a layer in a pinned host home (the reference's weight_loader redirect,
patch:689-709) and every other expert in HBM.
"""
import json
import os
import re

import numpy as np
import torch

from . import cache
from .store import ExpertStore

_MATS = (("w1", "gate"), ("w3", "up"), ("w2", "down"))


class Checkpoint:
    """Read-only view of safetensors files (tensors loaded on the CPU, nothing executed from the files)."""

    def __init__(self, path):
        from safetensors import safe_open
        self._open = safe_open
        if isinstance(path, (list, tuple)):
            files = [str(p) for p in path]
        elif os.path.isdir(path):
            idx = os.path.join(path, "model.safetensors.index.json")
            if os.path.exists(idx):
                with open(idx) as f:
                    wm = json.load(f)["weight_map"]
                files = sorted({os.path.join(path, v) for v in wm.values()})
            else:
                files = sorted(os.path.join(path, n) for n in os.listdir(path) if n.endswith(".safetensors"))
        else:
            files = [str(path)]
        self.where = {}
        self._h = {}
        for fn in files:
            with safe_open(fn, "pt") as h:
                for k in h.keys():
                    self.where[k] = fn
        self._index()

    def _index(self):
        # every key under its unprefixed name (from a "layers." that starts the key or follows a "."), the first
        # key of the checkpoint winning, and the routed experts present per layer: one pass over the keys, so a
        # lookup costs a dict probe whatever the prefix
        self._bare = {}
        self._experts = {}
        pat = re.compile(r"^layers\.(\d+)\.ffn\.experts\.(\d+)\.w1\.trellis$")
        for k in self.where:
            i = k.find("layers.")
            while i >= 0:
                if i == 0 or k[i - 1] == ".":
                    bare = k[i:]
                    self._bare.setdefault(bare, k)
                    m = pat.match(bare)
                    if m:
                        self._experts.setdefault(int(m.group(1)), set()).add(int(m.group(2)))
                i = k.find("layers.", i + 1)

    def keys(self):
        return self.where.keys()

    def get(self, name):
        fn = self.where[name]
        h = self._h.get(fn)
        if h is None:
            h = self._h[fn] = self._open(fn, "pt")
        return h.get_tensor(name)

    def _key(self, layer, e, w, part):
        base = f"layers.{layer}.ffn.experts.{e}.{w}.{part}"
        if base in self.where:
            return base
        k = self._bare.get(base)
        if k is None:
            raise KeyError(f"checkpoint has no tensor {base}")
        return k

    def expert_tensor(self, layer, e, w, part):
        return self.get(self._key(layer, e, w, part))

    def num_experts(self, layer):
        ids = self._experts.get(int(layer), set())
        if not ids:
            raise KeyError(f"checkpoint has no experts for layer {layer}")
        if ids != set(range(max(ids) + 1)):
            raise ValueError(f"layer {layer}: expert ids are not 0 .. {max(ids)}")
        return max(ids) + 1

    def shape(self, layer):
        """(E, H, I) of a layer's routed experts."""
        g = self.expert_tensor(layer, 0, "w1", "trellis")
        if g.dim() != 3 or g.shape[2] != 48:
            raise ValueError(f"layer {layer}: w1 trellis of shape {tuple(g.shape)} is not [H/16, I/16, 48] (3 bpw)")
        return self.num_experts(layer), int(g.shape[0]) * 16, int(g.shape[1]) * 16

    def check_codebook(self, layer):
        for w, _ in _MATS:
            for flag in ("mcg", "mcg_mult"):
                try:
                    t = self.expert_tensor(layer, 0, w, flag)
                except KeyError:
                    continue
                if t.numel() and bool(t.reshape(-1)[0].item()):
                    raise NotImplementedError(f"layer {layer}: the mcg codebook is not supported (mul1 only)")


def read_host_plan(path):
    with open(path) as f:
        plan = json.load(f)
    return {str(k): sorted(set(int(e) for e in v)) for k, v in plan.items()}


def host_plan_for(plan, layer_name):
    """The plan's host-resident experts of a layer (exact name, else a suffix match either way), or None."""
    if not plan:
        return None
    cold = plan.get(layer_name)
    if cold is None:
        for k, v in plan.items():
            if k.endswith(layer_name) or layer_name.endswith(k):
                cold = v
                break
    return sorted(set(int(e) for e in cold)) if cold else None


def write_host_plan(path, nlayers, E, name="model.layers.{}.ffn.experts"):
    """Every routed expert of every layer in host memory (pack/prepare_pack.py:85-86)."""
    with open(path, "w") as f:
        json.dump({name.format(i): list(range(E)) for i in range(nlayers)}, f)


def _scales(ck, layer, E, H, I):
    s13 = np.empty((E, 2, H), np.float16)
    v13 = np.empty((E, 2, I), np.float16)
    s2 = np.empty((E, I), np.float16)
    v2 = np.empty((E, H), np.float16)
    for e in range(E):
        for j, w in enumerate(("w1", "w3")):
            s13[e, j] = ck.expert_tensor(layer, e, w, "suh").to(torch.float16).numpy().reshape(H)
            v13[e, j] = ck.expert_tensor(layer, e, w, "svh").to(torch.float16).numpy().reshape(I)
        s2[e] = ck.expert_tensor(layer, e, "w2", "suh").to(torch.float16).numpy().reshape(I)
        v2[e] = ck.expert_tensor(layer, e, "w2", "svh").to(torch.float16).numpy().reshape(H)
    return s13, v13, s2, v2


def _trellis(ck, layer, e, H, I):
    """(gate, up, down) int16 arrays of expert e, checked against the layer shape."""
    out = []
    for w, _ in _MATS:
        t = ck.expert_tensor(layer, e, w, "trellis").to(torch.int16).numpy()
        want = (H // 16, I // 16, 48) if w != "w2" else (I // 16, H // 16, 48)
        if t.shape != want:
            raise ValueError(f"layer {layer} expert {e} {w}: trellis {t.shape}, expected {want}")
        out.append(np.ascontiguousarray(t))
    return out


def load_layer(ck, layer, device="cuda", cold=None, limit=10.0, exact=False, host_buffer=None, host_offset=0):
    """One layer's routed experts as an ExpertStore.

    cold: expert ids kept in a pinned host home (from the host plan); None or empty puts every expert in HBM.
    With a host home every expert has a home row (those not in `cold` are also copied to HBM rows that the pointer
    tables name, as permanently resident experts with slot numbers from 2^30 up, so the split counts them as
    hits and the expert cache leaves them alone). host_buffer / host_offset place the home in a shared pinned
    buffer."""
    if not isinstance(ck, Checkpoint):
        ck = Checkpoint(ck)
    ck.check_codebook(layer)
    E, H, I = ck.shape(layer)
    dev = torch.device(device)
    s13, v13, s2, v2 = _scales(ck, layer, E, H, I)
    if cold:
        cold = sorted(set(int(e) for e in cold if 0 <= int(e) < E))
        home = cache.HostHome(E, H, I, buffer=host_buffer, offset=host_offset)
        st = ExpertStore(E, H, I, device=dev, limit=limit, exact=exact, host_home=home)
        rows = home.rows
        raw = home.buffer.array(np.int16, offset=home.base - home.buffer.ptr)
        for e in range(E):
            g, u, d = _trellis(ck, layer, e, H, I)
            r0 = e * rows.row_words
            raw[r0:r0 + rows.n_mat] = g.reshape(-1)
            raw[r0 + rows.n_mat:r0 + 2 * rows.n_mat] = u.reshape(-1)
            raw[r0 + 2 * rows.n_mat:r0 + 3 * rows.n_mat] = d.reshape(-1)
        hot = [e for e in range(E) if e not in set(cold)]
        if hot:
            pool = cache.SlotPool(len(hot), H, I, dev)
            st._hot_pool = pool
            items = []
            for i, e in enumerate(hot):
                pool.t[i].copy_(torch.from_numpy(raw[e * rows.row_words:(e + 1) * rows.row_words]))
                g, u, d = pool.addrs(i)
                items.append((e, g, u, d, (1 << 30) + i))
            cache.point(st, items)
    else:
        st = ExpertStore(E, H, I, device=dev, limit=limit, exact=exact)
        for e in range(E):
            g, u, d = _trellis(ck, layer, e, H, I)
            st.w13_trellis[e, 0].copy_(torch.from_numpy(g))
            st.w13_trellis[e, 1].copy_(torch.from_numpy(u))
            st.w2_trellis[e].copy_(torch.from_numpy(d))
    st.w13_suh.copy_(torch.from_numpy(s13))
    st.w13_svh.copy_(torch.from_numpy(v13))
    st.w2_suh.copy_(torch.from_numpy(s2))
    st.w2_svh.copy_(torch.from_numpy(v2))
    st.layer_name = f"model.layers.{layer}.ffn.experts"
    return st


def load_model(path, layers=None, device="cuda", plan=None, limit=10.0, exact=False):
    """Every listed checkpoint layer (default: all with routed experts) as ExpertStores, experts of the host plan
    (a dict or a path to host-plan.json) in pinned host homes."""
    ck = Checkpoint(path)
    if isinstance(plan, str):
        plan = read_host_plan(plan)
    if layers is None:
        pat = re.compile(r"(?:^|\.)layers\.(\d+)\.ffn\.experts\.0\.w1\.trellis$")
        layers = sorted({int(m.group(1)) for k in ck.keys() for m in [pat.search(k)] if m})
    out = []
    for L in layers:
        cold = host_plan_for(plan, f"model.layers.{L}.ffn.experts") if plan else None
        out.append(load_layer(ck, L, device=device, cold=cold, limit=limit, exact=exact))
    return out
