"""Expert storage of one MoE layer in HBM, with the reference's pointer tables and scale parameters.

Layout and names follow the EXL3 MoE parameters of the reference's plugin
(patches/vllm-exl3-host-dma.patch:641-690, 713-751):
  w13 trellis int16 [E, 2, H/16, I/16, 48] (gate = 0, up = 1), w2 trellis int16 [E, I/16, H/16, 48],
  w13_suh fp16 [E, 2, H], w13_svh fp16 [E, 2, I], w2_suh fp16 [E, I], w2_svh fp16 [E, H],
  _exl3_ptrs {"gate_trellis", "up_trellis", "down_trellis"}: int64 [E] device addresses, read by the kernels
  on every call, so repointing an expert (cache slot, staging slot, home copy) is a table write.
On MI355X (288 GB HBM) every expert of every layer is resident: 384 routed + 1 shared experts of the
H=4096 / I=2048 shape take 3.65 GB per layer.
"""
import numpy as np
import torch

from . import _lib

KW = 48   # int16 words per 16x16 tile at 3 bpw


def trellis_words(K, N):
    return (K // 16) * (N // 16) * KW


class ExpertStore:
    """All experts of one layer: trellis in HBM (default), or in a pinned host home (`host_home`, a
    cache.HostHome) that kernels read over PCIe unless the pointer tables name a cache or staging slot.
    Scales always live in HBM.

    Slot-table state (the reference's layer._ct, ct/ct_vllm.py:106-116): `slotof` int32 [E] (cache slot or -1;
    HBM-resident experts are their own slot), `home` int64 [E, 3] (CPU) home addresses, `counts` int32 [E]
    routed counts accumulated by the split for the expert cache."""

    def __init__(self, E, H, I, device="cuda", limit=10.0, exact=False, host_home=None):
        if H % 128 or I % 128:
            raise ValueError(f"H and I must be multiples of 128 (H={H}, I={I})")
        self.E, self.H, self.I, self.limit = E, H, I, float(limit)
        self.exact = bool(exact)      # fp16-rounded weights (EXACT) instead of the AFFINE codebook evaluation
        dev = torch.device(device)
        it, ot = H // 16, I // 16
        self.host_home = host_home
        if host_home is None:
            self.w13_trellis = torch.empty((E, 2, it, ot, KW), dtype=torch.int16, device=dev)
            self.w2_trellis = torch.empty((E, ot, it, KW), dtype=torch.int16, device=dev)
        else:
            if host_home.E != E or host_home.rows.H != H or host_home.rows.I != I:
                raise ValueError("ExpertStore: host home shape differs from the layer")
            self.w13_trellis = self.w2_trellis = None
        self.w13_suh = torch.empty((E, 2, H), dtype=torch.float16, device=dev)
        self.w13_svh = torch.empty((E, 2, I), dtype=torch.float16, device=dev)
        self.w2_suh = torch.empty((E, I), dtype=torch.float16, device=dev)
        self.w2_svh = torch.empty((E, H), dtype=torch.float16, device=dev)
        self.home = self._home_pointers() if host_home is None else host_home.pointers()
        self._exl3_ptrs = {k: self.home[:, j].to(dev).contiguous() for j, k in
                           enumerate(("gate_trellis", "up_trellis", "down_trellis"))}
        if host_home is None:
            self.slotof = torch.arange(E, dtype=torch.int32, device=dev)   # every expert HBM-resident
        else:
            self.slotof = torch.full((E,), -1, dtype=torch.int32, device=dev)
        # host mirror of slotof, kept by cache.point, so host code can plan staging without reading the device
        self.slot_host = self.slotof.cpu().numpy().copy()
        self.counts = torch.zeros(E, dtype=torch.int32, device=dev)
        self._c = None

    @property
    def cold(self):
        """Experts whose home is in host memory (the reference's _exl3_host13.cold)."""
        return list(range(self.E)) if self.host_home is not None else []

    def _home_pointers(self):
        """int64 [E, 3] (CPU): addresses of each expert's gate / up / down trellis in this store."""
        E = self.E
        b13, b2 = self.w13_trellis.data_ptr(), self.w2_trellis.data_ptr()
        s13 = self.w13_trellis.stride(0) * 2
        sg = self.w13_trellis.stride(1) * 2
        s2 = self.w2_trellis.stride(0) * 2
        e = np.arange(E, dtype=np.int64)
        hp = np.stack([b13 + e * s13, b13 + e * s13 + sg, b2 + e * s2], axis=1)
        return torch.from_numpy(hp)

    def with_tables(self, gate, up, down):
        """A view of this layer whose kernels read the trellis through other pointer tables (int64 [E] device
        tensors): the same scales, shape and flags."""
        v = object.__new__(ExpertStore)
        v.__dict__.update(self.__dict__)
        v._exl3_ptrs = {"gate_trellis": gate, "up_trellis": up, "down_trellis": down}
        v._c = None
        return v

    def mm_layer(self):
        """The C ABI's mm_layer_t for this store (kept alive by the store)."""
        if self._c is None:
            self._c = _lib.MMLayer(self._exl3_ptrs["gate_trellis"].data_ptr(), self._exl3_ptrs["up_trellis"].data_ptr(),
                                   self._exl3_ptrs["down_trellis"].data_ptr(), self.w13_suh.data_ptr(),
                                   self.w13_svh.data_ptr(), self.w2_suh.data_ptr(), self.w2_svh.data_ptr(), self.E,
                                   self.H, self.I, self.limit, _lib.MMLayer.EXACT if self.exact else 0)
        return self._c

    # ------------------------------------------------------------------------------------------ synthetic
    def synthesize(self, layer_seed, stream=None, trellis=True):
        """Seeded synthetic weights: trellis words from the counter-based generator (per expert stream
        mm_expert_seed(layer_seed, e)), suh = +-1 and svh = fp16(|N(0, 0.02)|) from numpy default_rng.
        trellis=False writes the scales only (a layer sharing another layer's host home)."""
        if trellis:
            _lib.call("mm_synth_layer", self.mm_layer(), int(layer_seed), _lib.stream_ptr(stream))
        sc = synth_scales(layer_seed, self.E, self.H, self.I)
        for name, arr in sc.items():
            getattr(self, name).copy_(torch.from_numpy(arr))
        return self

    def scales_numpy(self, e):
        return {k: getattr(self, k)[e].cpu().numpy() for k in ("w13_suh", "w13_svh", "w2_suh", "w2_svh")}


def synth_scales(layer_seed, E, H, I):
    """Seeded scale vectors of one layer (numpy, fp16)."""
    rng = np.random.default_rng(int(layer_seed))
    sign = lambda shape: np.where(rng.integers(0, 2, shape) == 0, -1.0, 1.0).astype(np.float16)
    mag = lambda shape: np.abs(rng.normal(0.0, 0.02, shape)).astype(np.float16)
    return {"w13_suh": sign((E, 2, H)), "w13_svh": mag((E, 2, I)), "w2_suh": sign((E, I)), "w2_svh": mag((E, H))}
