"""Shared test helpers: synthetic stores and oracle evaluation of a MoE layer."""
import numpy as np

import oracle as O


def make_store(E, H, I, layer_seed, device="cuda", limit=10.0, exact=False):
    import torch
    from mi355moe.store import ExpertStore
    st = ExpertStore(E, H, I, device=device, limit=limit, exact=exact).synthesize(layer_seed)
    torch.cuda.synchronize()
    return st


class OracleLayer:
    """Oracle of one layer whose experts come from the synthetic generator (trellis) and the store's scales."""

    def __init__(self, store, layer_seed, cache=True):
        """layer_seed: the synthetic trellis stream of the layer's experts (the scales come from `store`).
        cache=False decodes each expert afresh and keeps nothing (100 MB per expert at 4096/2048)."""
        self.store, self.seed = store, layer_seed
        self.H, self.I = store.H, store.I
        self.keep = cache
        self._cache = {}

    def expert(self, e):
        if e in self._cache:
            return self._cache[e]
        tr = O.synth_expert_trellis(self.seed, e, self.H, self.I)
        s = self.store.scales_numpy(e)
        d = O.DenseExpert(*tr, s["w13_suh"][0], s["w13_svh"][0], s["w13_suh"][1], s["w13_svh"][1], s["w2_suh"],
                          s["w2_svh"], self.H, self.I)
        if self.keep:
            self._cache[e] = d
        return d

    def forward(self, x16, ids, w, limit=10.0):
        """float64 out [T, H] = sum_j w * expert(x) over valid routes (x16: fp16-valued fp32 [T, H])."""
        T = x16.shape[0]
        ids = np.asarray(ids).reshape(T, -1)
        w = np.asarray(w, np.float32).reshape(T, -1)
        out = np.zeros((T, self.H), np.float64)
        for e in np.unique(ids[(ids >= 0) & (ids < self.store.E)]):
            tt, jj = np.nonzero(ids == e)
            y = self.expert(int(e))(x16[tt], limit)
            for row, t, j in zip(y, tt, jj):
                out[t] += np.float64(w[t, j]) * row
        return out

    def per_route(self, x16, ids, limit=10.0):
        """Y fp32 [T*k, H] of every route (NaN rows for invalid routes)."""
        T = x16.shape[0]
        ids = np.asarray(ids).reshape(T, -1)
        Y = np.full((ids.size, self.H), np.nan, np.float32)
        for e in np.unique(ids[(ids >= 0) & (ids < self.store.E)]):
            tt, jj = np.nonzero(ids == e)
            y = self.expert(int(e))(x16[tt], limit)
            for row, t, j in zip(y, tt, jj):
                Y[t * ids.shape[1] + j] = row
        return Y


def within_tolerance(a, b, max_rel=2e-2, mean_rel=2e-3):
    mx, mean = O.tolerance_metrics(a, b)
    return (mx <= max_rel and mean <= mean_rel), (mx, mean)
