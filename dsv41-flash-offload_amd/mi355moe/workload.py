"""Seeded synthetic inputs of the benchmark configurations (routing, activations, cache maps).

Seeds follow one convention everywhere: weights 1000 + layer, routing 2000 + layer, activations 7.
"""
import numpy as np


def zipf_probs(E, s=1.1):
    r = np.arange(1, E + 1, dtype=np.float64)
    p = r ** -s
    return p / p.sum()


def zipf_routing(T, k, E, seed, s=1.1, perm_seed=None):
    """ids int64 [T, k]: k distinct experts per token, drawn Zipf(s) over a seeded permutation of the experts;
    weights fp32 [T, k]: softmax of N(0, 1) logits."""
    rng = np.random.default_rng(seed)
    perm = np.random.default_rng(seed if perm_seed is None else perm_seed).permutation(E)
    p = zipf_probs(E, s)
    ranks = np.stack([rng.choice(E, k, replace=False, p=p) for _ in range(T)])
    ids = perm[ranks].astype(np.int64)
    logits = rng.normal(0.0, 1.0, (T, k))
    w = np.exp(logits - logits.max(1, keepdims=True))
    w = (w / w.sum(1, keepdims=True)).astype(np.float32)
    return ids, w


def cache_map(ids, E, slots=709, frac_resident=0.4, seed=0, layers=40):
    """slotof int32 [E] of one layer of a `slots`-entry cache shared by `layers` layers: ~frac_resident of the
    experts selected in ids are resident, and the layer's remaining share of the slots (slots / layers) holds
    unselected experts; -1 = not resident. Slot numbers are distinct."""
    rng = np.random.default_rng(seed)
    sel = np.unique(ids[(ids >= 0) & (ids < E)])
    n_res = int(round(frac_resident * sel.size))
    res = rng.choice(sel, n_res, replace=False) if n_res else np.zeros(0, np.int64)
    rest = np.setdiff1d(np.arange(E), sel)
    n_fill = min(rest.size, max(0, int(round(slots / layers)) - n_res))
    fill = rng.choice(rest, n_fill, replace=False) if n_fill else np.zeros(0, np.int64)
    slotof = np.full(E, -1, np.int32)
    chosen = np.concatenate([np.asarray(res, np.int64), np.asarray(fill, np.int64)])
    slotof[chosen] = rng.choice(slots, chosen.size, replace=False).astype(np.int32)
    return slotof


def activations(T, H, seed=7):
    """bf16-representable N(0, 1) activations as float32 [T, H]."""
    x = np.random.default_rng(seed).normal(0.0, 1.0, (T, H)).astype(np.float32)
    u = x.view(np.uint32)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)   # round to bf16 (RNE)
    return u.view(np.float32)


def skewed_routing(T, k, E, seed, hot=64, hot_share=0.6):
    """Prefill routing: `hot` experts take `hot_share` of the assignments; k distinct experts per token."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(E)
    p = np.full(E, (1.0 - hot_share) / (E - hot))
    p[:hot] = hot_share / hot
    ranks = np.empty((T, k), np.int64)
    for t in range(T):
        ranks[t] = rng.choice(E, k, replace=False, p=p)
    ids = perm[ranks]
    logits = rng.normal(0.0, 1.0, (T, k))
    w = np.exp(logits - logits.max(1, keepdims=True))
    return ids.astype(np.int64), (w / w.sum(1, keepdims=True)).astype(np.float32)


def zipf_ids(T, k, E, rng, perm, s=1.1):
    """ids int64 [T, k]: k distinct experts per token, Zipf(s) over the expert ranking `perm` (perm[r] = expert of
    rank r), drawn without replacement by the Gumbel top-k method (the same distribution as successive weighted
    draws); weights fp32 [T, k] = softmax of N(0, 1) logits."""
    logp = np.log(zipf_probs(E, s))
    keys = logp[None, :] + rng.gumbel(size=(T, E))
    ranks = np.argpartition(-keys, k - 1, axis=1)[:, :k]
    ids = perm[ranks].astype(np.int64)
    logits = rng.normal(0.0, 1.0, (T, k))
    w = np.exp(logits - logits.max(1, keepdims=True))
    return ids, (w / w.sum(1, keepdims=True)).astype(np.float32)


def drift(perm, rng, frac=0.05):
    """Reshuffle `frac` of the ranking: that share of rank positions, chosen at random, trade experts among
    themselves."""
    E = perm.size
    m = max(2, int(round(frac * E)))
    pos = rng.choice(E, m, replace=False)
    out = perm.copy()
    out[pos] = perm[rng.permutation(pos)]
    return out
