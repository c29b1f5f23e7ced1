"""GPU parity of the routing kernels against the oracle (bit-exact for every integer output)."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("n,E,topk", [(1, 8, 1), (36, 385, 9), (4096, 384, 8), (8192, 385, 8), (8193, 384, 8),
                                      (131072, 384, 8), (40000, 1024, 4)])
def test_permute_bitexact(dev, n, E, topk):
    import torch
    from mi355moe import moe
    rng = np.random.default_rng(n + E)
    ids = rng.integers(0, E, n).astype(np.int64)
    ids[rng.random(n) < 0.01] = -1                                  # masked routes -> sentinel
    w = rng.normal(0, 1, n).astype(np.float32)
    print(f"permute n={n} E={E}", flush=True)
    r = moe.permute(_t(ids, dev), _t(w, dev), topk, E)
    torch.cuda.synchronize()
    counts, offsets, order, tok, ws = O.permute(ids, w, topk, E)
    assert np.array_equal(r["counts"].cpu().numpy(), counts)
    assert np.array_equal(r["offsets"].cpu().numpy(), offsets)
    assert np.array_equal(r["order"].cpu().numpy()[:n], order)
    assert np.array_equal(r["token_sorted"].cpu().numpy()[:n], tok)
    assert np.array_equal(r["weight_sorted"].cpu().numpy()[:n], ws)
    inv = np.empty(n, np.int32)
    inv[order] = np.arange(n, dtype=np.int32)
    assert np.array_equal(r["inv_order"].cpu().numpy()[:n], inv)
    act = np.nonzero(counts[:E])[0]
    assert int(r["nactive"].item()) == act.size
    assert np.array_equal(r["active"].cpu().numpy()[: act.size], act)


def _split_case(seed, pol, score_kind="zero", T=4):
    from mi355moe import workload
    ids, w = workload.zipf_routing(T, 8, 384, seed=seed)
    slotof = workload.cache_map(ids, 384, slots=709, frac_resident=0.4, seed=seed)
    z = np.random.default_rng(seed).normal(0, 1, (T, 4096)).astype(np.float16)
    score = np.zeros(384, np.float32) if score_kind == "zero" else np.random.default_rng(seed + 1).permutation(384).astype(np.float32)
    return ids, w, z, slotof, score, np.asarray(pol, np.float32)


POL_DEFAULT = [0.58, 0.03, 0.11, 0.20, 0.35, 384, -1, 0, 0]   # image defaults (cost model)
POL_CHEAP = [0.58, 0.03, 0.01, 0.05, 0.35, 384, -1, 0, 0]     # cheap CPU: several picks


@pytest.mark.parametrize("seed,pol,score_kind,T", [(1, POL_DEFAULT, "zero", 4), (2, POL_CHEAP, "zero", 4),
                                                   (3, POL_CHEAP, "perm", 4),
                                                   (4, [0.58, 0.03, 0.11, 0.2, 0.35, 384, 2, 0, 0], "zero", 4),
                                                   (5, [0.58, 0.03, 0.11, 0.2, 0.35, 384, 0, 1, 0], "zero", 4),
                                                   (6, POL_CHEAP, "perm", 160)])
def test_split_bitexact(dev, seed, pol, score_kind, T):
    """Split outputs bit-exact against the oracle; T = 160 (1,280 routes) also covers routes past the first 1,024
    that the kernel keeps in registers."""
    import torch
    from mi355moe import _lib
    from mi355moe.hostmem import HostBuffer
    ids, w, z, slotof, score, pol = _split_case(seed, pol, score_kind, T)
    n, bsz, H, E = ids.size, T, 4096, 384
    ref = O.split(ids, w, z, E, slotof, score, pol, seqc=5, li=7)
    hb = HostBuffer(16 * 8 + bsz * H * 2 + n * 3 * 4)
    ctrl = hb.array(np.int64, (16,), 0)
    hx = hb.array(np.uint16, (bsz * H,), 128)
    hp = hb.array(np.int32, (n * 3,), 128 + bsz * H * 2)
    ctrl[:] = 0
    d = {k: _t(v, dev) for k, v in dict(sel=ids.ravel(), w=w.ravel(), z=z.view(np.uint16), slotof=slotof, score=score,
                                        pol=pol).items()}
    seqc = torch.tensor([5], dtype=torch.int64, device=dev)
    sel_out = torch.empty(n, dtype=torch.int64, device=dev)
    w_out = torch.empty(n, dtype=torch.float32, device=dev)
    dflag = torch.full((1,), -7, dtype=torch.int64, device=dev)
    stats = torch.zeros(8, dtype=torch.int64, device=dev)
    counts = torch.zeros(E, dtype=torch.int32, device=dev)
    hits = torch.full((E,), -1, dtype=torch.int32, device=dev)
    misses = torch.full((E,), -1, dtype=torch.int32, device=dev)
    nhnm = torch.zeros(2, dtype=torch.int32, device=dev)
    print(f"split seed={seed}", flush=True)
    _lib.call("mm_split", d["sel"].data_ptr(), d["w"].data_ptr(), d["z"].data_ptr(), n, bsz, H, E, d["slotof"].data_ptr(),
              d["score"].data_ptr(), d["pol"].data_ptr(), hb.data_ptr(0), hb.data_ptr(128), hb.data_ptr(128 + bsz * H * 2),
              seqc.data_ptr(), 7, sel_out.data_ptr(), w_out.data_ptr(), dflag.data_ptr(), stats.data_ptr(),
              counts.data_ptr(), hits.data_ptr(), misses.data_ptr(), nhnm.data_ptr(), _lib.stream_ptr())
    torch.cuda.synchronize()
    nh, nm = nhnm.cpu().tolist()
    assert nh == len(ref["hits"]) and nm == len(ref["misses"])
    assert np.array_equal(hits.cpu().numpy()[:nh], ref["hits"])
    assert np.array_equal(misses.cpu().numpy()[:nm], ref["misses"])
    assert np.array_equal(sel_out.cpu().numpy(), ref["sel_out"])
    assert np.array_equal(w_out.cpu().numpy().view(np.uint32), ref["w_out"].view(np.uint32))
    assert np.array_equal(stats.cpu().numpy(), ref["stats"])
    assert np.array_equal(counts.cpu().numpy(), ref["counts"])
    assert int(dflag.item()) == int(ref["dflag"][0]) and int(seqc.item()) == int(ref["seqc"][0])
    if ref["dflag"][0]:
        assert np.array_equal(ctrl[[0, 2, 3, 4]], ref["ctrl"][[0, 2, 3, 4]])
        npk = int(ref["ctrl"][4])
        assert np.array_equal(hp[: 3 * npk], ref["hpicks"][: 3 * npk])
        assert np.array_equal(hx, ref["hx"])


def test_combine_host_paths(dev):
    """Host-partial add: no job, job done, and the bounded timeout path (the host never answers)."""
    import torch
    from mi355moe import _lib
    from mi355moe.hostmem import HostBuffer
    n = 4 * 4096
    hb = HostBuffer(128 + n * 4)
    ctrl = hb.array(np.int64, (16,), 0)
    hout = hb.array(np.float32, (n,), 128)
    hout[:] = np.arange(n, dtype=np.float32) * 0.5
    base = torch.randn(n, device=dev)
    stats = torch.zeros(8, dtype=torch.int64, device=dev)
    dflag = torch.zeros(1, dtype=torch.int64, device=dev)
    s = _lib.stream_ptr()
    # no job published: out unchanged
    out = base.clone()
    print("combine_host: no job", flush=True)
    _lib.call("mm_combine_host", out.data_ptr(), n, dflag.data_ptr(), hb.data_ptr(0), hb.data_ptr(128), stats.data_ptr(), 10**9, s)
    torch.cuda.synchronize()
    assert torch.equal(out, base)
    # job 3 published and already done by the host: out += hout
    dflag.fill_(3)
    ctrl[1] = 3
    out = base.clone()
    print("combine_host: done job", flush=True)
    _lib.call("mm_combine_host", out.data_ptr(), n, dflag.data_ptr(), hb.data_ptr(0), hb.data_ptr(128), stats.data_ptr(), 10**9, s)
    torch.cuda.synchronize()
    assert torch.equal(out, base + torch.from_numpy(hout.copy()).to(dev))
    st = stats.cpu().numpy()
    assert st[5] == 1 and st[6] == 0
    # job 4 never answered: 2 ms bounded wait, partial dropped, timeout counted
    dflag.fill_(4)
    out = base.clone()
    print("combine_host: timeout path (2 ms)", flush=True)
    _lib.call("mm_combine_host", out.data_ptr(), n, dflag.data_ptr(), hb.data_ptr(0), hb.data_ptr(128), stats.data_ptr(), 2_000_000, s)
    torch.cuda.synchronize()
    assert torch.equal(out, base)
    st = stats.cpu().numpy()
    assert st[6] == 1 and st[5] == 2 and st[4] >= 2_000_000
    assert int(dflag.item()) == 0          # the one decision: the whole partial dropped


@pytest.mark.parametrize("T,k", [(4, 9), (33, 8)])
def test_combine_matches_oracle(dev, T, k):
    import torch
    from mi355moe import moe
    rng = np.random.default_rng(T)
    H, E = 4096, 385
    Y = rng.normal(0, 1, (T * k, H)).astype(np.float32)
    ids = rng.integers(0, E, (T, k)).astype(np.int64)
    ids[0, 1] = -1
    w = rng.uniform(0, 1, (T, k)).astype(np.float32)
    out = moe.combine(_t(Y, dev), _t(ids, dev), _t(w, dev), T, k, H, E)
    torch.cuda.synchronize()
    wm = np.where((ids >= 0) & (ids < E), w, 0).astype(np.float32)
    ref = O.combine(np.zeros((T, H), np.float32), np.nan_to_num(Y), wm)
    assert np.array_equal(out.cpu().numpy(), ref)     # same fp32 fma chain in ascending j


@pytest.mark.parametrize("T,H,E,k", [(1, 4096, 384, 8), (4, 4096, 384, 8), (16, 4096, 384, 8), (64, 5120, 384, 6),
                                     (300, 4096, 384, 8), (4, 4096, 512, 8), (4, 2048, 1024, 8),
                                     (300, 2080, 512, 8), (129, 4096, 200, 8)])
def test_router_matches_oracle(dev, T, H, E, k):
    """Decode sizes (up to 4 tokens per workgroup, then 16), the DSV41 shape, MFMA-sized calls (with partial token
    and expert tiles and a hidden size that is an odd multiple of 32), and the top-k forms for up to 384, 512 and
    1024 experts."""
    import torch
    from mi355moe import _lib, workload
    x = workload.activations(T, H, seed=T)
    G = np.random.default_rng(5).normal(0, 0.02, (E, H)).astype(np.float32)
    xb = _t((x.view(np.uint32) >> 16).astype(np.uint16), dev)
    Gd = _t(G, dev)
    ids = torch.empty((T, k), dtype=torch.int64, device=dev)
    w = torch.empty((T, k), dtype=torch.float32, device=dev)
    logits = torch.empty((T, E), dtype=torch.float32, device=dev)
    print(f"router T={T} H={H} E={E} k={k}", flush=True)
    _lib.call("mm_router_topk", xb.data_ptr(), T, H, Gd.data_ptr(), E, k, logits.data_ptr(), ids.data_ptr(), w.data_ptr(),
              _lib.stream_ptr())
    torch.cuda.synchronize()
    rid, rw, rl = O.router(x, G, k)
    lg = logits.cpu().numpy()
    assert np.allclose(lg, rl, rtol=0, atol=5e-5)
    gi = ids.cpu().numpy()
    for t in range(T):
        if not np.array_equal(gi[t], rid[t]):
            # only a near-tie (|gap| below fp32 summation noise) may reorder the selection
            srt = np.sort(rl[t])[::-1]
            assert np.min(np.abs(np.diff(srt[: k + 1]))) < 1e-5, t
        else:
            assert np.allclose(w.cpu().numpy()[t], rw[t], rtol=1e-5, atol=1e-6)


def test_router_ties_pick_the_lower_expert(dev):
    """Exact ties in the router: gate rows duplicated in pairs give bit-identical logit pairs, and with an odd k the
    last slot splits a pair, which must go to the lower expert id; an all-zero gate ties every expert, so the
    picks are experts 0 .. k - 1 with equal weights."""
    import torch
    from mi355moe import _lib, workload
    H, E, k, T = 1024, 64, 5, 3
    x = workload.activations(T, H, seed=11)
    xb = _t((x.view(np.uint32) >> 16).astype(np.uint16), dev)
    base = np.random.default_rng(6).normal(0, 0.02, (E // 2, H)).astype(np.float32)
    for G in (np.repeat(base, 2, axis=0), np.zeros((E, H), np.float32)):
        Gd = _t(G, dev)
        ids = torch.empty((T, k), dtype=torch.int64, device=dev)
        w = torch.empty((T, k), dtype=torch.float32, device=dev)
        logits = torch.empty((T, E), dtype=torch.float32, device=dev)
        print("router ties", flush=True)
        _lib.call("mm_router_topk", xb.data_ptr(), T, H, Gd.data_ptr(), E, k, logits.data_ptr(), ids.data_ptr(),
                  w.data_ptr(), _lib.stream_ptr())
        torch.cuda.synchronize()
        lg, gi, gw = logits.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy()
        assert np.array_equal(lg[:, 0::2], lg[:, 1::2])              # the duplicated rows give equal logits
        for t in range(T):
            want = sorted(range(E), key=lambda e: (-float(lg[t, e]), e))[:k]
            assert list(gi[t]) == want, (t, list(gi[t]), want)
            z = np.exp(lg[t, want].astype(np.float64) - lg[t, want].max())
            assert np.allclose(gw[t], z / z.sum(), rtol=1e-5, atol=1e-6)


def test_router_at_prefill_size(dev):
    """The router at T = 16,384 (the prefill chunk): on 256 sampled rows the logits and picks equal the oracle's
    (as at decode sizes); on every row the picks are k distinct experts in descending logit order whose logits
    are at least the row's (k+1)-th largest, and the weights are the softmax of the picked logits."""
    import torch
    from mi355moe import _lib, workload
    T, H, E, k = 16384, 4096, 384, 8
    x = workload.activations(T, H, seed=16384)
    G = np.random.default_rng(5).normal(0, 0.02, (E, H)).astype(np.float32)
    xb = _t((x.view(np.uint32) >> 16).astype(np.uint16), dev)
    Gd = _t(G, dev)
    ids = torch.empty((T, k), dtype=torch.int64, device=dev)
    w = torch.empty((T, k), dtype=torch.float32, device=dev)
    logits = torch.empty((T, E), dtype=torch.float32, device=dev)
    print(f"router T={T}", flush=True)
    _lib.call("mm_router_topk", xb.data_ptr(), T, H, Gd.data_ptr(), E, k, logits.data_ptr(), ids.data_ptr(), w.data_ptr(),
              _lib.stream_ptr())
    torch.cuda.synchronize()
    sel = logits.gather(1, ids)
    kth = logits.topk(k + 1, dim=1).values[:, k:k + 1]
    assert bool((ids >= 0).all()) and bool((ids < E).all())
    assert bool((ids.sort(dim=1).values.diff(dim=1) > 0).all()), "picks not distinct"
    assert bool((sel >= kth).all()), "a pick below the row's top k"
    assert bool((sel[:, :-1] >= sel[:, 1:]).all()), "picks not in descending logit order"
    assert torch.allclose(w, torch.softmax(sel.double(), dim=1).float(), rtol=1e-5, atol=1e-6)
    rows = np.sort(np.random.default_rng(1).choice(T, 256, replace=False))
    # the oracle's inputs are the bf16 values the kernel reads
    xs = (x[rows].view(np.uint32) & 0xFFFF0000).view(np.float32)
    rid, rw, rl = O.router(xs, G, k)
    lg, gi = logits.cpu().numpy()[rows], ids.cpu().numpy()[rows]
    assert np.allclose(lg, rl, rtol=0, atol=5e-5)
    for t in range(rows.size):
        if not np.array_equal(gi[t], rid[t]):
            srt = np.sort(rl[t])[::-1]
            assert np.min(np.abs(np.diff(srt[: k + 1]))) < 1e-5, t
