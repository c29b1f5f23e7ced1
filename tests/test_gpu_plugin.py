"""GPU tests of the plugin entry points' argument handling: expert maps, the clamp switch, fp16 routing weights,
fully masked calls, counts given as a device tensor, and the fat threshold split of the fused call."""
import numpy as np
import pytest

from helpers import OracleLayer, make_store, within_tolerance

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_fused_moe_decode_call_semantics(dev):
    """A decode-sized call: contiguous fp32 [T, H], routing weights used in fp16, expert_map from global ids,
    limit None turns the clamp off, a fully masked call gives zeros."""
    import torch
    from mi355moe import exl3, moe
    H, I, E, T, k, seed = 512, 256, 12, 4, 3, 1212
    st = make_store(E, H, I, seed, device=dev, exact=True)
    rng = np.random.default_rng(3)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
    w = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
    x = _t(rng.normal(0, 1, (T, H)).astype(np.float32), dev).to(torch.bfloat16)
    print("fused decode call", flush=True)
    out = exl3.apply_exl3_fused_moe(x, _t(ids, dev), _t(w, dev), st, None, None, 10.0)
    w16 = w.astype(np.float16).astype(np.float32)
    ref = moe.moe_forward(st, x, _t(ids, dev), _t(w16, dev))
    torch.cuda.synchronize()
    assert out.dtype == torch.float32 and out.is_contiguous() and tuple(out.shape) == (T, H)
    assert torch.equal(out, ref)
    # global ids 0 .. 2E-1: this rank owns E .. 2E-1 (local = g - E), the others map to -1
    emap = torch.full((2 * E,), -1, dtype=torch.int32, device=dev)
    emap[E:] = torch.arange(E, dtype=torch.int32, device=dev)
    gids = ids + E
    gids[:, 0] = rng.integers(0, E, T)                          # first pick of every token is not local
    out_m = exl3.apply_exl3_fused_moe(x, _t(gids, dev), _t(w, dev), st, None, emap, 10.0)
    lids = np.where(gids >= E, gids - E, -1)
    ref_m = moe.moe_forward(st, x, _t(lids, dev), _t(w16, dev))
    torch.cuda.synchronize()
    assert torch.equal(out_m, ref_m)
    # clamp off
    out_n = exl3.apply_exl3_fused_moe(x, _t(ids, dev), _t(w, dev), st, None, None, None)
    torch.cuda.synchronize()
    x16 = x.half().cpu().numpy().astype(np.float32)
    ok, m = within_tolerance(out_n.cpu().numpy(), OracleLayer(st, seed).forward(x16, ids, w16, limit=0.0))
    assert ok, m
    # nothing routed
    z = exl3.apply_exl3_fused_moe(x, _t(np.full((T, k), -1, np.int64), dev), _t(w, dev), st, None, None, 10.0)
    torch.cuda.synchronize()
    assert torch.count_nonzero(z).item() == 0


def test_fused_moe_fat_threshold_split(dev, monkeypatch):
    """A prefill-sized call with the image's threshold (32): experts above it run on the grouped GEMM, the rest on
    the decode path; the sum matches the oracle."""
    import torch
    from mi355moe import exl3
    monkeypatch.setattr(exl3, "FAT_EXPERT_THRESHOLD", 32)
    H, I, E, T, k, seed = 512, 256, 10, 120, 2, 1313
    st = make_store(E, H, I, seed, device=dev, exact=True)
    rng = np.random.default_rng(4)
    p = np.array([0.3, 0.25, 0.15, 0.1, 0.06, 0.05, 0.04, 0.03, 0.01, 0.01])
    ids = np.stack([rng.choice(E, k, replace=False, p=p) for _ in range(T)]).astype(np.int64)
    counts = np.bincount(ids.reshape(-1), minlength=E)
    assert (counts > 32).any() and ((counts > 0) & (counts <= 32)).any()
    w = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
    x16 = rng.normal(0, 1, (T, H)).astype(np.float16)
    print(f"fused fat split counts={counts.tolist()}", flush=True)
    out = exl3.apply_exl3_fused_moe(_t(x16, dev), _t(ids, dev), _t(w, dev), st, None, None, 10.0)
    torch.cuda.synchronize()
    ref = OracleLayer(st, seed).forward(x16.astype(np.float32), ids, w.astype(np.float16).astype(np.float32))
    ok, m = within_tolerance(out.cpu().numpy(), ref)
    assert ok, m


def test_batched_fat_counts_tensor_and_no_skip(dev):
    """apply_exl3_batched_fat with per-expert counts as a device int64 tensor and no skip set equals the ids-form
    prefill over the same routes (cap 0), within tolerance (different summation order)."""
    import torch
    from mi355moe import exl3, moe
    H, I, E, T, k, seed = 512, 256, 6, 140, 2, 1414
    st = make_store(E, H, I, seed, device=dev, exact=True)
    rng = np.random.default_rng(5)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
    w = rng.uniform(0.1, 1.0, (T, k)).astype(np.float16).astype(np.float32)
    x16 = _t(rng.normal(0, 1, (T, H)).astype(np.float16), dev)
    r = moe.permute(_t(ids, dev), _t(w, dev), k, E)
    n = T * k
    out = torch.zeros((T, H), dtype=torch.float32, device=dev)
    print("batched fat, counts tensor", flush=True)
    exl3.apply_exl3_batched_fat(x16, r["token_sorted"][:n].long(), r["weight_sorted"][:n].half(),
                                r["counts"][:E].long(), exl3.layer_inners(st), 10.0, 0, out)
    ref = moe.moe_prefill(st, x16, _t(ids, dev), _t(w, dev))
    torch.cuda.synchronize()
    ok, m = within_tolerance(out.cpu().numpy(), ref.cpu().numpy().astype(np.float64))
    assert ok, m


def test_expert_cache_synchronous_copies(dev):
    """With async copies off, admitted experts point at their slots right after the replan and their slot rows hold
    the home bytes."""
    import torch
    from mi355moe.cache import ExpertCache, HostHome
    from mi355moe.store import ExpertStore
    H, I, E = 256, 256, 8
    st = ExpertStore(E, H, I, device=dev, exact=True, host_home=HostHome(E, H, I)).synthesize(1515)
    c = ExpertCache([st], slots=3, every=1, admit=3, warmup=0, async_copy=False, margin_mb=0, elastic=False)
    c.step(counts=np.array([[0, 5, 0, 9, 0, 0, 2, 0]]))
    torch.cuda.synchronize()
    assert c.pending is None and sorted(c.where) == [1, 3, 6]
    slotof = st.slotof.cpu().numpy()
    rows = st.host_home.buffer.array(np.int16, (E, c.pool.rows.row_words))
    for e in (1, 3, 6):
        s = c.where[e]
        assert slotof[e] == s and int(st._exl3_ptrs["gate_trellis"][e]) == c.pool.row(s)
        assert np.array_equal(c.pool.t[s].cpu().numpy(), rows[e])
    assert all(slotof[e] == -1 for e in (0, 2, 4, 5, 7))


@pytest.mark.parametrize("T", [64, 200, 300])
def test_fused_moe_captured_in_graph(dev, T):
    """apply_exl3_fused_moe above the fat threshold (decode path with a cap plus the fat-expert GEMM, split on the
    device) captures into a HIP graph; every replay, with eager work and synchronisations in between, equals the
    eager call bit for bit, and the eager call matches the oracle."""
    import torch
    from mi355moe import exl3
    H, I, E, k, seed = 256, 256, 12, 4, 6400 + T
    st = make_store(E, H, I, seed, device=dev, exact=True)
    rng = np.random.default_rng(T)
    p = np.array([0.3, 0.2, 0.1, 0.08, 0.07, 0.06, 0.05, 0.04, 0.04, 0.03, 0.02, 0.01])
    ids = np.stack([rng.choice(E, k, replace=False, p=p) for _ in range(T)]).astype(np.int64)
    counts = np.bincount(ids.ravel(), minlength=E)
    assert T > exl3.FAT_EXPERT_THRESHOLD and (counts > exl3.FAT_EXPERT_THRESHOLD).any()
    assert ((counts > 0) & (counts <= exl3.FAT_EXPERT_THRESHOLD)).any()
    w = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
    x = _t(rng.normal(0, 1, (T, H)).astype(np.float32), dev).to(torch.bfloat16)
    idd, wd = _t(ids, dev), _t(w, dev)
    print(f"graph capture T={T} counts={counts.tolist()}", flush=True)
    eager = exl3.apply_exl3_fused_moe(x, idd, wd, st, None, None, 10.0).clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        exl3.apply_exl3_fused_moe(x, idd, wd, st, None, None, 10.0)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        cap_out = exl3.apply_exl3_fused_moe(x, idd, wd, st, None, None, 10.0)
    for r in range(3):
        cap_out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(cap_out, eager), f"replay {r}"
        exl3.apply_exl3_fused_moe(x, idd, wd, st, None, None, 10.0)     # eager work between replays
        torch.cuda.synchronize()
    x16 = x.half().cpu().numpy().astype(np.float32)
    ref = OracleLayer(st, seed).forward(x16, ids, w.astype(np.float16).astype(np.float32))
    ok, m = within_tolerance(eager.cpu().numpy(), ref)
    assert ok, m
