"""GPU parity of the fat-expert path: per-expert grouped GEMM with the EXL3 weights decoded into LDS (fp16) and
multiplied on MFMA, fused output transforms / SwiGLU / down-input transform, and the prefill layer."""
import os

import numpy as np
import pytest

from helpers import OracleLayer, make_store, within_tolerance

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_fat_expert_matches_reference_golden(dev):
    """The two experts of the compiled reference's golden file, each fed 130 routes (one full 128-route tile and a
    partial one), through the grouped GEMM: every route's row equals the reference's output."""
    import torch
    from mi355moe import moe
    g = np.load(os.path.join(GOLD, "expert_4096x2048.npz"), allow_pickle=False)
    H, I = int(g["H"]), int(g["I"])
    E = 256
    st = make_store(E, H, I, int(g["layer_seed"]), device=dev, exact=True)
    es = [int(g["e0"]), int(g["e1"])]
    for j, e in enumerate(es):
        st.w13_suh[e, 0].copy_(_t(g[f"suh_g{j}"], dev)); st.w13_svh[e, 0].copy_(_t(g[f"svh_g{j}"], dev))
        st.w13_suh[e, 1].copy_(_t(g[f"suh_u{j}"], dev)); st.w13_svh[e, 1].copy_(_t(g[f"svh_u{j}"], dev))
        st.w2_suh[e].copy_(_t(g[f"suh_d{j}"], dev)); st.w2_svh[e].copy_(_t(g[f"svh_d{j}"], dev))
    R = 130
    x = np.concatenate([np.repeat(g["x0"][None, :], R, 0), np.repeat(g["x1"][None, :], R, 0)]).astype(np.float16)
    ids = np.array([[es[0]]] * R + [[es[1]]] * R, np.int64)
    for lim in (10, 0):
        st.limit = float(lim)
        st._c = None
        print(f"fat golden limit {lim}", flush=True)
        Y = moe.grouped_gemm(st, _t(x, dev), _t(ids, dev), cap=0)
        torch.cuda.synchronize()
        Yg = Y.cpu().numpy()
        for j in (0, 1):
            ref = np.repeat(g[f"y{j}_lim{lim}"][None, :], R, 0)
            ok, m = within_tolerance(Yg[j * R:(j + 1) * R], ref)
            assert ok, (j, m)


@pytest.mark.parametrize("H,I,E,T,k", [(256, 128, 4, 200, 2), (512, 384, 6, 300, 3), (1024, 256, 3, 150, 2)])
def test_fat_small_shapes_vs_oracle(dev, H, I, E, T, k):
    import torch
    from mi355moe import moe
    seed = 777 + H + I
    st = make_store(E, H, I, seed, device=dev, exact=True)
    rng = np.random.default_rng(H * 3 + I)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
    w = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
    x16 = rng.normal(0, 1, (T, H)).astype(np.float16)
    print(f"fat small H={H} I={I} E={E} T={T} k={k}", flush=True)
    out = moe.moe_prefill(st, _t(x16, dev), _t(ids, dev), _t(w, dev))
    torch.cuda.synchronize()
    ref = OracleLayer(st, seed).forward(x16.astype(np.float32), ids, w)
    ok, m = within_tolerance(out.cpu().numpy(), ref)
    assert ok, m


def test_fat_tile_boundaries(dev):
    """Experts with 1, 128, 129, 192, 256 and 257 routes: 128-route tiles holding one route, 256-route tiles whose
    second row half holds 1 or 64 routes (those waves skip their empty row blocks), a full tile, and a full tile
    followed by a one-route tile."""
    import torch
    from mi355moe import moe
    H, I, seed = 256, 128, 8080
    counts = [1, 128, 129, 192, 256, 257]
    E = len(counts)
    st = make_store(E, H, I, seed, device=dev, exact=True)
    rng = np.random.default_rng(12)
    ids = rng.permutation(np.repeat(np.arange(E), counts)).astype(np.int64)[:, None]
    T = ids.shape[0]
    w = np.ones((T, 1), np.float32)
    x16 = rng.normal(0, 1, (T, H)).astype(np.float16)
    print(f"fat tile boundaries T={T}", flush=True)
    out = moe.moe_prefill(st, _t(x16, dev), _t(ids, dev), _t(w, dev))
    torch.cuda.synchronize()
    ref = OracleLayer(st, seed).forward(x16.astype(np.float32), ids, w)
    for e in range(E):
        rows = ids[:, 0] == e
        ok, m = within_tolerance(out.cpu().numpy()[rows], ref[rows])
        assert ok, (counts[e], m)


def test_grouped_gemm_rows_of_fat_experts_only(dev):
    """Only routes of experts above cap get rows; masked ids (-1, >= E) and small experts are left untouched."""
    import torch
    from mi355moe import moe
    H, I, E, T, k = 512, 256, 6, 160, 2
    seed = 4321
    st = make_store(E, H, I, seed, device=dev, exact=True)
    rng = np.random.default_rng(8)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
    ids[ids == 5] = 4                                  # expert 4 busy, expert 5 idle
    ids[:, 1] = np.where(ids[:, 0] == 4, 2, ids[:, 1])  # no token picks 4 twice
    ids[::3, 1] = 1                                    # expert 1 busy too
    ids[np.arange(T) % 7 == 2, 0] = -1
    ids[np.arange(T) % 11 == 5, 1] = E + 3
    counts = np.bincount(ids[(ids >= 0) & (ids < E)], minlength=E)
    cap = int(np.sort(counts)[-3])                     # the two busiest experts are fat
    x16 = rng.normal(0, 1, (T, H)).astype(np.float16)
    print(f"grouped gemm cap={cap} counts={counts.tolist()}", flush=True)
    Y = moe.grouped_gemm(st, _t(x16, dev), _t(ids, dev), cap=cap)
    torch.cuda.synchronize()
    Yg = Y.cpu().numpy()
    flat = ids.reshape(-1)
    fat = (flat >= 0) & (flat < E) & (counts[np.clip(flat, 0, E - 1)] > cap)
    assert fat.sum() > 128 and (~fat).sum() > 0
    assert np.all(Yg[~fat] == 0.0)
    ref = OracleLayer(st, seed).per_route(x16.astype(np.float32), ids)
    ok, m = within_tolerance(Yg[fat], ref[fat])
    assert ok, m


def test_threshold_split_matches_oracle(dev):
    """moe_forward sends experts above the threshold to the grouped GEMM and the rest to the decode path."""
    import torch
    from mi355moe import moe
    H, I, E, T, k = 512, 256, 8, 120, 2
    seed = 515
    st = make_store(E, H, I, seed, device=dev, exact=True)
    rng = np.random.default_rng(12)
    p = np.array([0.4, 0.3, 0.1, 0.08, 0.05, 0.04, 0.02, 0.01])
    ids = np.stack([rng.choice(E, k, replace=False, p=p) for _ in range(T)]).astype(np.int64)
    w = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
    x16 = rng.normal(0, 1, (T, H)).astype(np.float16)
    counts = np.bincount(ids.reshape(-1), minlength=E)
    print(f"threshold split counts={counts.tolist()}", flush=True)
    assert (counts > 40).any() and ((counts > 0) & (counts <= 40)).any()
    out = moe.moe_forward(st, _t(x16, dev), _t(ids, dev), _t(w, dev), fat_threshold=40)
    torch.cuda.synchronize()
    ref = OracleLayer(st, seed).forward(x16.astype(np.float32), ids, w)
    ok, m = within_tolerance(out.cpu().numpy(), ref)
    assert ok, m


def test_prefill_full_shape_matches_decode_path(dev):
    """H 4096, I 2048, 384 routed + 1 shared expert, top-8 Zipf routing over 256 tokens: the prefill layer equals
    the decode path (every expert <= 256 routes) with fp16 weights, and the oracle on sampled tokens."""
    import torch
    from mi355moe import moe, workload
    H, I, E, T = 4096, 2048, 384, 256
    seed = 3100
    st = make_store(E + 1, H, I, seed, device=dev, exact=True)
    ids, w = workload.zipf_routing(T, 8, E, seed=3101)
    x16 = workload.activations(T, H, seed=3102).astype(np.float16)
    xd, idd, wd = _t(x16, dev), _t(ids, dev), _t(w, dev)
    print("prefill full shape T=256", flush=True)
    a = moe.moe_prefill(st, xd, idd, wd, shared_expert=E)
    b = moe.moe_forward(st, xd, idd, wd, shared_expert=E, fat_threshold=T)
    torch.cuda.synchronize()
    a, b = a.cpu().numpy(), b.cpu().numpy()
    ok, m = within_tolerance(a, b.astype(np.float64))
    print("prefill vs decode", m, flush=True)
    assert ok, m
    rows = [0, 97, 255]
    ids_ext = np.concatenate([ids, np.full((T, 1), E)], 1)
    w_ext = np.concatenate([w, np.ones((T, 1), np.float32)], 1)
    ref = OracleLayer(st, seed).forward(x16[rows].astype(np.float32), ids_ext[rows], w_ext[rows])
    ok, m = within_tolerance(a[rows], ref)
    assert ok, m


def test_prefill_16k_tokens_deterministic_and_sampled(dev):
    """The 16k-token prefill layer (16384 tokens, top-8 Zipf over 384 experts + shared): two runs are bit-equal,
    accumulate adds onto out, and sampled tokens match the oracle."""
    import torch
    from mi355moe import moe, workload
    H, I, E, T = 4096, 2048, 384, 16384
    seed = 3200
    st = make_store(E + 1, H, I, seed, device=dev, exact=True)
    ids, w = workload.zipf_routing(T, 8, E, seed=3201)
    x16 = workload.activations(T, H, seed=3202).astype(np.float16)
    xd, idd, wd = _t(x16, dev), _t(ids, dev), _t(w, dev)
    print("prefill 16k tokens", flush=True)
    a = moe.moe_prefill(st, xd, idd, wd, shared_expert=E)
    b = moe.moe_prefill(st, xd, idd, wd, shared_expert=E)
    c = moe.moe_prefill(st, xd, idd, wd, shared_expert=E, out=a.clone())
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    # accumulate: out starts from a and adds the same routes in the same order
    assert torch.allclose(c, a + a, rtol=1e-5, atol=1e-5 * float(a.abs().max()))
    rows = [0, 8191, 16383]
    ids_ext = np.concatenate([ids, np.full((T, 1), E)], 1)
    w_ext = np.concatenate([w, np.ones((T, 1), np.float32)], 1)
    ref = OracleLayer(st, seed).forward(x16[rows].astype(np.float32), ids_ext[rows], w_ext[rows])
    ok, m = within_tolerance(a.cpu().numpy()[rows], ref)
    print("16k sampled", m, flush=True)
    assert ok, m


@pytest.mark.parametrize("T,k,E,cap", [(600, 4, 40, 32), (90, 6, 24, 20)])
def test_fused_moe_device_split_vs_oracle(dev, T, k, E, cap):
    """mm_fused_moe: experts above cap on the grouped GEMM, the rest on the decode path, split on the device --
    through the decode path's permutation (2,400 routes, positions bounded by E x cap) and its in-kernel routing
    (540 routes)."""
    import torch
    from mi355moe import moe
    H, I = 512, 256
    seed = 7700 + T
    st = make_store(E, H, I, seed, device=dev)
    rng = np.random.default_rng(T)
    p = np.concatenate([np.full(E // 4, 3.0), np.ones(E - E // 4)])
    p /= p.sum()
    ids = np.stack([rng.choice(E, k, replace=False, p=p) for _ in range(T)]).astype(np.int64)
    ids[::11, 1] = -1
    counts = np.bincount(ids[ids >= 0], minlength=E)
    assert (counts > cap).any() and ((counts > 0) & (counts <= cap)).any()
    w = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
    x16 = rng.normal(0, 1, (T, H)).astype(np.float16)
    print(f"fused device split T={T} k={k} counts={counts.tolist()}", flush=True)
    out = moe.fused_moe(st, _t(x16, dev), _t(ids, dev), _t(w, dev), cap)
    again = moe.fused_moe(st, _t(x16, dev), _t(ids, dev), _t(w, dev), cap)
    torch.cuda.synchronize()
    assert torch.equal(out, again)
    ref = OracleLayer(st, seed).forward(x16.astype(np.float32), ids, w)
    ok, m = within_tolerance(out.cpu().numpy(), ref)
    assert ok, m
