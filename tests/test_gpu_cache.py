"""GPU tests of expert placement: slot-table repoints, copy-engine staging, experts read zero-copy from a pinned
host home, the expert cache end to end, the sorted-route fat entry and the staged prefill."""
import numpy as np
import pytest

from helpers import OracleLayer, make_store, within_tolerance

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _host_store(E, H, I, seed, dev, exact=True):
    import torch
    from mi355moe.cache import HostHome
    from mi355moe.store import ExpertStore
    st = ExpertStore(E, H, I, device=dev, exact=exact, host_home=HostHome(E, H, I)).synthesize(seed)
    torch.cuda.synchronize()
    return st


def test_slot_point_last_item_wins_and_skips_out_of_range(dev):
    import torch
    from mi355moe import _lib
    E = 50
    rng = np.random.default_rng(5)
    g0 = rng.integers(1, 1 << 40, E)
    tabs = [_t(g0 + j, dev) for j in range(3)]
    slotof = _t(np.full(E, -1, np.int32), dev)
    items = np.stack([rng.integers(-3, E + 3, 300), rng.integers(0, 1 << 40, 300), rng.integers(0, 1 << 40, 300),
                      rng.integers(0, 1 << 40, 300), rng.integers(-1, 700, 300)], 1).astype(np.int64)
    exp = [g0.copy(), g0 + 1, g0 + 2]
    exp_s = np.full(E, -1, np.int32)
    for it in items:                          # sequential application: the last item of an expert wins
        e = int(it[0])
        if 0 <= e < E:
            for j in range(3):
                exp[j][e] = it[1 + j]
            exp_s[e] = it[4]
    items_d = _t(items, dev)
    print("slot point 300 items", flush=True)
    _lib.call("mm_slot_point", tabs[0].data_ptr(), tabs[1].data_ptr(), tabs[2].data_ptr(), slotof.data_ptr(), E,
              items_d.data_ptr(), len(items), _lib.stream_ptr())
    torch.cuda.synchronize()
    for j in range(3):
        assert np.array_equal(tabs[j].cpu().numpy(), exp[j])
    assert np.array_equal(slotof.cpu().numpy(), exp_s)


def test_stage_copy_merges_and_moves_bytes(dev):
    import torch
    from mi355moe import cache
    from mi355moe.hostmem import HostBuffer
    hb = HostBuffer(1 << 20)
    src = hb.array(np.uint8)
    src[:] = np.random.default_rng(1).integers(0, 256, src.size, dtype=np.uint8)
    dst = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)
    d0, s0 = dst.data_ptr(), hb.ptr
    copies = [(d0, s0, 4096), (d0 + 4096, s0 + 4096, 8192), (d0 + 65536, s0 + 131072, 1000),
              (d0 + 200000, s0 + 300000, 0), (d0 + 500000, s0 + 10, 77)]
    print("stage copy", flush=True)
    n = cache.stage_copy(copies)
    torch.cuda.synchronize()
    assert n == 3                                         # the first two merge, the empty one is dropped
    got = dst.cpu().numpy()
    exp = np.zeros_like(got)
    for d, s, b in copies:
        exp[d - d0:d - d0 + b] = src[s - s0:s - s0 + b]
    assert np.array_equal(got, exp)


def test_copy_streams_checked_kept_and_ordered(dev):
    """mm_copy_stream: a stream seen to run beside the compute stream (MM_OK, not MM_COPY_UNVERIFIED), the same one
    on later calls, another one for another index; bad indices, devices and a capturing compute stream are errors;
    a staging copy on it ordered after the compute stream's write and before its read moves the right bytes."""
    import ctypes
    import torch
    from mi355moe import _lib, cache
    from mi355moe.hostmem import HostBuffer
    print("copy streams", flush=True)
    main = torch.cuda.current_stream()

    def raw(d, i, comp):
        p = _lib.vp()
        return _lib.load().mm_copy_stream(d, i, comp, ctypes.byref(p)), p.value
    rc0, p0 = raw(dev.index or 0, 0, main.cuda_stream)
    rc0b, p0b = raw(dev.index or 0, 0, main.cuda_stream)
    rc1, p1 = raw(dev.index or 0, 1, main.cuda_stream)
    assert (rc0, rc0b, rc1) == (0, 0, 0)
    assert p0 == p0b and p0 != p1 and p0 not in (None, main.cuda_stream)
    assert _lib.copy_stream(dev, 0).cuda_stream == p0
    for d, i in ((0, -1), (0, 4), (-1, 0), (torch.cuda.device_count(), 0)):
        assert raw(d, i, main.cuda_stream)[0] < 0
    comp = torch.cuda.Stream()                         # another compute stream: its own checked copy stream
    rc2, p2 = raw(dev.index or 0, 0, comp.cuda_stream)
    assert rc2 == 0 and p2 not in (None, comp.cuda_stream)
    with torch.cuda.stream(comp):
        assert _lib.copy_stream(dev, 0).cuda_stream == p2
    side = torch.cuda.Stream()
    one = torch.ones(1, device=dev)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        rc_cap = raw(dev.index or 0, 2, torch.cuda.current_stream().cuda_stream)[0]
        one.add_(1)
    assert rc_cap < 0
    n = 3 << 20
    hb = HostBuffer(n)
    src = hb.array(np.uint8)
    src[:] = np.random.default_rng(2).integers(0, 256, n, dtype=np.uint8)
    dst = torch.empty(n, dtype=torch.uint8, device=dev)
    dst.fill_(7)                                       # compute-stream write the copy must follow
    cs = _lib.copy_stream(dev, _lib.COPY_STAGING)
    cs.wait_stream(main)
    cache.stage_copy([(dst.data_ptr(), hb.ptr, n)], cs)
    ev = torch.cuda.Event()
    ev.record(cs)
    main.wait_event(ev)
    assert np.array_equal(dst.cpu().numpy(), src)


def test_host_resident_experts_zero_copy_equal_hbm(dev):
    """Experts read over PCIe from the pinned home give the HBM store's exact bits (same kernels, same words) and
    match the oracle; the synthetic words land in the host rows."""
    import torch
    from mi355moe import moe
    from mi355moe.store import trellis_words
    H, I, E, T, k, seed = 512, 256, 12, 6, 4, 77
    hs = _host_store(E, H, I, seed, dev)
    ds = make_store(E, H, I, seed, device=dev, exact=True)
    rows = hs.host_home.rows
    host = hs.host_home.buffer.array(np.int16, (E, rows.row_words))
    nm = trellis_words(H, I)
    assert np.array_equal(host[3, :2 * nm], ds.w13_trellis[3].cpu().numpy().reshape(-1))
    assert np.array_equal(host[3, 2 * nm:], ds.w2_trellis[3].cpu().numpy().reshape(-1))
    rng = np.random.default_rng(3)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
    w = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
    x16 = rng.normal(0, 1, (T, H)).astype(np.float16)
    print("zero-copy decode", flush=True)
    a = moe.moe_forward(hs, _t(x16, dev), _t(ids, dev), _t(w, dev))
    b = moe.moe_forward(ds, _t(x16, dev), _t(ids, dev), _t(w, dev))
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    ok, m = within_tolerance(a.cpu().numpy(), OracleLayer(ds, seed).forward(x16.astype(np.float32), ids, w))
    assert ok, m


def test_expert_cache_end_to_end(dev):
    """Three host-home layers, 10 cache slots, replans on routed counts: after every step the slot table names
    the cache's residents, resident slots hold the home bytes, the rest point home, and the layer output is
    bit-identical to the all-home output."""
    import torch
    from mi355moe import moe
    from mi355moe.cache import ExpertCache
    H, I, E, L, N = 256, 256, 16, 3, 10
    layers = [_host_store(E, H, I, 900 + li, dev) for li in range(L)]
    for st in layers:
        st.home_np = st.home.numpy().copy()
    c = ExpertCache(layers, slots=N, every=1, admit=4, decay=0.9, hyst=1.0, warmup=0, async_copy=True,
                    margin_mb=0, elastic=False)
    rng = np.random.default_rng(4)
    T, k = 4, 3
    x16 = _t(rng.normal(0, 1, (T, H)).astype(np.float16), dev)
    ids = [_t(np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64), dev) for _ in range(L)]
    w = _t(rng.uniform(0.1, 1.0, (T, k)).astype(np.float32), dev)
    base = [moe.moe_forward(st, x16, ids[li], w).clone() for li, st in enumerate(layers)]
    for step in range(12):
        counts = rng.poisson(rng.gamma(0.4, 4.0, (L, E)))
        c.step(counts=counts)
        torch.cuda.synchronize()
        live = dict(c.where)
        if c.pending:                                       # newcomers go live at the next replan
            for li, items in c.pending["items"].items():
                for it in items:
                    live.pop(li * E + it[0], None)
        rows = c.pool.rows
        for li, st in enumerate(layers):
            tabs = [st._exl3_ptrs[kk].cpu().numpy() for kk in ("gate_trellis", "up_trellis", "down_trellis")]
            slotof = st.slotof.cpu().numpy()
            for e in range(E):
                i = li * E + e
                if i in live:
                    s = live[i]
                    assert slotof[e] == s and tabs[0][e] == c.pool.row(s)
                    assert tabs[1][e] == c.pool.row(s) + 2 * rows.n_mat and tabs[2][e] == c.pool.row(s) + 4 * rows.n_mat
                    host = st.host_home.buffer.array(np.int16, (E, rows.row_words))[e]
                    assert np.array_equal(c.pool.t[s].cpu().numpy(), host)
                else:
                    assert slotof[e] == -1 and all(tabs[j][e] == st.home_np[e, j] for j in range(3))
            out = moe.moe_forward(st, x16, ids[li], w)
            torch.cuda.synchronize()
            assert torch.equal(out, base[li]), (step, li)
        print(f"cache step {step}: {c.summary()}", flush=True)
    assert c.admits > N and c.evicts > 0
    # release: every expert back home, then rewarm re-admits the kept set
    c.release()
    for st in layers:
        assert np.all(st.slotof.cpu().numpy() == -1)
    c.rewarm()
    torch.cuda.synchronize()
    assert len(c.where) == min(N, len(c.keep))
    for li, st in enumerate(layers):
        assert torch.equal(moe.moe_forward(st, x16, ids[li], w), base[li])


def test_fat_batched_sorted_routes_match_oracle(dev):
    """mm_fat_batched on expert-sorted routes (fp16 weights, skip set, cap) against the oracle on the selected
    experts, accumulating into out."""
    import torch
    from mi355moe import exl3, moe
    H, I, E, T, k, seed = 512, 256, 8, 160, 3, 606
    st = make_store(E, H, I, seed, device=dev, exact=True)
    rng = np.random.default_rng(7)
    p = np.array([0.3, 0.25, 0.15, 0.1, 0.08, 0.06, 0.04, 0.02])
    ids = np.stack([rng.choice(E, k, replace=False, p=p) for _ in range(T)]).astype(np.int64)
    w = rng.uniform(0.1, 1.0, (T, k)).astype(np.float16).astype(np.float32)
    x16 = rng.normal(0, 1, (T, H)).astype(np.float16)
    r = moe.permute(_t(ids, dev), _t(w, dev), k, E)
    counts = r["counts"][:E].cpu().numpy()
    cap = int(np.sort(counts)[2])                     # the three least-routed experts are not fat
    skip = {int(np.argmax(counts))}                   # and the busiest is handled elsewhere
    n = T * k
    base = _t(rng.normal(0, 1, (T, H)).astype(np.float32), dev)
    out = base.clone()
    print(f"fat batched cap={cap} skip={skip} counts={counts.tolist()}", flush=True)
    exl3.apply_exl3_batched_fat(_t(x16, dev), r["token_sorted"][:n].long(), r["weight_sorted"][:n].half(),
                                counts.tolist(), exl3.layer_inners(st), 10.0, cap, out, skip=skip)
    torch.cuda.synchronize()
    sel = np.array([(counts[e] > cap) and (e not in skip) for e in range(E)])
    mids = np.where(sel[ids], ids, -1)
    ref = OracleLayer(st, seed).forward(x16.astype(np.float32), mids, w)
    got = (out - base).cpu().numpy()
    ok, m = within_tolerance(got, ref)
    assert ok, m
    # the same routes through mm_moe_prefill (ids form, cap) agree within tolerance
    pre = moe.moe_prefill(st, _t(x16, dev), _t(mids, dev), _t(w, dev), cap=cap)
    ok, m = within_tolerance(got, pre.cpu().numpy().astype(np.float64))
    assert ok, m


def test_run_batch_from_staging_slots(dev):
    """dma_gemm.run_batch: busy experts of one batch run from their staging-slot rows (filled by the copy
    engines from the pinned home) and equal the same experts computed from the home copy."""
    import torch
    from mi355moe import cache, dma_gemm, exl3, moe
    H, I, E, T, k, seed = 256, 256, 12, 200, 2, 707
    st = _host_store(E, H, I, seed, dev)
    rng = np.random.default_rng(8)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
    w = rng.uniform(0.1, 1.0, (T, k)).astype(np.float16).astype(np.float32)
    x16 = _t(rng.normal(0, 1, (T, H)).astype(np.float16), dev)
    r = moe.permute(_t(ids, dev), _t(w, dev), k, E)
    counts = r["counts"][:E].cpu().numpy().tolist()
    n = T * k
    NS, B = 2, 4
    pool = cache.SlotPool(NS * B, H, I, dev)
    stg = {"slots": pool, "free": [None] * NS}
    cold = list(range(E))
    D = {"batches": [(i, min(i + B, E)) for i in range(0, E, B)], "cold": cold}
    batch = 1
    slot = batch % NS
    first, last = D["batches"][batch]
    cl = [(pool.row(slot * B + r_), st.host_home.row(e), pool.rows.row_bytes) for r_, e in enumerate(cold[first:last])]
    cache.stage_copy(cl)
    cap = 30
    tok, wsd = r["token_sorted"][:n].long(), r["weight_sorted"][:n].half()
    out = torch.zeros((T, H), dtype=torch.float32, device=dev)
    print(f"run_batch counts={counts}", flush=True)
    dma_gemm.run_batch(D, stg, batch, exl3.layer_inners(st), counts, cap, x16, tok, wsd, 10.0, out,
                       exl3.apply_exl3_batched_fat, True)
    busy = {e for e in cold[first:last] if counts[e] > cap}
    assert busy
    ref = torch.zeros_like(out)
    exl3.apply_exl3_batched_fat(x16, tok, wsd, counts, exl3.layer_inners(st), 10.0, cap, ref,
                                skip=set(range(E)) - busy)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert float(out.abs().max()) > 0


def test_staged_prefill_matches_hbm_layer(dev):
    """apply_exl3_fused_moe with host-resident experts and the staging path (some experts cached in slots, the
    rest streamed in batches of B through NS slots) matches the oracle and the HBM store's fat path."""
    import torch
    from mi355moe import exl3, moe
    from mi355moe.cache import ExpertCache
    H, I, E, T, k, seed = 512, 256, 20, 300, 4, 808
    hs = _host_store(E, H, I, seed, dev)
    ds = make_store(E, H, I, seed, device=dev, exact=True)
    saved = (exl3._EXL3_HOST_DMA_MODE, exl3._DMA_B, exl3._DMA_NS, exl3._DMA_MIN_TOKENS, dict(exl3._DMA_STATE))
    try:
        exl3._EXL3_HOST_DMA_MODE, exl3._DMA_B, exl3._DMA_NS, exl3._DMA_MIN_TOKENS = 1, 3, 2, 64
        exl3._DMA_STATE.clear()
        exl3._DMA_LAST.clear()
        exl3.Exl3MoEMethod().process_weights_after_loading(hs)
        c = ExpertCache([hs], slots=5, every=1, admit=5, warmup=0, async_copy=False, margin_mb=0, elastic=False)
        cnt = np.zeros((1, E))
        cnt[0, [2, 5, 11, 17, 19]] = [9, 8, 7, 6, 5]
        c.step(counts=cnt)                                  # five experts cached in slots
        rng = np.random.default_rng(9)
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
        ids[::7, 0] = -1
        wts = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
        x = rng.normal(0, 1, (T, H)).astype(np.float32)
        xb = _t(x, dev).to(torch.bfloat16)
        print("staged prefill", flush=True)
        out = exl3.apply_exl3_fused_moe(xb, _t(ids, dev), _t(wts, dev), hs, None, None, 10.0)
        torch.cuda.synchronize()
        assert hs._exl3_dma["batches"] == 5 and hs._exl3_dma["bytes"] == 15 * hs.host_home.rows.row_bytes
        w16 = wts.astype(np.float16).astype(np.float32)
        x16 = xb.half().cpu().numpy().astype(np.float32)
        ok, m = within_tolerance(out.cpu().numpy(), OracleLayer(ds, seed).forward(x16, ids, w16))
        assert ok, m
        ref = moe.moe_prefill(ds, xb, _t(ids, dev), _t(w16, dev))
        ok, m = within_tolerance(out.cpu().numpy(), ref.cpu().numpy().astype(np.float64))
        assert ok, m
    finally:
        exl3._EXL3_HOST_DMA_MODE, exl3._DMA_B, exl3._DMA_NS, exl3._DMA_MIN_TOKENS = saved[:4]
        exl3._DMA_STATE.clear()
        exl3._DMA_LAST.clear()
        exl3._DMA_STATE.update(saved[4])


def test_plugin_entry_and_tier_split(dev, monkeypatch):
    """install() wraps the plugin: decode-sized calls of a tier layer go through mm_split (hit / miss counts per
    distinct expert against the slot table, routed counts for the cache) and give the plugin's own output."""
    import torch
    from mi355moe import ct_vllm, exl3
    import oracle as O
    H, I, E, T, k, seed = 512, 256, 24, 4, 8, 909
    hs = _host_store(E, H, I, seed, dev)
    ct_vllm.reset()
    monkeypatch.setenv("DSV41_CT_LAYERS", "1")
    try:
        ct_vllm.install(exl3)
        exl3.Exl3MoEMethod().process_weights_after_loading(hs)       # the wrapped hook registers the layer
        assert ct_vllm.S["layers"] == [hs] and ct_vllm.S["started"] and hs._ct["li"] == 0
        slot = np.full(E, -1, np.int32)
        slot[[1, 4, 9, 10, 15]] = [0, 1, 2, 3, 4]
        hs.slotof.copy_(_t(slot, dev))
        rng = np.random.default_rng(10)
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
        wts = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
        xb = _t(rng.normal(0, 1, (T, H)).astype(np.float32), dev).to(torch.bfloat16)
        print("tier split", flush=True)
        out = exl3.apply_exl3_fused_moe(xb, _t(ids, dev), _t(wts, dev), hs, None, None, 10.0)
        direct = ct_vllm._ORIG["fused"](xb, _t(ids, dev), _t(wts, dev), hs, None, None, 10.0)
        torch.cuda.synchronize()
        assert torch.equal(out, direct)
        s = ct_vllm.summary()
        touched = np.unique(ids)
        assert s["hits"] == int((slot[touched] >= 0).sum()) and s["misses"] == int((slot[touched] < 0).sum())
        assert np.array_equal(hs.counts.cpu().numpy(), np.bincount(ids.reshape(-1), minlength=E))
        ref = O.split(ids.reshape(-1), wts.reshape(-1), xb.half().cpu().numpy(), E, slot, np.zeros(E, np.float32),
                      ct_vllm.S["pol"].cpu().numpy())
        assert s["hits"] == int(ref["stats"][0]) and s["misses"] == int(ref["stats"][1])
    finally:
        ct_vllm.uninstall(exl3)
        ct_vllm.reset()


def test_cross_layer_prefetch_outputs_identical(dev):
    """Staged prefill through three host-resident layers: with the cross-layer prefetch the second and third
    layers start on batches the previous layer queued, and every layer's output is bit-identical to the run
    without it."""
    import torch
    from mi355moe import exl3
    H, I, E, T, k = 512, 256, 24, 200, 4
    saved = (exl3._EXL3_HOST_DMA_MODE, exl3._DMA_B, exl3._DMA_NS, exl3._DMA_MIN_TOKENS, exl3._DMA_PREFETCH,
             dict(exl3._DMA_STATE), dict(exl3._DMA_LAST))
    try:
        exl3._EXL3_HOST_DMA_MODE, exl3._DMA_B, exl3._DMA_NS, exl3._DMA_MIN_TOKENS = 1, 4, 2, 64
        exl3._DMA_STATE.clear()
        exl3._DMA_LAST.clear()
        layers = [_host_store(E, H, I, 1700 + l, dev, exact=False) for l in range(3)]
        for st in layers:
            exl3.Exl3MoEMethod().process_weights_after_loading(st)
        rng = np.random.default_rng(17)
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
        wts = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
        x = _t(rng.normal(0, 1, (T, H)).astype(np.float32), dev).to(torch.bfloat16)
        outs = {}
        for pf in (False, True):
            exl3._DMA_PREFETCH = pf
            for st in layers:
                st._exl3_dma["prefetched"] = 0
            print(f"three staged layers, prefetch {pf}", flush=True)
            outs[pf] = [exl3.apply_exl3_fused_moe(x, _t(ids, dev), _t(wts, dev), st, None, None, 10.0) for st in layers]
            torch.cuda.synchronize()
            pre = [st._exl3_dma["prefetched"] for st in layers]
            assert pre == ([0, 2, 2] if pf else [0, 0, 0]), pre
        for a, b in zip(outs[False], outs[True]):
            assert torch.equal(a, b)
    finally:
        (exl3._EXL3_HOST_DMA_MODE, exl3._DMA_B, exl3._DMA_NS, exl3._DMA_MIN_TOKENS, exl3._DMA_PREFETCH) = saved[:5]
        exl3._DMA_STATE.clear()
        exl3._DMA_STATE.update(saved[5])
        exl3._DMA_LAST.clear()
        exl3._DMA_LAST.update(saved[6])


def test_read_probe_reads_every_word(dev):
    """The HBM read calibration loads every 16-byte vector once: its xor equals numpy's over the buffer, for a
    size that leaves a remainder past the four-vector loop, with the default and a small grid."""
    import torch
    from mi355moe import _lib
    rng = np.random.default_rng(5)
    words = rng.integers(0, 2 ** 32, (1 << 20) + 44, dtype=np.uint64).astype(np.uint32)
    want = np.bitwise_xor.reduce(words)
    buf = torch.from_numpy(words.view(np.int32)).to(dev)
    for blocks in (0, 3):
        sink = torch.zeros(1, dtype=torch.int32, device=dev)
        _lib.call("mm_read_probe", buf.data_ptr(), words.nbytes, sink.data_ptr(), blocks, _lib.stream_ptr())
        torch.cuda.synchronize()
        assert int(sink.cpu().numpy().view(np.uint32)[0]) == int(want)
