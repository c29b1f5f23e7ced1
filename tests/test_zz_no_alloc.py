"""mm_moe_decode_noalloc (the decode layer on the library's own device scratch) against mm_moe_decode with a
caller workspace: bit-identical outputs on two calls in a row, the second with fewer routes, a clear error for a
call beyond the scratch size, and the call captured in a graph (after the device's first, eager call) replayed."""
import numpy as np
import pytest

from helpers import make_store

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _decode(st, x, ids, w, T, k, dev, noalloc):
    import torch
    from mi355moe import _lib
    out = torch.full((T, st.H), float("nan"), dtype=torch.float32, device=dev)
    if noalloc:
        _lib.call("mm_moe_decode_noalloc", st.mm_layer(), x.data_ptr(), _lib.DTYPE_BF16, 1, T, k, ids.data_ptr(),
                  w.data_ptr(), T * k, out.data_ptr(), _lib.stream_ptr())
    else:
        wsb = _lib.load().mm_gemv_workspace(T * k, st.E, st.H, st.I)
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        _lib.call("mm_moe_decode", st.mm_layer(), x.data_ptr(), _lib.DTYPE_BF16, 1, T, k, ids.data_ptr(), w.data_ptr(),
                  T * k, out.data_ptr(), ws.data_ptr(), wsb, _lib.stream_ptr())
    torch.cuda.synchronize()
    return out


def test_noalloc_decode_equals_workspace_decode(dev):
    import torch
    from mi355moe import _lib, workload
    H, I, E = 4096, 2048, 384
    st = make_store(E + 1, H, I, 7100, device=dev)
    for T in (6, 2):                     # the second call has fewer routes than the first
        ids, w = workload.zipf_routing(T, 8, E, seed=7200 + T)
        ids = np.concatenate([ids, np.full((T, 1), E)], 1)
        w = np.concatenate([w, np.ones((T, 1), np.float32)], 1)
        x = _t(workload.activations(T, H, seed=7300 + T), dev).to(torch.bfloat16)
        idd, wd = _t(ids, dev), _t(w, dev)
        print(f"noalloc decode T={T} routes={T * 9}", flush=True)
        a = _decode(st, x, idd, wd, T, 9, dev, noalloc=True)
        b = _decode(st, x, idd, wd, T, 9, dev, noalloc=False)
        assert torch.isfinite(a).all()
        assert torch.equal(a, b), f"T={T}: max diff {(a - b).abs().max().item()}"
    # beyond the scratch: a clear error, no device work (every argument sized for the call all the same)
    T = 8
    ids = np.tile(np.arange(9, dtype=np.int64), (T, 1))
    idd, wd, out = _t(ids, dev), _t(np.ones((T, 9), np.float32), dev), torch.empty((T, H), device=dev)
    x = _t(workload.activations(T, H, seed=7308), dev).to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="scratch"):
        _lib.call("mm_moe_decode_noalloc", st.mm_layer(), x.data_ptr(), _lib.DTYPE_BF16, 1, T, 9, idd.data_ptr(),
                  wd.data_ptr(), T * 9, out.data_ptr(), _lib.stream_ptr())


def test_noalloc_decode_captured_in_a_graph(dev):
    """The device's first call runs eagerly (it looks up the scratch address); a later call captured in a graph
    replays bit-identically to the workspace entry, three replays with eager work and synchronisations between."""
    import torch
    from mi355moe import _lib, workload
    H, I, E, T = 4096, 2048, 384, 4
    st = make_store(E + 1, H, I, 7400, device=dev)
    ids, w = workload.zipf_routing(T, 8, E, seed=7500)
    ids = np.concatenate([ids, np.full((T, 1), E)], 1)
    w = np.concatenate([w, np.ones((T, 1), np.float32)], 1)
    x = _t(workload.activations(T, H, seed=7600), dev).to(torch.bfloat16)
    idd, wd = _t(ids, dev), _t(w, dev)
    want = _decode(st, x, idd, wd, T, 9, dev, noalloc=False)
    first = _decode(st, x, idd, wd, T, 9, dev, noalloc=True)          # eager: the scratch address is looked up
    assert torch.equal(first, want)
    out = torch.empty((T, H), dtype=torch.float32, device=dev)
    layer = st.mm_layer()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            _lib.call("mm_moe_decode_noalloc", layer, x.data_ptr(), _lib.DTYPE_BF16, 1, T, 9, idd.data_ptr(),
                      wd.data_ptr(), T * 9, out.data_ptr(), _lib.stream_ptr())
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for r in range(3):
        out.fill_(float("nan"))
        junk = torch.randn(1 << 20, device=dev).sum()        # the program's own eager work between the replays
        torch.cuda.synchronize()
        print(f"noalloc graph replay {r}", flush=True)
        g.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        assert torch.equal(out, want), f"replay {r}: max diff {(out - want).abs().max().item()}"
