"""Checkpoint loading on the GPU: a checkpoint written from the synthetic generator loads into the same bits as
ExpertStore.synthesize, all in HBM or with the host plan's experts in a pinned host home (the rest in HBM rows),
and the loaded layers compute exactly what the synthesized layer computes."""
import numpy as np
import pytest

from golden import make_checkpoint

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_loaded_layers_equal_synthesized(dev, tmp_path):
    import torch
    from mi355moe import loader, moe
    from mi355moe.store import ExpertStore
    H, I, E, T, k = 512, 256, 6, 5, 3
    d = make_checkpoint.write(str(tmp_path / "ck"), layers=(0, 1), E=E, H=H, I=I,
                              plan={"model.layers.1.ffn.experts": [0, 2, 3]})
    print("loading checkpoint", flush=True)
    a, b = loader.load_model(d, device=dev, plan=str(tmp_path / "ck" / "host-plan.json"))
    ref = [ExpertStore(E, H, I, device=dev).synthesize(1000 + L) for L in (0, 1)]
    torch.cuda.synchronize()
    assert a.host_home is None and torch.equal(a.w13_trellis, ref[0].w13_trellis)
    assert torch.equal(a.w2_trellis, ref[0].w2_trellis)
    assert b.host_home is not None
    slot = b.slotof.cpu().numpy()
    assert (slot[[0, 2, 3]] == -1).all() and (slot[[1, 4, 5]] >= 1 << 30).all()
    g = b._exl3_ptrs["gate_trellis"].cpu().numpy()
    assert np.array_equal(g[[0, 2, 3]], b.home.numpy()[[0, 2, 3], 0])
    for k_ in ("w13_suh", "w13_svh", "w2_suh", "w2_svh"):
        assert torch.equal(getattr(b, k_), getattr(ref[1], k_))
    rng = np.random.default_rng(3)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int64)
    w = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
    x = _t(rng.normal(0, 1, (T, H)).astype(np.float32), dev).to(torch.bfloat16)
    for st, r in ((a, ref[0]), (b, ref[1])):
        o1 = moe.moe_forward(st, x, _t(ids, dev), _t(w, dev))
        o2 = moe.moe_forward(r, x, _t(ids, dev), _t(w, dev))
        torch.cuda.synchronize()
        assert torch.equal(o1, o2)
