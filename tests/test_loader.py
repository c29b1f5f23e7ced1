"""The EXL3 checkpoint loader and the host plan on the CPU: a checkpoint written by tests/golden/make_checkpoint.py
from the synthetic generator loads into exactly the generator's words and scales; plan matching, refusal of the
mcg codebook and of mismatched shapes."""
import json

import numpy as np
import pytest

import oracle as O
from golden import make_checkpoint


def test_checkpoint_loads_generator_bits(tmp_path):
    from mi355moe import loader
    from mi355moe.store import synth_scales
    H, I, E = 256, 128, 5
    d = make_checkpoint.write(str(tmp_path / "ck"), layers=(0, 3), E=E, H=H, I=I, prefix="language_model.model.")
    ck = loader.Checkpoint(d)
    assert ck.shape(3) == (E, H, I)
    for L in (0, 3):
        st = loader.load_layer(ck, L, device="cpu")
        sc = synth_scales(1000 + L, E, H, I)
        for e in range(E):
            g, u, dd = O.synth_expert_trellis(1000 + L, e, H, I)
            assert np.array_equal(st.w13_trellis[e, 0].numpy().view(np.uint16), g)
            assert np.array_equal(st.w13_trellis[e, 1].numpy().view(np.uint16), u)
            assert np.array_equal(st.w2_trellis[e].numpy().view(np.uint16), dd)
        for k in ("w13_suh", "w13_svh", "w2_suh", "w2_svh"):
            assert np.array_equal(getattr(st, k).numpy(), sc[k]), k


def test_host_plan_matching(tmp_path):
    from mi355moe import loader
    p = str(tmp_path / "plan.json")
    loader.write_host_plan(p, 3, 4)
    plan = loader.read_host_plan(p)
    assert loader.host_plan_for(plan, "model.layers.2.ffn.experts") == [0, 1, 2, 3]
    assert loader.host_plan_for(plan, "language_model.model.layers.1.ffn.experts") == [0, 1, 2, 3]
    assert loader.host_plan_for(plan, "layers.0.ffn.experts") == [0, 1, 2, 3]
    assert loader.host_plan_for(plan, "model.layers.7.ffn.experts") is None
    with open(p, "w") as f:
        json.dump({"model.layers.0.ffn.experts": [3, 1, 3]}, f)
    assert loader.host_plan_for(loader.read_host_plan(p), "model.layers.0.ffn.experts") == [1, 3]


def test_refuses_mcg_codebook_and_bad_shapes(tmp_path):
    import torch
    from safetensors.torch import save_file
    from mi355moe import loader
    d = make_checkpoint.write(str(tmp_path / "mcg"), layers=(0,), E=2, mcg=True)
    with pytest.raises(NotImplementedError):
        loader.load_layer(d, 0, device="cpu")
    bad = str(tmp_path / "bad.safetensors")
    t = {}
    for e in range(2):
        for w, shp in (("w1", (16, 8, 48)), ("w3", (16, 8, 48)), ("w2", (8, 16, 40))):
            t[f"layers.0.ffn.experts.{e}.{w}.trellis"] = torch.zeros(shp, dtype=torch.int16)
            t[f"layers.0.ffn.experts.{e}.{w}.suh"] = torch.zeros(256 if w != "w2" else 128, dtype=torch.float16)
            t[f"layers.0.ffn.experts.{e}.{w}.svh"] = torch.zeros(128 if w != "w2" else 256, dtype=torch.float16)
    save_file(t, bad)
    with pytest.raises(ValueError):
        loader.load_layer(bad, 0, device="cpu")


def test_prefixed_key_lookup_is_indexed():
    """A full-size key set with a prefix (40 layers x 384 experts x 9 tensors): every lookup is a dict probe, so
    all of one layer's expert lookups take well under a second."""
    import time
    from mi355moe.loader import Checkpoint
    ck = object.__new__(Checkpoint)
    ck.where = {f"model.layers.{L}.ffn.experts.{e}.{w}.{p}": "f" for L in range(40) for e in range(384)
                for w in ("w1", "w3", "w2") for p in ("trellis", "suh", "svh")}
    ck.where["model.layers.0.self_attn.q_proj.weight"] = "f"
    ck._index()
    t0 = time.perf_counter()
    for e in range(384):
        for w in ("w1", "w3", "w2"):
            for p in ("trellis", "suh", "svh"):
                assert ck._key(39, e, w, p) == f"model.layers.39.ffn.experts.{e}.{w}.{p}"
    assert time.perf_counter() - t0 < 1.0
    assert ck.num_experts(39) == 384
