"""Writes a small EXL3 checkpoint in the served pack's key layout from this build's synthetic generator (the same
words ExpertStore.synthesize puts on the GPU): layers.{L}.ffn.experts.{e}.{w1,w3,w2}.{trellis,suh,svh}, split
over two safetensors files with a model.safetensors.index.json, plus a host-plan.json. Used by the loader tests;
run as a script to write one into a directory:  python tests/golden/make_checkpoint.py OUT_DIR"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (os.path.join(ROOT, "oracle"), os.path.join(ROOT, "dsv41-flash-offload_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def write(out, layers=(0, 1), E=5, H=256, I=128, seed0=1000, prefix="model.", mcg=False, plan=None):
    """Layer L's experts use the generator streams of layer seed seed0 + L. Returns the directory."""
    import torch
    from safetensors.torch import save_file
    import oracle as O
    from mi355moe.store import synth_scales
    os.makedirs(out, exist_ok=True)
    files = [{}, {}]
    for li, L in enumerate(layers):
        seed = seed0 + L
        sc = synth_scales(seed, E, H, I)
        for e in range(E):
            g, u, d = O.synth_expert_trellis(seed, e, H, I)
            b = f"{prefix}layers.{L}.ffn.experts.{e}"
            part = files[(li + e) % 2]
            for w, tr, s, v in (("w1", g, sc["w13_suh"][e, 0], sc["w13_svh"][e, 0]),
                                ("w3", u, sc["w13_suh"][e, 1], sc["w13_svh"][e, 1]),
                                ("w2", d, sc["w2_suh"][e], sc["w2_svh"][e])):
                part[f"{b}.{w}.trellis"] = torch.from_numpy(tr.view(np.int16).copy())
                part[f"{b}.{w}.suh"] = torch.from_numpy(np.ascontiguousarray(s))
                part[f"{b}.{w}.svh"] = torch.from_numpy(np.ascontiguousarray(v))
                if mcg:
                    part[f"{b}.{w}.mcg"] = torch.ones(1, dtype=torch.int32)
    wm = {}
    for j, part in enumerate(files):
        name = f"model-{j + 1:05d}-of-00002.safetensors"
        save_file(part, os.path.join(out, name))
        wm.update({k: name for k in part})
    with open(os.path.join(out, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wm}, f)
    if plan is None:
        plan = {f"model.layers.{L}.ffn.experts": list(range(E)) for L in layers}
    with open(os.path.join(out, "host-plan.json"), "w") as f:
        json.dump(plan, f)
    return out


if __name__ == "__main__":
    print(write(sys.argv[1] if len(sys.argv) > 1 else "ckpt"))
