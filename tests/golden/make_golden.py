"""Write the golden vectors that pin the oracle, from the reference's own CPU expert kernel.

Builds oracle/_ref/libftref.so from the reference checkout (kernels/cpu_avx2/ft_core.h, compiled in place by
oracle/Makefile) and records, for seeded synthetic inputs:
  dense_256x256.npz     dense fp16 weights of a 256 x 256 trellis matrix (ft_core.h:977-992)
  expert_4096x2048.npz  double-accumulation expert outputs of two experts, SwiGLU limit 10 and 0
                        (ft_core.h:1004-1011)
  tier_t4.npz           the CPU tier's MoE forward for 4 tokens in modes AFFINE / EXACT / I16
                        (ft_core.h:703-727)
Inputs are stored with the outputs, except trellis words, which come from the synthetic generator
(stored as seeds plus a checksum that the tests re-verify).

Run from the repo root:  python tests/golden/make_golden.py
With --check nothing is written: every vector is recomputed and compared bit for bit with the committed fixture
(oracle/asan_check.sh runs this against the sanitizer build of the reference kernel, named by MM_REF_LIB).
"""
import ctypes
import hashlib
import os
import subprocess
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
REF = os.environ.get("REF", "/root/reference")


def P(a):
    return ctypes.c_void_p(a.ctypes.data)


def padded(a):
    """Copy into a buffer with a 4 KiB tail: the reference's AVX2 decode reads 8 B past a tile's end."""
    b = np.zeros(a.size + 2048, dtype=np.uint16)
    b[: a.size] = a.ravel()
    return b


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main():
    check = "--check" in sys.argv[1:]
    lib = os.environ.get("MM_REF_LIB")
    if not lib:
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "ref", f"REF={REF}"], check=True)
        lib = os.path.join(ROOT, "oracle", "_ref", "libftref.so")
    R = ctypes.CDLL(lib)

    def save(name, **rec):
        path = os.path.join(OUT, name)
        if not check:
            np.savez_compressed(path, **rec)
            return
        old = np.load(path, allow_pickle=False)
        worst = 0.0
        for k, v in rec.items():
            a, b = np.asarray(v), old[k]
            if a.shape != b.shape:
                raise SystemExit(f"{name}: {k} has another shape than the committed fixture")
            if a.tobytes() == b.tobytes():
                continue
            if a.dtype != np.float32:
                raise SystemExit(f"{name}: {k} differs from the committed fixture")
            # fp32 outputs of a build at another optimisation level: the summation order may differ (the AFFINE
            # tier mode forms KINV * S + KBIAS * sum(x), which amplifies it); the bound is the parity tolerance
            rel = float(np.abs(a.astype(np.float64) - b).max() / max(np.abs(b).max(), 1e-30))
            worst = max(worst, rel)
            if rel > 2e-3:
                raise SystemExit(f"{name}: {k} differs from the committed fixture (max rel {rel:.2e})")
        print(f"{name}: {len(rec)} entries equal the committed fixture (fp32 outputs within {worst:.1e})")

    # dense weights
    K = N = 256
    seed = 0x5EED0001
    tr = O.synth_u16(seed, 0, K * N * 3 // 16)
    W = np.empty((K, N), np.float32)
    trp = padded(tr)                       # keep the buffer alive across the call
    R.ref_dense(P(trp), K, N, P(W))
    save("dense_256x256.npz", seed=np.uint64(seed), K=K, N=N, trellis_sha256=sha(tr), W=W.astype(np.float16))

    # single experts at the benchmark shape
    H, I = 4096, 2048
    layer_seed = 1000
    rng = np.random.default_rng(77)
    rec = {"H": H, "I": I, "layer_seed": layer_seed}
    for j, e in enumerate((3, 201)):
        tg, tu, td = O.synth_expert_trellis(layer_seed, e, H, I)
        sg = np.where(rng.integers(0, 2, H) == 0, -1.0, 1.0).astype(np.float16)
        vg = np.abs(rng.normal(0, 0.02, I)).astype(np.float16)
        su = np.where(rng.integers(0, 2, H) == 0, -1.0, 1.0).astype(np.float16)
        vu = np.abs(rng.normal(0, 0.02, I)).astype(np.float16)
        sd = np.where(rng.integers(0, 2, I) == 0, -1.0, 1.0).astype(np.float16)
        vd = np.abs(rng.normal(0, 0.02, H)).astype(np.float16)
        x = rng.normal(0, 1, H).astype(np.float16).astype(np.float32)
        scales = [a.view(np.uint16) for a in (sg, vg, su, vu, sd, vd)]
        mats = [padded(m) for m in (tg, tu, td)]   # keep the buffers alive across the calls
        for lim in (10.0, 0.0):
            y = np.empty(H, np.float32)
            R.ref_expert_fwd(P(mats[0]), P(mats[1]), P(mats[2]), *[P(s) for s in scales], H, I,
                             ctypes.c_float(lim), P(x), P(y))
            rec[f"y{j}_lim{int(lim)}"] = y
        rec[f"e{j}"] = e
        rec[f"x{j}"] = x
        for name, a in zip(("suh_g", "svh_g", "suh_u", "svh_u", "suh_d", "svh_d"), (sg, vg, su, vu, sd, vd)):
            rec[f"{name}{j}"] = a
        rec[f"trellis_sha256_{j}"] = sha(np.concatenate([tg.ravel(), tu.ravel(), td.ravel()]))
    save("expert_4096x2048.npz", **rec)

    # CPU tier MoE forward, 4 tokens over 6 experts
    E = 6
    tiers = [O.synth_expert_trellis(2000, e, H, I) for e in range(E)]
    bufs = [[padded(m) for m in t] for t in tiers]
    ptrs = np.array([[b[0].ctypes.data, b[1].ctypes.data, b[2].ctypes.data] for b in bufs], dtype=np.int64)
    rng = np.random.default_rng(99)
    sc = {"suh_g": np.where(rng.integers(0, 2, (E, H)) == 0, -1.0, 1.0), "svh_g": np.abs(rng.normal(0, 0.02, (E, I))),
          "suh_u": np.where(rng.integers(0, 2, (E, H)) == 0, -1.0, 1.0), "svh_u": np.abs(rng.normal(0, 0.02, (E, I))),
          "suh_d": np.where(rng.integers(0, 2, (E, I)) == 0, -1.0, 1.0), "svh_d": np.abs(rng.normal(0, 0.02, (E, H)))}
    sc = {k: v.astype(np.float16) for k, v in sc.items()}
    cpus = (ctypes.c_int * 4)(0, 1, 2, 3)
    R.ref_pool_start(4, cpus, 4)
    R.ref_set_limit(ctypes.c_float(10.0))
    sc16 = [sc[k].view(np.uint16) for k in ("suh_g", "svh_g", "suh_u", "svh_u", "suh_d", "svh_d")]
    R.ref_add_layer(0, E, H, I, P(ptrs), *[P(a) for a in sc16])
    T = 4
    x = (rng.normal(0, 1, (T, H))).astype(np.float16).astype(np.float32)
    tok = np.array([0, 0, 0, 1, 1, 2, 2, 2, 3, 3, 3, 3], dtype=np.int32)
    exp = np.array([0, 2, 5, 2, 3, 0, 1, 5, 0, 2, 3, 4], dtype=np.int32)
    wts = rng.uniform(0.05, 0.5, tok.size).astype(np.float32)
    rec = {"H": H, "I": I, "E": E, "layer_seed": 2000, "x": x, "tok": tok, "exp": exp, "w": wts, **sc}
    for mode in (0, 1, 2):
        out = np.zeros((T, H), np.float32)
        md = R.ref_moe_forward(0, P(x), T, P(tok), P(exp), P(wts), tok.size, P(out), mode)
        assert md == mode
        rec[f"out_mode{mode}"] = out
    save("tier_t4.npz", **rec)
    print("golden vectors checked" if check else f"golden vectors written to {OUT}")


if __name__ == "__main__":
    main()
