"""The host expert tier on the CPU (no GPU): its AVX-512 expert kernel against the oracle and the reference's
golden outputs, and the mailbox served by its worker thread, driven from the host the way the split kernel drives
it (the reference's no-GPU repro pattern, experimental/b70-tier/repro/rep_ct.py:104-163)."""
import os
import time

import numpy as np
import pytest

import oracle as O


def _avx512():
    try:
        flags = open("/proc/cpuinfo").read()
    except OSError:
        return False
    return all(f in flags for f in ("avx512f", "avx512bw", "avx512vl", "avx512_vbmi2", "avx512_vnni", "f16c", "fma"))


pytestmark = pytest.mark.skipif(not _avx512(), reason="the host tier needs an AVX-512 (VBMI2, VNNI) host")


@pytest.fixture
def tier():
    from mi355moe import tier as T
    yield T
    T.shutdown()


def _layer(seed, E, H, I):
    """Synthetic experts of one layer in host memory: tiles as the trellis words, scales from the store's
    generator. Returns (ptrs int64 [E, 3], scales dict, keep-alive list)."""
    from mi355moe.store import synth_scales
    sc = synth_scales(seed, E, H, I)
    keep, ptrs = [], np.zeros((E, 3), np.int64)
    for e in range(E):
        mats = [np.ascontiguousarray(m) for m in O.synth_expert_trellis(seed, e, H, I)]
        keep.append(mats)
        ptrs[e] = [m.ctypes.data for m in mats]
    scales = {"suh_g": sc["w13_suh"][:, 0], "svh_g": sc["w13_svh"][:, 0], "suh_u": sc["w13_suh"][:, 1],
              "svh_u": sc["w13_svh"][:, 1], "suh_d": sc["w2_suh"], "svh_d": sc["w2_svh"]}
    return ptrs, scales, keep


def _oracle(seed, scales, x, sel, w, H, I, limit):
    out = np.zeros((x.shape[0], H), np.float64)
    for e in np.unique(sel[sel >= 0]):
        tr = O.synth_expert_trellis(seed, int(e), H, I)
        DE = O.DenseExpert(*tr, *[scales[k][e] for k in ("suh_g", "svh_g", "suh_u", "svh_u", "suh_d", "svh_d")], H, I)
        tt, jj = np.nonzero(sel == e)
        for row, t, j in zip(DE(x[tt], limit), tt, jj):
            out[t] += np.float64(w[t, j]) * row
    return out


@pytest.mark.parametrize("mode", [1, 0, 2])
@pytest.mark.parametrize("H,I,E,T,k", [(512, 256, 6, 5, 3), (1024, 384, 9, 9, 4)])
def test_forward_matches_oracle(tier, mode, H, I, E, T, k):
    """EXACT (mode 1), AFFINE (mode 0) and I16 (mode 2) against the oracle's EXACT expert; groups of 1 to 9 tokens
    per expert (GEMV passes of 3), masked picks, clamp on."""
    seed = 900 + H
    ptrs, sc, keep = _layer(seed, E, H, I)
    tier.init(H, I, 1, threads=4, cpus=sorted(os.sched_getaffinity(0))[:4])
    tier.set_limit(10.0)
    tier.add_layer(0, ptrs=ptrs, scales=sc)
    rng = np.random.default_rng(H + T)
    sel = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    sel[1, 0] = -1
    w = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
    x = rng.normal(0, 1, (T, H)).astype(np.float16).astype(np.float32)
    got = tier.forward(0, x, sel, w, mode)
    ref = _oracle(seed, sc, x, sel, w, H, I, 10.0)
    mx, mean = O.tolerance_metrics(got, ref)
    print(f"mode {mode} H={H}: {mx:.2e} {mean:.2e}")
    assert mx <= 2e-2 and mean <= 2e-3, (mx, mean)


def test_forward_matches_reference_golden_expert(tier):
    """The reference's own EXACT expert (compiled ref_expert) on its golden inputs, limits 10 and 0."""
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "expert_4096x2048.npz"))
    H, I = int(g["H"]), int(g["I"])
    tier.init(H, I, 2, threads=8, cpus=sorted(os.sched_getaffinity(0))[:8])
    keep = []
    for j in (0, 1):
        mats = [np.ascontiguousarray(m) for m in O.synth_expert_trellis(int(g["layer_seed"]), int(g[f"e{j}"]), H, I)]
        keep.append(mats)
        sc = {k: g[f"{k}{j}"][None] for k in ("suh_g", "svh_g", "suh_u", "svh_u", "suh_d", "svh_d")}
        tier.add_layer(j, ptrs=np.array([[m.ctypes.data for m in mats]], np.int64), scales=sc)
    for j in (0, 1):
        for lim in (10.0, 0.0):
            tier.set_limit(lim)
            for mode in (1, 0):
                got = tier.forward(j, g[f"x{j}"][None], np.zeros((1, 1), np.int32), np.ones((1, 1), np.float32), mode)
                mx, mean = O.tolerance_metrics(got[0], g[f"y{j}_lim{int(lim)}"].astype(np.float64))
                assert mx <= 2e-2 and mean <= 2e-3, (j, lim, mode, mx, mean)


def test_forward_matches_reference_tier_modes(tier):
    """The reference's CPU tier on a T=4 layer (6 experts, 12 picks): EXACT against its EXACT output, AFFINE
    against its AFFINE output, I16 against its I16 output, each within the parity tolerance (I16's int16 inputs
    and block scales follow the reference's quantisation, so I16 is closer to the reference's I16 output than to
    its AFFINE output)."""
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "tier_t4.npz"))
    H, I, E = int(g["H"]), int(g["I"]), int(g["E"])
    seed = int(g["layer_seed"])
    keep, ptrs = [], np.zeros((E, 3), np.int64)
    for e in range(E):
        mats = [np.ascontiguousarray(m) for m in O.synth_expert_trellis(seed, e, H, I)]
        keep.append(mats)
        ptrs[e] = [m.ctypes.data for m in mats]
    tier.init(H, I, 1, threads=8, cpus=sorted(os.sched_getaffinity(0))[:8])
    tier.set_limit(10.0)
    tier.add_layer(0, ptrs=ptrs, scales={k: g[k] for k in ("suh_g", "svh_g", "suh_u", "svh_u", "suh_d", "svh_d")})
    T = g["x"].shape[0]
    k = int(np.bincount(g["tok"], minlength=T).max())
    sel = np.full((T, k), -1, np.int32)
    w = np.zeros((T, k), np.float32)
    fill = np.zeros(T, int)
    for t, e, wt in zip(g["tok"], g["exp"], g["w"]):
        sel[t, fill[t]], w[t, fill[t]] = e, wt
        fill[t] += 1
    for mode in (1, 0, 2):
        got = tier.forward(0, g["x"], sel, w, mode)
        mx, mean = O.tolerance_metrics(got, g[f"out_mode{mode}"].astype(np.float64))
        print(f"mode {mode} vs the reference tier: {mx:.2e} {mean:.2e}")
        assert mx <= 2e-2 and mean <= 2e-3, (mode, mx, mean)
        if mode == 2:
            _, m0 = O.tolerance_metrics(got, g["out_mode0"].astype(np.float64))
            print(f"mode 2 vs the reference tier's AFFINE output: {m0:.2e}")
            assert mean < m0, (mean, m0)


def test_mailbox_worker_serves_jobs(tier):
    """The worker thread serves jobs published in the split's mailbox layout and answers with the done word; the
    partial equals the synchronous forward bit for bit; an empty job zeroes the partial; picks whose expert or
    token is out of range are left out; forward is refused while the worker runs."""
    H, I, E, T, k = 512, 256, 8, 4, 3
    seed = 4711
    ptrs, sc, keep = _layer(seed, E, H, I)
    ctrl = np.zeros(16, np.int64)
    hx = np.zeros((T, H), np.float16)
    picks = np.zeros((T * k + 3, 3), np.int32)
    hout = np.full((T, H), np.nan, np.float32)
    mb = {k_: a.ctypes.data for k_, a in (("ctrl", ctrl), ("hx", hx), ("picks", picks), ("hout", hout))}
    mb.update(maxtok=T, maxpicks=picks.shape[0])
    tier.init(H, I, 2, mailbox=mb, threads=3, cpus=sorted(os.sched_getaffinity(0))[:3], mode=0)
    tier.set_limit(10.0)
    tier.add_layer(1, ptrs=ptrs, scales=sc)
    rng = np.random.default_rng(2)
    sel = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    w = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
    x16 = rng.normal(0, 1, (T, H)).astype(np.float16)
    want = tier.forward(1, x16.astype(np.float32), sel, w, 0)
    tier.start(-1)
    with pytest.raises(RuntimeError):
        tier.forward(1, x16.astype(np.float32), sel, w, 0)

    def job(seq, npk):
        ctrl[2], ctrl[3], ctrl[4] = 1, T, npk
        ctrl[0] = seq                      # the payload is written first; x86 keeps stores in order
        t0 = time.time()
        while ctrl[1] != seq:
            assert time.time() - t0 < 20, "the worker did not answer"
            time.sleep(1e-4)

    hx[:] = x16
    flat = [(t, int(sel[t, j]), w[t, j]) for t in range(T) for j in range(k)]
    for p, (t, e, wt) in enumerate(flat):
        picks[p] = (t, e, np.float32(wt).view(np.int32))
    job(1, len(flat))
    assert np.array_equal(hout, want)
    job(2, 0)
    assert np.count_nonzero(hout) == 0
    s = tier.stats()
    assert s["jobs"] == 2 and s["picks"] == len(flat) and s["empty"] == 1 and s["tokens"] == 2 * T
    # a malformed job: an expert past E, a negative expert and a token past the job's rows among the valid picks
    bad = [(0, E, 1.0), (1, -1, 1.0), (T, int(sel[0, 0]), 1.0)]
    rows = flat[:5] + bad + flat[5:]
    for p, (t, e, wt) in enumerate(rows):
        picks[p] = (t, e, np.float32(wt).view(np.int32))
    job(3, len(rows))
    assert np.array_equal(hout, want)
    # jobs larger than the mailbox (tokens, then picks) and one naming a layer never added: answered, not
    # computed, the hout rows zeroed, counted as rejected
    for seq, (li, bsz, npk) in enumerate(((1, T + 1, 4), (1, T, picks.shape[0] + 1), (0, T, 4)), start=4):
        hout[:] = 1.0
        ctrl[2], ctrl[3], ctrl[4] = li, bsz, npk
        ctrl[0] = seq
        t0 = time.time()
        while ctrl[1] != seq:
            assert time.time() - t0 < 20, "the worker did not answer"
            time.sleep(1e-4)
        assert np.count_nonzero(hout) == 0
    s = tier.stats()
    assert s["jobs"] == 6 and s["rejected"] == 3 and s["stale"] == 0
    tier.stop()


def test_tier_holds_the_memory_its_workers_read(tier):
    """The mailbox's owner is held while the tier is up (HostBuffer.free refuses it) and released by shutdown."""
    from mi355moe.hostmem import HostBuffer
    owner = object.__new__(HostBuffer)        # the bookkeeping only: no pinned allocation on a CPU-only host
    owner.holders, owner.ptr, owner.nbytes = 0, None, 0
    H, I, T = 512, 256, 2
    ctrl = np.zeros(16, np.int64)
    hx = np.zeros((T, H), np.float16)
    picks = np.zeros((8, 3), np.int32)
    hout = np.zeros((T, H), np.float32)
    mb = {k_: a.ctypes.data for k_, a in (("ctrl", ctrl), ("hx", hx), ("picks", picks), ("hout", hout))}
    mb.update(maxtok=T, maxpicks=8, owner=owner)
    tier.init(H, I, 1, mailbox=mb, threads=2, cpus=sorted(os.sched_getaffinity(0))[:2])
    assert owner.holders == 1
    with pytest.raises(RuntimeError):
        owner.free()
    tier.shutdown()
    assert owner.holders == 0
    owner.free()                              # nothing allocated: a no-op once released


def test_mailbox_needs_its_capacity(tier):
    from mi355moe import _lib  # noqa: F401  (the library loads)
    ctrl = np.zeros(16, np.int64)
    buf = np.zeros(4096, np.float32)
    mb = {"ctrl": ctrl.ctypes.data, "hx": buf.ctypes.data, "picks": buf.ctypes.data, "hout": buf.ctypes.data}
    with pytest.raises(RuntimeError, match="capacities"):
        tier.init(512, 256, 1, mailbox=mb, threads=1, cpus=[])


@pytest.mark.parametrize("mode", [1, 0])
def test_many_rows_per_expert_bitwise_equal_to_single_rows(tier, mode):
    """Experts with many rows (a prefill tail job: 40 tokens over 6 experts, every expert 20-40 rows) take the
    chunked GEMV that decodes each weight once for all rows; every output equals the same token computed alone
    (the per-token path) bit for bit, in EXACT and in AFFINE mode."""
    H, I, E, T, k = 512, 256, 6, 40, 4
    seed = 99
    ptrs, sc, keep = _layer(seed, E, H, I)
    tier.init(H, I, 1, threads=4, cpus=sorted(os.sched_getaffinity(0))[:4])
    tier.set_limit(10.0)
    tier.add_layer(0, ptrs=ptrs, scales=sc)
    rng = np.random.default_rng(5)
    sel = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    w = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
    x = rng.normal(0, 1, (T, H)).astype(np.float16).astype(np.float32)
    got = tier.forward(0, x, sel, w, mode)
    for t in range(T):
        one = tier.forward(0, x[t:t + 1], sel[t:t + 1], w[t:t + 1], mode)
        assert np.array_equal(got[t], one[0]), t
    ref = _oracle(seed, sc, x, sel, w, H, I, 10.0)
    mx, mean = O.tolerance_metrics(got, ref)
    assert mx <= 2e-2 and mean <= 2e-3, (mx, mean)


def test_automatic_mode_selection(tier):
    """The automatic mode (the reference's ft_tier_ext.cpp:130-132): a job whose experts have at most two rows each
    is computed in I16 (bit for bit equal to mode 2), a job with an expert of three rows in AFFINE (mode 0)."""
    H, I, E = 512, 256, 8
    seed = 321
    ptrs, sc, keep = _layer(seed, E, H, I)
    tier.init(H, I, 1, threads=4, cpus=sorted(os.sched_getaffinity(0))[:4])
    tier.set_limit(10.0)
    tier.add_layer(0, ptrs=ptrs, scales=sc)
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (3, H)).astype(np.float16).astype(np.float32)
    w = rng.uniform(0.1, 1.0, (3, 2)).astype(np.float32)
    two = np.array([[0, 1], [1, 2], [3, 4]], np.int32)           # expert 1 has two rows
    three = np.array([[0, 1], [1, 2], [1, 4]], np.int32)         # expert 1 has three rows
    assert np.array_equal(tier.forward(0, x, two, w, -1), tier.forward(0, x, two, w, 2))
    assert np.array_equal(tier.forward(0, x, three, w, -1), tier.forward(0, x, three, w, 0))
    assert not np.array_equal(tier.forward(0, x, two, w, 2), tier.forward(0, x, two, w, 0))
