"""Expert-cache replanning (ct/ct_vllm.py:283-436): the oracle pinned by invariants and known-answer sequences,
then the product's planner (mi355moe.cache.ExpertCache.plan) against the oracle, step by step."""
import numpy as np
import pytest

from ec_oracle import ECOracle


def _counts(rng, L, E, scale=5.0):
    # continuous-looking counts: distinct decayed sums stay tie-free (ties are broken by index in both)
    return rng.poisson(rng.gamma(0.3, scale, (L, E)))


def _check_invariants(o, ev, ad, before_resident):
    flat = o.score
    res = [i for i, _ in o.resident]
    slots = [s for _, s in o.resident]
    assert len(set(slots)) == len(slots)                       # one pair per slot
    assert len(set(res)) == len(res)
    assert len(ad) <= o.admit                                  # at most ADMIT newcomers per replan
    assert len(res) <= o.N
    assert set(slots).isdisjoint(o.free)
    assert sorted(slots + o.free) == list(range(o.N))          # every slot either owned or free
    ranked = sorted(range(len(flat)), key=lambda i: (-flat[i], i))
    topn = set(i for i in ranked[: o.N] if flat[i] > 0)
    newly = set(i for i, _ in ad)
    assert newly <= topn                                       # only wanted pairs are admitted
    for v, _ in ev:                                            # only unwanted pairs are evicted
        assert v not in topn and v in before_resident
    # hysteresis: every eviction pairs a newcomer whose score exceeds hyst x the victim's
    adm_after_free = [i for i, _ in ad][len(ad) - len(ev):]
    for (v, _), i in zip(ev, adm_after_free):
        assert flat[i] > o.hyst * flat[v]
    # admits come in descending score
    sc = [flat[i] for i, _ in ad]
    assert all(a >= b for a, b in zip(sc, sc[1:]))


def test_oracle_known_answer_lifo_and_admit_cap():
    """L=1, E=6, N=3, ADMIT=2: hand-computed sequence."""
    o = ECOracle(1, 6, 3, admit=2, decay=0.5, hyst=1.0)
    # step 1: scores = counts; wanted top-3 = {5, 2, 0}; admit cap 2 -> 5 (slot 2), 2 (slot 1) (free popped from end)
    ev, ad = o.step([[3, 0, 7, 0, 0, 9]])
    assert ev == [] and ad == [(5, 2), (2, 1)]
    # step 2: scores 1.5, 0, 3.5, 0, 4, 4.5 -> top-3 = {5, 4, 2}; newcomer 4 takes the last free slot 0
    ev, ad = o.step([[0, 0, 0, 0, 4, 0]])
    assert ev == [] and ad == [(4, 0)]
    # step 3: scores 0.75, 6, 1.75, 0, 2, 2.25 -> top-3 = {1, 5, 4}; victim 2 (1.75 < 6) evicted, 1 takes slot 1
    ev, ad = o.step([[0, 6, 0, 0, 0, 0]])
    assert ev == [(2, 1)] and ad == [(1, 1)]
    # step 4: zero counts: no replan, no decay
    assert o.step([[0] * 6]) is None
    assert o.replans == 3 and o.admits == 4 and o.evicts == 1


def test_oracle_hysteresis_blocks_eviction():
    o = ECOracle(1, 4, 1, admit=4, decay=1.0, hyst=2.0)
    assert o.step([[5, 0, 0, 0]]) == ([], [(0, 0)])
    # expert 1 overtakes (6 > 5) but not by the hysteresis factor (6 <= 2 x 5): nothing moves
    assert o.step([[0, 6, 0, 0]]) == ([], [])
    assert o.resident == [(0, 0)]
    # 11 > 2 x 5: evicted
    assert o.step([[0, 5, 0, 0]]) == ([(0, 0)], [(1, 0)])


def test_oracle_release_rewarm_keeps_order():
    o = ECOracle(2, 4, 3, admit=8, decay=0.9, hyst=1.0)
    o.step([[1, 0, 4, 0], [0, 9, 0, 2]])
    kept = [i for i, _ in o.resident]
    o.release()
    assert o.resident == [] and o.free == [] and o.keep == kept
    ad = o.rewarm(2)
    assert [i for i, _ in ad] == sorted(kept, key=lambda i: -o.score[i])[:2]
    assert [s for _, s in ad] == [1, 0]


@pytest.mark.parametrize("seed,L,E,N,admit,hyst", [(1, 3, 20, 12, 4, 1.0), (2, 2, 30, 40, 48, 1.0),
                                                   (3, 4, 16, 9, 3, 1.5), (4, 1, 64, 5, 2, 1.0)])
def test_oracle_invariants_random(seed, L, E, N, admit, hyst):
    rng = np.random.default_rng(seed)
    o = ECOracle(L, E, N, admit=admit, decay=0.9, hyst=hyst)
    for _ in range(40):
        before = set(i for i, _ in o.resident)
        r = o.step(_counts(rng, L, E))
        if r is None:
            continue
        _check_invariants(o, r[0], r[1], before)


class _Layer:
    def __init__(self, E):
        self.E = E


@pytest.mark.parametrize("seed,L,E,N,admit,hyst", [(11, 3, 20, 12, 4, 1.0), (12, 2, 30, 40, 48, 1.0),
                                                   (13, 4, 16, 9, 3, 1.5), (14, 40, 384, 709, 48, 1.0)])
def test_planner_matches_oracle(seed, L, E, N, admit, hyst):
    """The product's planner gives the oracle's evictions, admissions and slot numbers at every replan."""
    from mi355moe.cache import ExpertCache
    rng = np.random.default_rng(seed)
    o = ECOracle(L, E, N, admit=admit, decay=0.9, hyst=hyst)
    c = ExpertCache([_Layer(E)] * L, admit=admit, decay=0.9, hyst=hyst)
    c.N, c.owner, c.free = N, [None] * N, list(range(N))
    steps = 25 if L * E > 5000 else 60
    for _ in range(steps):
        cnt = _counts(rng, L, E)
        a = o.step(cnt)
        b = c.plan(cnt)
        assert a == (None if b is None else (list(b[0]), list(b[1])))
        assert [(i, s) for i, s in c.where.items()] == o.resident
        assert c.free == o.free
        assert np.array_equal(c.score.reshape(-1), np.array(o.score))
    assert (c.admits, c.evicts, c.replans) == (o.admits, o.evicts, o.replans)
