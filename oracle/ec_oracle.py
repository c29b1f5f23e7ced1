"""CPU ORACLE of the expert cache's replanning -- TEST INFRASTRUCTURE ONLY (imported by tests/ only).

Restates ct/ct_vllm.py:283-427 (ec_step's planning part, ec_release, ec_rewarm) on plain Python lists, as a
sequence of explicit passes over every (layer, expert) pair, without the product's data structures:

  step(counts)   ct/ct_vllm.py:336-391   decay + add counts (float64), top-N wanted set (scores > 0), admits in
                                         descending score (at most ADMIT), victims in ascending score (ties in
                                         residency order), free slots popped from the end of the list, eviction
                                         only when the newcomer's score exceeds HYST x the victim's
  release()      ct/ct_vllm.py:394-416   the resident set kept in residency order, every slot given back
  rewarm(N)      ct/ct_vllm.py:419-436   kept set re-admitted in descending score (ties in residency order) onto
                                         a fresh slot list

Ties in score (which the reference leaves to torch.topk and to set iteration order) are broken here toward the
lower flat index (layer * E + expert); the tests use tie-free scores. The planner is pinned by invariants that do
not restate it (tests/test_ec.py): the resident set is a subset of the top-N scores, at most ADMIT admits per
replan, LIFO slot order on known-answer sequences, no eviction below the hysteresis ratio, every slot owned by at
most one pair.
"""


class ECOracle:
    def __init__(self, L, E, N, admit=48, decay=0.9, hyst=1.0):
        self.L, self.E, self.N = L, E, N
        self.admit, self.decay, self.hyst = admit, decay, hyst
        self.score = [0.0] * (L * E)
        self.resident = []          # [(flat index, slot)] in residency order
        self.free = list(range(N))
        self.admits = self.evicts = self.replans = 0
        self.keep = []

    def _slot_of(self, i):
        for j, s in self.resident:
            if j == i:
                return s
        return None

    def step(self, counts):
        """counts: L x E nested lists / array of routed counts since the last replan. Returns (evicted, admitted)
        as lists of (flat index, slot) in the order they happen; None when the counts are all zero."""
        flat_counts = [float(counts[li][e]) for li in range(self.L) for e in range(self.E)]
        if sum(flat_counts) == 0:
            return None
        self.score = [s * self.decay + c for s, c in zip(self.score, flat_counts)]
        ranked = sorted(range(self.L * self.E), key=lambda i: (-self.score[i], i))
        want = [i for i in ranked[: self.N] if self.score[i] > 0]
        candidates = [i for i in want if self._slot_of(i) is None]
        candidates.sort(key=lambda i: (-self.score[i], i))
        candidates = candidates[: self.admit]
        if not candidates:
            return [], []
        victims = [i for i, _ in self.resident if i not in want]
        victims.sort(key=lambda i: self.score[i])          # stable: residency order among equal scores
        evicted, admitted = [], []
        for i in candidates:
            if self.free:
                s = self.free[-1]
                self.free = self.free[:-1]
            elif victims and self.score[i] > self.hyst * self.score[victims[0]]:
                v = victims[0]
                victims = victims[1:]
                s = self._slot_of(v)
                self.resident = [(j, t) for j, t in self.resident if j != v]
                self.evicts += 1
                evicted.append((v, s))
            else:
                break
            self.resident.append((i, s))
            self.admits += 1
            admitted.append((i, s))
        self.replans += 1
        return evicted, admitted

    def release(self):
        self.keep = [i for i, _ in self.resident]
        self.resident = []
        self.free = []
        self.N = 0

    def rewarm(self, N):
        self.N = N
        self.free = list(range(N))
        # descending score; equal scores keep their residency order (the reference's stable sort of the kept
        # list, ct/ct_vllm.py:421)
        keep = sorted(self.keep, key=lambda i: -self.score[i])[:N]
        admitted = []
        for i in keep:
            s = self.free[-1]
            self.free = self.free[:-1]
            self.resident.append((i, s))
            admitted.append((i, s))
        return admitted
