"""Busy experts of one staged batch through the fat-expert GEMM (the reference's runtime/dma_gemm.py:5-26).

run_batch(D, st, batch, inners, counts, cap, x, token_sorted, weight_sorted, limit, out, apply_fat, use_kernel):
the experts of staging batch `batch` (D["batches"][batch] = (first, last) into D["cold"], the host-resident
experts in staging order) with more than `cap` routes run from staging slot batch % NS, row = their index in
the batch: their matrices in a copy of `inners` point at the slot's rows, every other expert is skipped, and
apply_fat (exl3.apply_exl3_batched_fat) accumulates them into `out`. `st` is the device's staging state
(exl3._DMA_STATE[device]: "slots" SlotPool of NS x B rows).
"""
from copy import copy


def run_batch(D, st, batch, inners, counts, cap, x, token_sorted, weight_sorted, limit, out, apply_fat, use_kernel):
    first, last = D["batches"][batch]
    cold = D["cold"] if "cold" in D else D["h13"].cold
    experts = cold[first:last]
    busy = {e for e in experts if counts[e] > cap}
    if not busy:
        return
    pool = st["slots"]
    B = pool.n // len(st["free"])
    slot = batch % len(st["free"])
    staged = list(inners)
    for row, e in enumerate(experts):
        if e not in busy:
            continue
        entry = dict(inners[e])
        for key, addr in zip(("gate", "up", "down"), pool.addrs(slot * B + row)):
            m = copy(entry[key])
            m.trellis = addr
            entry[key] = m
        staged[e] = entry
    apply_fat(x, token_sorted, weight_sorted, counts, staged, limit, cap, out, use_kernel=use_kernel,
              skip=set(range(len(inners))) - busy)
