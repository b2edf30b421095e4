"""Seeded speculation cycles driven through both ownership models (shared by
the CPU and GPU timeline tests): every cycle forks children under some
frontier lanes, decodes every depth of every lane, then retains a random
part of the new frontier; the last cycle retains nothing."""

import random


def cycles(seed: int, n_cycles: int, depths: int = 2, max_children: int = 2):
    rng = random.Random(seed)
    frontier = [(0, 0)]
    next_branch = 1
    for c in range(n_cycles):
        grown = []
        for branch, parent in frontier:
            k = rng.randint(0, max_children)
            if k == 0 and branch != 0:
                grown.append((branch, parent))
            for _ in range(max(k, 1 if branch == 0 else 0)):
                grown.append((next_branch, branch))
                next_branch += 1
        decode = [(d, b, p) for b, p in grown for d in range(depths)]
        last = c == n_cycles - 1
        keep = [] if last else rng.sample(grown, rng.randint(1, len(grown)))
        yield decode, keep
        frontier = keep
