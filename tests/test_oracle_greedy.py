"""CPU checks that pin the greedy oracle (no GPU)."""

import itertools
import math

import numpy as np
import pytest
import torch

from oracle import greedy, torch_ref
from loopspec_amd import workloads


def brute_argmax(row):
    """Pure-Python torch.argmax rule: first NaN, else first index of the max."""
    best = None
    for i, x in enumerate(row):
        if math.isnan(x):
            return i
        if best is None or x > row[best]:
            best = i
    return best


@pytest.mark.parametrize("seed", range(5))
def test_argmax_matches_bruteforce_with_ties(seed):
    rng = np.random.default_rng(seed)
    x = rng.integers(-5, 6, size=(40, 37)).astype(np.float32)  # many exact ties
    x[3, 7] = np.nan
    x[3, 20] = np.nan
    x[5] = -0.0
    x[5, 9] = 0.0
    x[6] = -np.inf
    got = greedy.argmax_first(x)
    want = [brute_argmax(list(r)) for r in x.tolist()]
    assert got.tolist() == want
    assert got[3] == 7 and got[5] == 0 and got[6] == 0


def test_argmax_agrees_with_torch_argmax():
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(64, 4096, generator=g) * 3).to(torch.bfloat16)  # natural bf16 ties
    x[0, 100] = float("nan")
    want = torch.argmax(x.float(), dim=-1)
    got = greedy.argmax_first(x.float().numpy())
    assert np.array_equal(got, want.numpy())


def test_resolve_final_rules():
    # decisions.py:163-170
    assert greedy.resolve_final(5, None, None) == (0, False, False)
    assert greedy.resolve_final(5, 5, None) == (1, False, False)
    assert greedy.resolve_final(5, 4, None) == (0, True, False)
    assert greedy.resolve_final(5, 4, 5) == (2, True, False)
    assert greedy.resolve_final(5, 4, 6) == (0, True, True)
    assert greedy.resolve_final(0, 0, None) == (1, False, False)  # token id 0 is a valid proposal


@pytest.mark.parametrize("k", [1, 2, 3, 4])
def test_chain_exhaustive_patterns(k):
    """Every (match/mismatch)^k pattern: accept length = leading matches."""
    for pattern in itertools.product([True, False], repeat=k):
        t = np.arange(10, 10 + k + 1, dtype=np.int64)[None]
        d = np.array([[t[0, i] if m else t[0, i] + 100 for i, m in enumerate(pattern)]], dtype=np.int64)
        acc, tok = greedy.greedy_chain(t, d)
        lead = next((i for i, m in enumerate(pattern) if not m), k)
        assert acc[0] == lead
        assert tok[0, : lead + 1].tolist() == t[0, : lead + 1].tolist()
        assert (tok[0, lead + 1:] == -1).all()


def test_torch_ref_step_matches_oracle_c1():
    cfg = workloads.C1
    for seed in range(3):
        target, draft = workloads.greedy_inputs(cfg, seed)
        acc, tok, _ = greedy.greedy_verify(target.numpy(), draft.numpy())
        a2, emitted = torch_ref.greedy_verify_step(target[0], draft[0])
        assert a2 == acc[0]
        assert emitted == tok[0, : a2 + 1].tolist()


def test_c2_inputs_acceptance_and_ties():
    cfg = workloads.GreedyConfig("small", 64, 2, 4096, torch.bfloat16, tie_frac=0.2)
    target, draft = workloads.greedy_inputs(cfg, 1)
    acc, tok, rows = greedy.greedy_verify(target.float().numpy(), draft.float().numpy())
    assert target.shape == (64, 3, 4096) and draft.shape == (64, 2, 4096)
    # planted ties exist: some row has its max at >= 2 positions
    flat = torch.cat([target.reshape(-1, 4096), draft.reshape(-1, 4096)]).float()
    counts = (flat == flat.max(dim=-1, keepdim=True).values).sum(-1)
    assert (counts >= 2).sum() >= 10
    assert 0 <= acc.mean() <= 2
