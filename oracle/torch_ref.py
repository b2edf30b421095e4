"""Literal torch-CPU restatements of the reference's hot path.

These follow the reference's own torch formulation line by line (with the
CUDA guards dropped and Triton kernels written as torch ops), so they can run
in a CPU-only process. They serve two purposes:

1. The CPU baseline timed by bench.py (the reference itself is CUDA-only and
   cannot run here).
2. Pinning the declared arithmetic of ``oracle.sampling``: on seeded inputs
   the two must agree on probabilities within 1e-6 relative and on every
   cutoff/token except boundary-ambiguous draws (tests/test_oracle_sampling.py).
"""

from __future__ import annotations

import torch

from . import greedy as _greedy


# ---------------------------------------------------------------------------
# Greedy (sglang_recurrent/loopspec/decisions.py:99-184)
# ---------------------------------------------------------------------------

def greedy_queue(logits: torch.Tensor) -> torch.Tensor:
    """GreedyDecisionPolicy.queue: argmax over every endpoint row (decisions.py:116)."""
    return torch.argmax(logits, dim=-1, keepdim=True)


def greedy_verify_step(target_logits: torch.Tensor, draft_logits: torch.Tensor) -> tuple[int, list[int]]:
    """One batch-1 greedy verify step as the reference performs it.

    The q1 (draft) and final (target) endpoint rows are argmax'd together in
    one call (decisions.py:99-117), read back with tolist() (decisions.py:80-89)
    and resolved per row on the CPU (decisions.py:136-184) along the accept
    prefix. target_logits [k+1, V], draft_logits [k, V].
    Returns (accept_len, emitted tokens).
    """
    k = draft_logits.shape[0]
    rows = torch.cat([draft_logits, target_logits])
    choices = [row[0] for row in greedy_queue(rows).tolist()]
    drafts, finals = choices[:k], choices[k:]
    emitted = []
    accepted = 0
    for i in range(k + 1):
        emitted.append(finals[i])
        if i == k:
            break
        code, _, _ = _greedy.resolve_final(finals[i], drafts[i], None)
        if code != 1:
            break
        accepted += 1
    return accepted, emitted
