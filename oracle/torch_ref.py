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


# ---------------------------------------------------------------------------
# Sampling (sglang_recurrent/loopspec/sampling/*.py), CPU tensors
# ---------------------------------------------------------------------------

CHUNK = 2048  # sampler.py:494


def filtered_probabilities(logits: torch.Tensor, temperature: float, top_k: int, top_p: float,
                           top_p_thresholds: torch.Tensor | None = None) -> torch.Tensor:
    """distributions.py:14-86 with the CUDA guard dropped (top-k-only path omitted)."""
    vocabulary_size = logits.shape[-1]
    effective_top_k = 0 if top_k >= vocabulary_size else top_k
    probs = (
        torch.softmax(logits, dim=-1, dtype=torch.float32)
        if temperature == 1
        else torch.softmax(logits.float() / temperature, dim=-1)
    )
    if effective_top_k == 0 and top_p == 1:
        return probs
    sorted_probs = probs.sort(dim=-1, descending=True).values
    cumulative = sorted_probs.cumsum(dim=-1)
    thresholds = (
        torch.full((logits.shape[0], 1), top_p, dtype=torch.float32)
        if top_p_thresholds is None else top_p_thresholds[: logits.shape[0]]
    )
    cutoff_indices = torch.searchsorted(cumulative, thresholds, right=False).clamp_max_(vocabulary_size - 1)
    cutoffs = sorted_probs.gather(-1, cutoff_indices)
    if effective_top_k:
        if top_p == 1:
            raise NotImplementedError("top-k-only uses sgl_kernel.top_k_renorm_prob (not available)")
        cutoffs = torch.maximum(sorted_probs[:, effective_top_k - 1: effective_top_k], cutoffs)
    filtered = torch.where(probs >= cutoffs, probs, 0)
    return filtered / filtered.sum(dim=-1, keepdim=True)


def top_p_context(logits: torch.Tensor, temperature: float, top_p: float):
    """The (probs, sorted_probs, cutoff_indices) context of distributions.py:120-139."""
    probs = (
        torch.softmax(logits, dim=-1, dtype=torch.float32)
        if temperature == 1
        else torch.softmax(logits.float() / temperature, dim=-1)
    )
    sorted_probs = probs.sort(dim=-1, descending=True).values
    cumulative = sorted_probs.cumsum(dim=-1)
    thresholds = torch.full((logits.shape[0], 1), top_p, dtype=torch.float32)
    cutoff_indices = torch.searchsorted(cumulative, thresholds, right=False).clamp_max_(logits.shape[-1] - 1)
    return probs, sorted_probs, cutoff_indices


def categorical_pick(probs: torch.Tensor, uniforms: torch.Tensor) -> torch.Tensor:
    """_categorical_chunk_sums_kernel + _categorical_pick_kernel (sampler.py:22-102) as torch ops."""
    rows, vocab = probs.shape
    chunks = -(-vocab // CHUNK)
    padded = torch.zeros((rows, chunks * CHUNK), dtype=torch.float32)
    padded[:, :vocab] = probs.float()
    blocks = padded.view(rows, chunks, CHUNK)
    sums = blocks.sum(dim=-1)
    out = torch.zeros(rows, dtype=torch.int64)
    for r in range(rows):
        total = sums[r].sum()
        target = uniforms[r].float() * total
        cdf = sums[r].cumsum(0)
        hit = torch.nonzero(cdf > target)
        chunk = int(hit[0]) if hit.numel() else 0
        preceding = sums[r, :chunk].sum()
        tcdf = blocks[r, chunk].cumsum(0)
        hit = torch.nonzero(tcdf > target - preceding)
        out[r] = chunk * CHUNK + (int(hit[0]) if hit.numel() else 0)
    return out


def verify(target_masses: torch.Tensor, proposal_masses: torch.Tensor, tokens: torch.Tensor,
           uniforms: torch.Tensor) -> torch.Tensor:
    """_verification_decisions_kernel (sampler.py:428-460)."""
    acceptance = torch.minimum(torch.ones_like(target_masses), target_masses / proposal_masses)
    accepted = uniforms < acceptance
    prediction = torch.where(accepted, tokens, torch.full_like(tokens, -1))
    zero = torch.zeros_like(tokens)
    return torch.stack([prediction, zero, accepted.long(), (~accepted).long(), zero], dim=1)


def rejection_run(first: torch.Tensor, target: torch.Tensor, second: torch.Tensor, token: int,
                  has_second: bool, u0: float, u1: float) -> tuple[int, int, int]:
    """RejectionSampler._run (rejection.py:42-97) on [1, V] CPU rows."""
    first, target, second = first.view(1, -1), target.view(1, -1), second.view(1, -1)
    first_delta = (target - first).clamp_min(0)
    first_mass = first_delta.sum(dim=-1, keepdim=True)
    has_first_residual = first_mass > 0
    target_mass = target.sum(dim=-1, keepdim=True)
    normalized_target = target / torch.where(target_mass > 0, target_mass, torch.ones_like(target_mass))
    first_residual = first_delta / torch.where(has_first_residual, first_mass, torch.ones_like(first_mass))
    first_residual = torch.where(has_first_residual, first_residual, normalized_target)
    tok = torch.tensor([token])
    hs = torch.tensor([has_second])
    target_m = first_residual.gather(1, tok.unsqueeze(1)).squeeze(1)
    proposal_m = second.gather(1, tok.unsqueeze(1)).squeeze(1)
    proposal_m = torch.where(hs, proposal_m, torch.ones_like(proposal_m))
    acceptance = torch.minimum(torch.ones_like(target_m), target_m / proposal_m)
    accepted = hs & (torch.tensor([u0]) < acceptance)
    second_delta = (first_residual - second).clamp_min(0)
    second_mass = second_delta.sum(dim=-1, keepdim=True)
    has_second_residual = second_mass > 0
    second_residual = second_delta / torch.where(has_second_residual, second_mass, torch.ones_like(second_mass))
    fallback = torch.where(hs.unsqueeze(1) & has_second_residual, second_residual, first_residual)
    sampled = categorical_pick(fallback, torch.tensor([u1]))
    prediction = torch.where(accepted, tok, sampled)
    return int(prediction[0]), int(accepted[0]), int((hs & ~accepted)[0])


def apply_penalty(rows: torch.Tensor, history: torch.Tensor, penalty: float) -> torch.Tensor:
    """Repetition penalty over a token history: for ids in the history,
    l < 0 ? l * penalty : l / penalty (transformers' closed form,
    generation/logits_process.py:409-412; SGLang's penalizer, which the
    reference's baseline path would use, is not installed)."""
    out = rows.clone()
    ids = torch.unique(history.long())
    sel = out[:, ids]
    out[:, ids] = torch.where(sel < 0, sel * penalty, sel / penalty)
    return out


def speculative_verify(target_logits: torch.Tensor, draft_logits: torch.Tensor, draft_tokens: torch.Tensor,
                       uniforms: torch.Tensor, temperature: float, top_p: float, penalty: float = 1.0,
                       histories=None):
    """Chain-of-k lossless verify built from the reference's own ops.

    Per batch element: filter every endpoint row together (policy.py:228-233),
    verify position by position with the q1 rule (sampler.py:451-452); on the
    first rejection sample the residual fallback (rejection.py:60-69 and the
    sample_with_uniforms callback); if all accept, sample the last target row
    directly (policy.py:156-165). With penalty != 1 the rows of element b are
    penalised over histories[b] first.
    Returns (accept_len int32 [B], tokens int64 [B, k+1]).
    """
    b_n, kp1, vocab = target_logits.shape
    k = kp1 - 1
    acc = torch.zeros(b_n, dtype=torch.int32)
    tok = torch.full((b_n, kp1), -1, dtype=torch.int64)
    for b in range(b_n):
        rows = torch.cat([target_logits[b], draft_logits[b]]).float()
        if penalty != 1.0:
            rows = apply_penalty(rows, histories[b], penalty)
        dist = filtered_probabilities(rows, temperature, 1 << 30, top_p)
        P, Q = dist[:kp1], dist[kp1:]
        a = 0
        while a < k:
            x = int(draft_tokens[b, a])
            dec = verify(P[a, x].view(1), Q[a, x].view(1), torch.tensor([x]), uniforms[b, a].view(1))
            if dec[0, 2] == 0:
                break
            tok[b, a] = x
            a += 1
        if a < k:
            first_delta = (P[a] - Q[a]).clamp_min(0)
            mass = first_delta.sum()
            fallback = first_delta / mass if mass > 0 else P[a] / P[a].sum()
            tok[b, a] = categorical_pick(fallback.view(1, -1), uniforms[b, k + a].view(1))[0]
        else:
            tok[b, a] = categorical_pick(P[k].view(1, -1), uniforms[b, 2 * k].view(1))[0]
        acc[b] = a
    return acc, tok
