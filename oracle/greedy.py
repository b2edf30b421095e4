"""Greedy verification oracle (exact integer/index semantics; numpy).

Pinned by: brute-force pure-Python argmax, planted and natural bf16 ties,
NaN/-0 cases (tests/test_oracle_greedy.py), and exhaustive enumeration of
every (match/mismatch)^k draft pattern against the per-lane rule.
"""

from __future__ import annotations

import numpy as np


def argmax_first(x: np.ndarray) -> np.ndarray:
    """Row-wise argmax with torch.argmax semantics.

    Follows sglang_recurrent/loopspec/decisions.py:116 (torch.argmax): the
    first index of the maximum; NaN compares above every number (the first NaN
    wins); -0.0 and +0.0 are equal. numpy's argmax has the same rules.
    x: float array [..., V]; returns int64 [...].
    """
    x = np.asarray(x)
    if x.dtype not in (np.float32, np.float64, np.float16):
        x = x.astype(np.float32)
    return np.argmax(x, axis=-1).astype(np.int64)


def resolve_final(prediction: int, first_token: int | None, second_token: int | None):
    """Final-endpoint greedy rule of GreedyDecisionPolicy.resolve.

    Follows sglang_recurrent/loopspec/decisions.py:163-170: q1 is accepted when
    the final argmax equals it; otherwise q2 (if proposed) when it equals q2.
    Returns (accepted_code, first_rejected, second_rejected) with
    accepted_code 1 = q1, 2 = q2, 0 = none.
    """
    if first_token is None:
        return 0, False, False
    if prediction == first_token:
        return 1, False, False
    if second_token is None:
        return 0, True, False
    if prediction == second_token:
        return 2, True, False
    return 0, True, True


def greedy_chain(target_argmax: np.ndarray, draft_ids: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Accept-prefix over k positions from per-row argmaxes.

    target_argmax: int64 [B, k+1]; draft_ids: int64 [B, k].
    Position i is accepted by the q1 rule (decisions.py:163-166) only if every
    earlier position was accepted, because a rejection discards all descendant
    lanes (sglang_recurrent/loopspec/pipeline.py:379-412). The emitted tokens
    are the target argmaxes up to and including the first mismatch (the
    correction token) or the bonus token at position k.
    Returns (accept_len int32 [B], tokens int64 [B, k+1] with -1 padding).
    """
    t = np.asarray(target_argmax, dtype=np.int64)
    d = np.asarray(draft_ids, dtype=np.int64)
    batch, kp1 = t.shape
    k = kp1 - 1
    accept = np.zeros(batch, dtype=np.int32)
    tokens = np.full((batch, kp1), -1, dtype=np.int64)
    for b in range(batch):
        a = 0
        while a < k:
            code, _, _ = resolve_final(int(t[b, a]), int(d[b, a]), None)
            if code != 1:
                break
            a += 1
        accept[b] = a
        tokens[b, : a + 1] = t[b, : a + 1]
    return accept, tokens


def greedy_verify(target_logits: np.ndarray, draft_logits: np.ndarray | None = None,
                  draft_tokens: np.ndarray | None = None):
    """Oracle of ls_greedy_verify: argmax every row, then the accept prefix.

    target_logits: [B, k+1, V]; draft_logits: [B, k, V] (draft ids are their
    argmax, as the reference argmaxes q1 endpoint rows together with the final
    rows, decisions.py:99-117) or draft_tokens: int64 [B, k].
    Returns (accept_len, tokens, row_argmax [B, 2k+1]).
    """
    t = argmax_first(target_logits)
    d = argmax_first(draft_logits) if draft_logits is not None else np.asarray(draft_tokens, dtype=np.int64)
    accept, tokens = greedy_chain(t, d)
    return accept, tokens, np.concatenate([t, d], axis=1)
