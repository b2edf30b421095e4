"""Batched fused entry points of the verify-and-sample path.

These are the chain-of-k versions of the reference's per-position rules:
the reference verifies one position per pipeline lane and prunes every
descendant of a rejected lane (sglang_recurrent/loopspec/pipeline.py:365-412),
which, over k draft positions, is exactly an accept-prefix scan.
"""

from __future__ import annotations

import torch

from . import _lib


def _check_rows(t: torch.Tensor, what: str) -> None:
    _lib.require_cuda(t, what)
    if t.stride(-1) != 1:
        raise ValueError(f"{what}: the vocabulary axis must be contiguous")


def argmax_rows(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Row-wise argmax of CUDA logits [M, V] with torch.argmax tie/NaN rules.

    Returns int64 [M]. Replaces torch.argmax in GreedyDecisionPolicy.queue
    (sglang_recurrent/loopspec/decisions.py:116).
    """
    _check_rows(logits, "argmax")
    if logits.dim() != 2:
        raise ValueError("argmax_rows expects [rows, vocab] logits")
    rows, vocab = logits.shape
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=logits.device)
    elif out.shape != (rows,) or out.dtype != torch.int64 or not out.is_contiguous():
        raise ValueError("argmax_rows: out must be contiguous int64 [rows]")
    nbytes = _lib.query("ls_argmax_rows_workspace", rows, vocab)
    ws = _lib.WORKSPACE.get(logits.device, nbytes, "argmax")
    _lib.call(
        "ls_argmax_rows", logits.data_ptr(), _lib.dtype_code(logits), rows, vocab, logits.stride(0),
        out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream(logits.device),
    )
    return out


def greedy_verify(
    target_logits: torch.Tensor,
    draft_logits: torch.Tensor | None = None,
    draft_tokens: torch.Tensor | None = None,
    *,
    accept_len: torch.Tensor | None = None,
    tokens: torch.Tensor | None = None,
    row_argmax: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Greedy chain verification in one launch.

    target_logits: [B, k+1, V]; draft_logits: [B, k, V] (same dtype) or
    draft_tokens: int64 [B, k]. Returns (accept_len int32 [B], tokens int64
    [B, k+1]); tokens[b, :accept_len+1] are the target argmaxes (accepted
    drafts then the correction/bonus token), the rest are -1. If row_argmax
    (int64 [B, 2k+1]) is given it receives every row's argmax.
    """
    _check_rows(target_logits, "greedy_verify")
    if target_logits.dim() != 3:
        raise ValueError("target_logits must be [B, k+1, V]")
    batch, kp1, vocab = target_logits.shape
    k = kp1 - 1
    if k < 1:
        raise ValueError("greedy_verify needs at least one draft position")
    dev = target_logits.device
    if draft_logits is not None:
        _check_rows(draft_logits, "greedy_verify")
        if draft_logits.shape != (batch, k, vocab) or draft_logits.dtype != target_logits.dtype:
            raise ValueError("draft_logits must be [B, k, V] with the target's dtype")
        d_ptr, d_bs, d_ps = draft_logits.data_ptr(), draft_logits.stride(0), draft_logits.stride(1)
        tok_ptr = None
    else:
        if draft_tokens is None:
            raise ValueError("greedy_verify needs draft_logits or draft_tokens")
        if draft_tokens.shape != (batch, k) or draft_tokens.dtype != torch.int64:
            raise ValueError("draft_tokens must be int64 [B, k]")
        draft_tokens = draft_tokens.contiguous()
        d_ptr, d_bs, d_ps, tok_ptr = None, 0, 0, draft_tokens.data_ptr()
    if accept_len is None:
        accept_len = torch.empty(batch, dtype=torch.int32, device=dev)
    if tokens is None:
        tokens = torch.empty((batch, kp1), dtype=torch.int64, device=dev)
    if accept_len.shape != (batch,) or accept_len.dtype != torch.int32 or not accept_len.is_contiguous():
        raise ValueError("accept_len must be contiguous int32 [B]")
    if tokens.shape != (batch, kp1) or tokens.dtype != torch.int64 or not tokens.is_contiguous():
        raise ValueError("tokens must be contiguous int64 [B, k+1]")
    if row_argmax is not None and (
        row_argmax.shape != (batch, 2 * k + 1) or row_argmax.dtype != torch.int64 or not row_argmax.is_contiguous()
    ):
        raise ValueError("row_argmax must be contiguous int64 [B, 2k+1]")
    nbytes = _lib.query("ls_greedy_verify_workspace", batch, k, vocab)
    ws = workspace if workspace is not None else _lib.WORKSPACE.get(dev, nbytes, "greedy")
    _lib.call(
        "ls_greedy_verify",
        target_logits.data_ptr(), target_logits.stride(0), target_logits.stride(1),
        d_ptr, d_bs, d_ps, tok_ptr,
        _lib.dtype_code(target_logits), batch, k, vocab,
        accept_len.data_ptr(), tokens.data_ptr(), _lib.ptr(row_argmax),
        ws.data_ptr(), ws.numel(), _lib.stream(dev),
    )
    return accept_len, tokens


def greedy_verify_workspace_bytes(batch: int, k: int, vocab: int) -> int:
    return _lib.query("ls_greedy_verify_workspace", batch, k, vocab)
