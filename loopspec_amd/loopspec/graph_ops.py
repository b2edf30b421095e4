"""KV-slot allocation, request-mapping update and state-row copies (drop-in).

Same call signatures and in-place semantics as the reference's graph ops
(sglang_recurrent/loopspec/graph_ops.py:53-271); every call enqueues one gfx950
kernel on the current stream and is safe to record into a HIP graph (no host
synchronisation, no allocation for int64 index tensors). Plus ``commit_kv``,
the batched branch -> main KV-timeline commit of accepted draft tokens.

Differences a caller can observe, all on inputs the reference declares invalid:
non-negative row indices outside the bank and append positions outside the
mapping row are skipped instead of written out of bounds.
"""

from __future__ import annotations

from typing import Any

import torch

from .. import _lib


def _index(t: torch.Tensor, what: str) -> torch.Tensor:
    _lib.require_cuda(t, what)
    if t.dtype != torch.int64:
        t = t.to(torch.int64)
    if not t.is_contiguous():
        t = t.contiguous()
    return t


def _out_index(t: torch.Tensor, what: str) -> torch.Tensor:
    _lib.require_cuda(t, what)
    if t.dtype != torch.int64 or not t.is_contiguous():
        raise ValueError(f"{what} must be a contiguous CUDA int64 tensor")
    return t


def copy_state_rows(source: Any, destination: Any, row_indices: Any, *, gather: bool) -> None:
    """Gather destination[b] = source[row_indices[b]] or scatter
    destination[row_indices[b]] = source[b]; negative indices skip the row.

    source/destination: contiguous CUDA tensors of one dtype with equal row
    width W ([N, W] bank and [B, W] batch; 1-D tensors have W = 1).
    Follows sglang_recurrent/loopspec/graph_ops.py:20-94.
    """
    for t, what in ((source, "copy_state_rows source"), (destination, "copy_state_rows destination")):
        _lib.require_cuda(t, what)
        if not t.is_contiguous():
            raise ValueError(f"{what} must be contiguous")
    if source.dtype != destination.dtype:
        raise ValueError("copy_state_rows: source and destination dtypes differ")
    idx = _index(row_indices, "copy_state_rows row_indices")
    width = source.shape[1] if source.dim() > 1 else 1
    dwidth = destination.shape[1] if destination.dim() > 1 else 1
    if width != dwidth:
        raise ValueError("copy_state_rows: source and destination row widths differ")
    row_width = source[0].numel() if source.dim() > 1 and source.shape[0] else width
    bank = source if gather else destination
    bank_rows = bank.shape[0] if bank.dim() > 0 else 1
    batch = idx.shape[0]
    if batch == 0:
        return
    _lib.call(
        "ls_copy_state_rows", source.data_ptr(), destination.data_ptr(), idx.data_ptr(), batch, bank_rows,
        row_width * source.element_size(), 1 if gather else 0, _lib.stream(source.device),
    )


def allocate_decode_slots(free_slots: Any, allocation_cursor: Any, valid_markers: Any, out_cache_locs: Any) -> None:
    """Rows with valid_markers >= 0 take ring entries free_slots[(cursor + rank)
    % C] in batch order; the device cursor advances by the number of valid rows.

    free_slots int64 [C], allocation_cursor int64 scalar (both updated/read on
    device), valid_markers [B], out_cache_locs int64 [B] (skipped rows keep
    their value). Follows sglang_recurrent/loopspec/graph_ops.py:97-172.
    """
    free = _out_index(free_slots, "allocate_decode_slots free_slots")
    cursor = _out_index(allocation_cursor, "allocate_decode_slots allocation_cursor")
    markers = _index(valid_markers, "allocate_decode_slots valid_markers")
    out = _out_index(out_cache_locs, "allocate_decode_slots out_cache_locs")
    if cursor.numel() != 1:
        raise ValueError("allocate_decode_slots: allocation_cursor must hold one int64")
    batch = markers.shape[0]
    if out.shape[0] < batch:
        raise ValueError("allocate_decode_slots: out_cache_locs is shorter than valid_markers")
    _lib.call(
        "ls_allocate_decode_slots", free.data_ptr(), free.shape[0], cursor.data_ptr(), markers.data_ptr(), batch,
        out.data_ptr(), _lib.stream(free.device),
    )


def update_request_mapping(mapping: Any, request_rows: Any, source_rows: Any, copy_lens: Any, positions: Any,
                           out_cache_locs: Any) -> None:
    """copy_lens > 0 copies mapping[source, :copy_len] to mapping[request, :copy_len];
    copy_lens >= 0 appends mapping[request, position] = int32(out_cache_loc);
    copy_lens < 0 writes nothing for the row.

    mapping: CUDA int32 [request_capacity, max_context_len], contiguous columns.
    Follows sglang_recurrent/loopspec/graph_ops.py:175-271.
    """
    _lib.require_cuda(mapping, "update_request_mapping mapping")
    if mapping.dtype != torch.int32 or mapping.dim() != 2 or mapping.stride(1) != 1:
        raise ValueError("update_request_mapping: mapping must be int32 [rows, context] with contiguous columns")
    args = [_index(t, "update_request_mapping " + n) for t, n in (
        (request_rows, "request_rows"), (source_rows, "source_rows"), (copy_lens, "copy_lens"),
        (positions, "positions"), (out_cache_locs, "out_cache_locs"))]
    batch = args[0].shape[0]
    if any(a.shape[0] < batch for a in args):
        raise ValueError("update_request_mapping: [B] arrays must have equal length")
    if batch == 0:
        return
    _lib.call(
        "ls_update_request_mapping", mapping.data_ptr(), mapping.stride(0), mapping.shape[1],
        *(a.data_ptr() for a in args), batch, _lib.stream(mapping.device),
    )


def commit_kv(kv: torch.Tensor | None, accept_len: torch.Tensor, branch_slots: torch.Tensor,
              page_table: torch.Tensor, ctx_len: torch.Tensor, free_pages: torch.Tensor,
              page_state: torch.Tensor, page_size: int, *, dst_slots: torch.Tensor | None = None,
              status: torch.Tensor | None = None) -> torch.Tensor:
    """Commit each row's accepted branch tokens into its main KV timeline.

    kv: [planes, num_pages * page_size, *token_shape] (planes = layers x loops x
    {K, V}) or None to only plan. accept_len int32 [B]; branch_slots int64
    [B, k]; page_table int32 [B, max_pages]; ctx_len int64 [B]; free_pages
    int64 ring; page_state int64 [2] = (next, end): ring entries next .. end-1
    hold free pages. Positions ctx_len.. take the row's pages, new pages come
    from the ring in batch order (the allocation rule of graph_ops.py:117-134);
    page_table, ctx_len and page_state[0] are updated in
    place and every plane's token row is copied branch slot -> destination slot.
    Returns dst_slots int64 [B, k] (-1 for tokens that were not accepted).
    The reference's own commit is an ownership transfer of page-size-1 slots
    (sglang_recurrent/loopspec/branching/manager.py:410-482).
    """
    for t, n in ((accept_len, "accept_len"), (branch_slots, "branch_slots"), (page_table, "page_table"),
                 (ctx_len, "ctx_len"), (free_pages, "free_pages"), (page_state, "page_state")):
        _lib.require_cuda(t, "commit_kv " + n)
        if not t.is_contiguous():
            raise ValueError(f"commit_kv: {n} must be contiguous")
    if accept_len.dtype != torch.int32 or page_table.dtype != torch.int32:
        raise ValueError("commit_kv: accept_len and page_table must be int32")
    for t, n in ((branch_slots, "branch_slots"), (ctx_len, "ctx_len"), (free_pages, "free_pages"),
                 (page_state, "page_state")):
        if t.dtype != torch.int64:
            raise ValueError(f"commit_kv: {n} must be int64")
    if page_state.numel() != 2:
        raise ValueError("commit_kv: page_state must hold (next, end)")
    batch, k = branch_slots.shape
    if dst_slots is None:
        dst_slots = torch.empty((batch, k), dtype=torch.int64, device=branch_slots.device)
    if kv is not None:
        if not kv.is_contiguous():
            raise ValueError("commit_kv: kv must be contiguous")
        planes = kv.shape[0]
        token_bytes = kv[0, 0].numel() * kv.element_size()
        plane_bytes = kv[0].numel() * kv.element_size()
        slots = kv.shape[1]
        kv_ptr = kv.data_ptr()
    else:
        planes, token_bytes, plane_bytes, kv_ptr = 0, 16, 0, None
        slots = None
    num_pages = (slots // page_size) if slots is not None else 2**31 - 1
    _lib.call(
        "ls_kv_commit", kv_ptr, planes, plane_bytes, token_bytes, num_pages, page_size, accept_len.data_ptr(),
        branch_slots.data_ptr(), batch, k, page_table.data_ptr(), page_table.shape[1], ctx_len.data_ptr(),
        free_pages.data_ptr(), free_pages.shape[0], page_state.data_ptr(), dst_slots.data_ptr(),
        _lib.ptr(status), _lib.stream(branch_slots.device),
    )
    return dst_slots
