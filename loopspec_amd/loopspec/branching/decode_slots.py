"""GPU-resident decode KV slot pool.

Replaces DecodeSlotPool (sglang_recurrent/loopspec/branching/decode_slots.py:13-166),
whose CPU sequence, recycle list and live set mirror the device ring so that
the CPU can name each graph's slots before replay. Here the ring, the
allocation cursor, the end of the ID sequence, the live set and the error
bits all stay on the device: allocate() writes the slots of the valid rows
straight into the graph's out_cache_locs buffer (as allocate_decode_slots,
graph_ops.py:137-172, does from the same ring), release() appends freed IDs
after the unconsumed ones in release order, and nothing is read back unless
the caller asks (check()). The IDs come out in the reference's order: its
lazy refill appends recycled IDs at the same place, after the unconsumed IDs.

Calls must be ordered on one stream (like the reference, this is not a
thread-safe pool); every call may be captured in a HIP graph.
"""

from __future__ import annotations

import torch

from ... import _lib

ERR_EXHAUSTED = 1
ERR_LIVE = 2
ERR_UNOWNED = 4


class DeviceSlotPool:
    def __init__(self, capacity: int, device: torch.device | str | int) -> None:
        """capacity usable KV token slots with IDs 1..capacity; a non-CUDA
        device raises ValueError (decode_slots.py:24-48)."""
        self.capacity = int(capacity)
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("decode slot pools require a CUDA device")
        if self.capacity <= 0:
            raise ValueError("capacity must be positive")
        self.free_slots = torch.arange(1, self.capacity + 1, dtype=torch.int64, device=self.device)
        self.state = torch.zeros(3, dtype=torch.int64, device=self.device)
        # the allocation cursor, as the reference's allocation_cursor scalar
        self.allocation_cursor = self.state[0]
        words = _lib.query("ls_slot_pool_live_words", self.capacity)
        self.live = torch.zeros(words, dtype=torch.int32, device=self.device)

    def _stream(self):
        return _lib.stream(self.device)

    def begin(self, allocated_slots: int) -> None:
        """Reset after full-prompt prefill: IDs 1..allocated_slots stay with the
        prompt (decode_slots.py:50-74)."""
        if not 0 <= allocated_slots <= self.capacity:
            raise ValueError("invalid graph decode KV allocation offset")
        _lib.call("ls_slot_pool_begin", self.free_slots.data_ptr(), self.capacity, self.state.data_ptr(),
                  self.live.data_ptr(), int(allocated_slots), self._stream())

    def allocate(self, valid_markers: torch.Tensor, out_cache_locs: torch.Tensor) -> None:
        """Rows with valid_markers[b] >= 0 take the next IDs in batch order into
        out_cache_locs[b] (int64 [B] device tensors); they become live
        (decode_slots.py:113-151 + graph_ops.py:137-172, one launch)."""
        for t, what in ((valid_markers, "valid_markers"), (out_cache_locs, "out_cache_locs")):
            _lib.require_cuda(t, "slot pool allocate")
            if t.dtype != torch.int64 or t.dim() != 1 or not t.is_contiguous():
                raise ValueError(f"slot pool allocate: {what} must be contiguous int64 [B]")
        if valid_markers.shape != out_cache_locs.shape:
            raise ValueError("slot pool allocate: valid_markers and out_cache_locs differ in shape")
        _lib.call("ls_slot_pool_allocate", self.free_slots.data_ptr(), self.capacity, self.state.data_ptr(),
                  self.live.data_ptr(), valid_markers.data_ptr(), valid_markers.numel(),
                  out_cache_locs.data_ptr(), self._stream())

    def release(self, slots: torch.Tensor) -> None:
        """Give live IDs (int64 [n] device tensor, in order) back to the pool
        (decode_slots.py:153-166)."""
        _lib.require_cuda(slots, "slot pool release")
        if slots.dtype != torch.int64 or slots.dim() != 1 or not slots.is_contiguous():
            raise ValueError("slot pool release: slots must be contiguous int64 [n]")
        _lib.call("ls_slot_pool_release", self.free_slots.data_ptr(), self.capacity, self.state.data_ptr(),
                  self.live.data_ptr(), slots.data_ptr(), slots.numel(), self._stream())

    def step(self, slots: torch.Tensor, valid_markers: torch.Tensor, out_cache_locs: torch.Tensor) -> None:
        """release(slots) then allocate(valid_markers, out_cache_locs), in one
        launch (a decode step's order: pruned timelines give their IDs back
        before the next rows take theirs)."""
        for t, what in ((slots, "slots"), (valid_markers, "valid_markers"), (out_cache_locs, "out_cache_locs")):
            _lib.require_cuda(t, "slot pool step")
            if t.dtype != torch.int64 or t.dim() != 1 or not t.is_contiguous():
                raise ValueError(f"slot pool step: {what} must be contiguous int64 [n]")
        if valid_markers.shape != out_cache_locs.shape:
            raise ValueError("slot pool step: valid_markers and out_cache_locs differ in shape")
        _lib.call("ls_slot_pool_step", self.free_slots.data_ptr(), self.capacity, self.state.data_ptr(),
                  self.live.data_ptr(), slots.data_ptr(), slots.numel(), valid_markers.data_ptr(),
                  valid_markers.numel(), out_cache_locs.data_ptr(), self._stream())

    def errors(self) -> int:
        """The error bits so far (one device read)."""
        return int(self.state[2].item())

    def check(self) -> None:
        """Raise RuntimeError with the reference's message for the first kind
        of error recorded (one device read)."""
        e = self.errors()
        if e & ERR_EXHAUSTED:
            raise RuntimeError("recurrent decode ran out of KV cache slots")
        if e & ERR_LIVE:
            raise RuntimeError("recurrent decode allocated a live KV slot")
        if e & ERR_UNOWNED:
            raise RuntimeError("recurrent decode released an unowned KV slot")
