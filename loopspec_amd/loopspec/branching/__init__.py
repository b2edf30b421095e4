"""Branch-side KV bookkeeping (sglang_recurrent/loopspec/branching/)."""

from .decode_slots import DeviceSlotPool

__all__ = ["DeviceSlotPool"]
