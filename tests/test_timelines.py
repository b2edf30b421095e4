"""DeviceTimelines' host bookkeeping against oracle.branches (the restated
reference rules, manager.py:390-482) on seeded speculation cycles, with a
recording stand-in for the device pool: the IDs handed back, in order, the
released request rows and every branch's ownership must agree after every
step."""

import pytest
import torch

from loopspec_amd.loopspec.branching.timelines import DeviceTimelines
from oracle.branches import BranchTimelines, Cursor
from tests.timeline_cycles import cycles


class RecordingPool:
    """CPU stand-in for DeviceSlotPool: hands out 1, 2, 3, ... and records releases."""

    def __init__(self, capacity: int) -> None:
        self.capacity = capacity
        self.device = torch.device("cpu")
        self.next = 1
        self.released: list[int] = []

    def step(self, slots, markers, out) -> None:
        self.released.extend(int(s) for s in slots)
        for b in range(out.numel()):
            out[b] = self.next
            self.next += 1

    def release(self, slots) -> None:
        self.released.extend(int(s) for s in slots)


@pytest.mark.parametrize("seed", range(6))
def test_device_timelines_follow_the_reference_rules(seed):
    fork = 48
    pool = RecordingPool(4096)
    dev = DeviceTimelines(pool, list(reversed(range(100, 100 + fork))))
    ref = BranchTimelines(fork_rows=fork)
    dev.initialize_root({"core": {0: (1, 10), 1: (2, 10)}})
    ref.initialize_root({"core": {0: Cursor(1, 10), 1: Cursor(2, 10)}})
    for decode, keep in cycles(seed, 8):
        depths = [d for d, _, _ in decode]
        branches = [b for _, b, _ in decode]
        parents = [p for _, _, p in decode]
        dt = dev.timelines("core", depths, branches, parents)
        rt = ref.cursors("core", depths, branches, parents)
        assert [t.row for t in dt] == [c.row for c in rt]
        out = torch.zeros(len(dt), dtype=torch.int64)
        dev.decode(dt, out)
        for c, slot in zip(rt, out.tolist()):
            ref.decode(c, slot)
        dev.retain_branches(keep)
        ref.retain_branches(keep)
        dev.flush()
        assert pool.released == ref.released
        assert dev.released_rows == ref.released_rows
        assert set(dev.branches) == set(ref.nodes)
        for b in ref.nodes:
            assert dev.owned_slots(b) == ref.owned(b), b
    assert dev.finished and ref.finished
    assert sorted(pool.released) == list(range(1, pool.next))  # every decode ID came back once


def test_fork_rows_exhaust_like_the_reference():
    pool = RecordingPool(64)
    dev = DeviceTimelines(pool, [101, 100])
    dev.initialize_root({"core": {0: (1, 5)}})
    dev.timelines("core", [0, 0], [1, 2], [0, 0])
    with pytest.raises(RuntimeError, match="ran out of request-pool rows"):
        dev.timelines("core", [0], [3], [0])


def test_metadata_payload_layout():
    from loopspec_amd.loopspec.metadata import DECODE_METADATA_ROWS, MetadataRow, payload_size, payload_views

    assert DECODE_METADATA_ROWS == 8 and [r.name for r in MetadataRow] == [
        "REQUEST", "SEQUENCE_LENGTH", "POSITION", "TOKEN", "PARENT_REQUEST", "MAPPING_COPY_LENGTH",
        "STATE_INPUT", "STATE_OUTPUT"]
    b = 5
    assert payload_size(b) == b * (8 * 8 + 4)
    payload = torch.zeros(payload_size(b), dtype=torch.uint8)
    rows, lengths = payload_views(payload, b)
    assert rows.shape == (8, b) and rows.dtype == torch.int64 and lengths.shape == (b,) and lengths.dtype == torch.int32
    rows[MetadataRow.TOKEN] = torch.arange(b)
    lengths[:] = 7
    # the lengths follow the rows, in the same storage
    assert payload[8 * 8 * b:].view(torch.int32).tolist() == [7] * b
    assert payload[3 * 8 * b: 4 * 8 * b].view(torch.int64).tolist() == list(range(b))
