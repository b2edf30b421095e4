"""DeviceTimelines on the device decode-slot pool against the restated
reference (oracle.branches for the ownership rules, manager.py:390-482;
oracle.graph_ops.DecodeSlotPool for the ID order, decode_slots.py:113-166):
every decode's IDs, every branch's owned IDs after each prune, and, once all
is released, the order in which the pool hands the recycled IDs out again."""

import pytest
import torch

from loopspec_amd.loopspec.branching.decode_slots import DeviceSlotPool
from loopspec_amd.loopspec.branching.timelines import DeviceTimelines
from oracle import graph_ops as og
from oracle.branches import BranchTimelines, Cursor
from tests.conftest import announce
from tests.timeline_cycles import cycles

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", [0, 3, 4])
def test_device_timelines_match_the_reference_pool(gpu, seed):
    cap, pre, fork = 256, 7, 48
    announce(f"device timelines seed={seed} cap={cap}")
    pool = DeviceSlotPool(cap, gpu)
    pool.begin(pre)
    ref_pool = og.DecodeSlotPool(cap)
    ref_pool.begin(pre)
    dev = DeviceTimelines(pool, list(reversed(range(100, 100 + fork))))
    ref = BranchTimelines(fork_rows=fork)
    dev.initialize_root({"core": {0: (1, 10), 1: (2, 10)}})
    ref.initialize_root({"core": {0: Cursor(1, 10), 1: Cursor(2, 10)}})
    given = 0
    for decode, keep in cycles(seed, 8):
        depths = [d for d, _, _ in decode]
        branches = [b for _, b, _ in decode]
        parents = [p for _, _, p in decode]
        dt = dev.timelines("core", depths, branches, parents)
        rt = ref.cursors("core", depths, branches, parents)
        out = torch.zeros(len(dt), dtype=torch.int64, device=gpu)
        dev.decode(dt, out)
        ref_pool.release(ref.released[given:])
        given = len(ref.released)
        want = ref_pool.allocate(len(rt))
        assert out.cpu().tolist() == want
        for c, slot in zip(rt, want):
            ref.decode(c, slot)
        dev.retain_branches(keep)
        ref.retain_branches(keep)
        for b in ref.nodes:
            assert dev.owned_slots(b) == ref.owned(b), b
    dev.flush()
    ref_pool.release(ref.released[given:])
    assert dev.finished and pool.errors() == 0
    # every ID is free again: the pool hands them out in the reference's order
    rest = cap - pre
    out = torch.zeros(rest, dtype=torch.int64, device=gpu)
    pool.allocate(torch.arange(rest, dtype=torch.int64, device=gpu), out)
    assert out.cpu().tolist() == ref_pool.allocate(rest)
    assert pool.errors() == 0


@pytest.mark.parametrize("seed", [1, 2])
def test_decode_metadata_and_mapping_follow_the_reference(gpu, seed):
    """Each decode stages its rows from the timelines (a fork copies its
    parent's prefix once), takes IDs from the pool and updates the request
    mapping through graph_ops: the table must equal the restated reference's
    (oracle pool + branch rules + update_request_mapping) after every step."""
    import numpy as np

    from loopspec_amd.loopspec import graph_ops as go
    from loopspec_amd.loopspec.metadata import DecodeStagingSlot, MetadataRow, payload_size

    cap, pre, fork, ctx = 512, 20, 48, 40
    announce(f"timelines + metadata + mapping seed={seed}")
    pool = DeviceSlotPool(cap, gpu)
    pool.begin(pre)
    ref_pool = og.DecodeSlotPool(cap)
    ref_pool.begin(pre)
    dev = DeviceTimelines(pool, list(reversed(range(100, 100 + fork))))
    ref = BranchTimelines(fork_rows=fork)
    dev.initialize_root({"core": {0: (1, 10), 1: (2, 10)}})
    ref.initialize_root({"core": {0: Cursor(1, 10), 1: Cursor(2, 10)}})
    table = np.zeros((160, ctx), dtype=np.int32)
    table[1, :10] = np.arange(1, 11)
    table[2, :10] = np.arange(11, 21)
    mapping = torch.from_numpy(table).to(gpu)
    given = 0
    for step, (decode, keep) in enumerate(cycles(seed, 8)):
        depths = [d for d, _, _ in decode]
        branches = [b for _, b, _ in decode]
        parents = [p for _, _, p in decode]
        dt = dev.timelines("core", depths, branches, parents)
        rt = ref.cursors("core", depths, branches, parents)
        n = len(dt)
        tokens = [1000 + 10 * step + i for i in range(n)]
        payload = torch.zeros(payload_size(n), dtype=torch.uint8, device=gpu)
        rows, _, tok, _ = DecodeStagingSlot(n).stage(dt, tokens, payload)
        # the reference's staging rule on its own cursors (metadata.py:137-178)
        want_rows = [[c.row for c in rt], [c.seq_len + 1 for c in rt], [c.seq_len for c in rt], tokens,
                     [c.row if c.pending_parent is None else c.pending_parent for c in rt],
                     [0 if c.pending_parent is None else c.seq_len for c in rt], [-1] * n, [-1] * n]
        out = torch.zeros(n, dtype=torch.int64, device=gpu)
        dev.decode(dt, out)
        go.update_request_mapping(mapping, rows[MetadataRow.REQUEST], rows[MetadataRow.PARENT_REQUEST],
                                  rows[MetadataRow.MAPPING_COPY_LENGTH], rows[MetadataRow.POSITION], out)
        ref_pool.release(ref.released[given:])
        given = len(ref.released)
        slots = ref_pool.allocate(n)
        og.update_request_mapping(table, want_rows[0], want_rows[4], want_rows[5], want_rows[2], slots)
        for c, slot in zip(rt, slots):
            ref.decode(c, slot)
        assert rows.cpu().tolist() == want_rows and tok.cpu().tolist() == tokens
        assert out.cpu().tolist() == slots
        assert np.array_equal(mapping.cpu().numpy(), table), step
        dev.retain_branches(keep)
        ref.retain_branches(keep)
    dev.flush()
    assert dev.finished and pool.errors() == 0
