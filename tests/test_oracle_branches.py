"""oracle.branches: the reference's timeline-ownership rules on hand-worked
trees (manager.py:390-482), and the released slots going back to the
decode-slot pool model in release order (decode_slots.py:153-166)."""

import pytest

from oracle import graph_ops as og
from oracle.branches import BranchTimelines, Cursor


def _root(tl: BranchTimelines) -> None:
    # two recurrent depths with prefill rows 1 and 2 (no decode slots owned yet)
    tl.initialize_root({"core": {0: Cursor(1, 10), 1: Cursor(2, 10)}})


def _decode(tl, branch, parent, slot, stage=0):
    (cur,) = tl.cursors("core", [stage], [branch], [parent])
    tl.decode(cur, slot)
    return cur


def test_accepted_chain_inherits_everything_and_frees_nothing():
    tl = BranchTimelines(fork_rows=4)
    _root(tl)
    c1 = _decode(tl, 1, 0, 11)
    c2 = _decode(tl, 2, 1, 12)
    assert (c1.row, c2.row) == (100, 101) and c2.seq_len == 12 and c2.pending_parent is None
    tl.retain_branches([(2, 1)])
    assert tl.released == []
    assert tl.released_rows == [1]  # the root's depth-0 prefill row, its ownership moved down
    assert list(tl.nodes) == [2]
    assert tl.owned(2) == {"pre": {}, "core": {0: [11, 12], 1: []}, "post": {}}
    assert tl.nodes[2].cursors["core"][1].row == 2  # depth 1 moved whole, with its row
    assert tl.available_rows == [103, 102, 100]


def test_rejection_releases_the_pruned_subtree_deepest_first():
    tl = BranchTimelines(fork_rows=4)
    _root(tl)
    _decode(tl, 1, 0, 11)
    _decode(tl, 2, 1, 12)
    _decode(tl, 3, 0, 13)
    tl.retain_branches([(3, 0)])
    assert tl.released == [12, 11]
    assert tl.released_rows == [1]
    assert list(tl.nodes) == [3]
    assert tl.owned(3) == {"pre": {}, "core": {0: [13], 1: []}, "post": {}}
    assert sorted(tl.available_rows) == [100, 101, 103]


def test_live_parent_keeps_its_slots_until_pruned():
    tl = BranchTimelines(fork_rows=4)
    _root(tl)
    _decode(tl, 1, 0, 11)
    _decode(tl, 2, 1, 12)
    _decode(tl, 3, 1, 13)
    tl.retain_branches([(2, 1), (3, 1)])  # branch 1 has two children: it stays, owning 11
    assert tl.released == [] and set(tl.nodes) == {1, 2, 3}
    # the unretained root's sole child, branch 1, took over its depths (depth 1 whole)
    assert tl.owned(1)["core"] == {0: [11], 1: []} and tl.released_rows == [1]
    tl.retain_branches([(3, 1)])  # branch 2 pruned; 3 is now 1's sole child and inherits 11
    assert tl.released == [12]
    assert tl.owned(3)["core"] == {0: [11, 13], 1: []}


def test_empty_frontier_releases_all_and_finishes():
    tl = BranchTimelines(fork_rows=4)
    _root(tl)
    _decode(tl, 1, 0, 11)
    _decode(tl, 2, 1, 12)
    tl.retain_branches([(2, 1)])
    tl.retain_branches([])
    assert tl.released == [11, 12]
    assert tl.released_rows == [1, 2]
    assert tl.finished and sorted(tl.available_rows) == [100, 101, 102, 103]


def test_unknown_parent_and_row_exhaustion_raise():
    tl = BranchTimelines(fork_rows=1)
    _root(tl)
    with pytest.raises(RuntimeError, match="unavailable parent"):
        tl.cursors("core", [0], [5], [4])
    _decode(tl, 1, 0, 11)
    with pytest.raises(RuntimeError, match="request-pool rows"):
        tl.cursors("core", [1], [1], [0])


def test_released_slots_return_to_the_pool_in_release_order():
    pool = og.DecodeSlotPool(8)
    pool.begin(0)
    slots = pool.allocate(3)  # the decodes of branches 1, 2 and 3
    tl = BranchTimelines(fork_rows=4)
    _root(tl)
    _decode(tl, 1, 0, slots[0])
    _decode(tl, 2, 1, slots[1])
    _decode(tl, 3, 0, slots[2])
    tl.retain_branches([(3, 0)])
    assert tl.released == [slots[1], slots[0]]
    pool.release(tl.released)
    # the sequence runs out after the 5 unused IDs, then the released IDs come back in release order
    got = pool.allocate(7)
    assert got[:5] == [4, 5, 6, 7, 8] and got[5:] == tl.released
