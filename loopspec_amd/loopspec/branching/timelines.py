"""Decode-KV ownership of recurrent timelines, with the slot IDs on the device.

The reference's BranchManager (sglang_recurrent/loopspec/branching/manager.py)
keeps, per branch node, one TimelineCursor per (role, depth) whose
owned_kv_slots lists the decode KV IDs that timeline must give back
(:45-63); a decode appends the new ID, a fork starts empty (:207-232), a
pruned timeline releases its IDs to the decode-slot pool in list order
(:234-251), and a sole child inherits an unused parent's timelines or, where
it has its own, the parent's IDs ahead of its own (:410-451), which is the
"commit" of accepted speculation (retain_branches, :453-482).

The reference can name every ID on the CPU because its pool mirrors the
device ring there (decode_slots.py). With DeviceSlotPool the IDs exist only
on the device, so here the host keeps the tree and, per timeline, the
positions of its IDs in a device-resident log that every decode appends to
(the allocation writes the IDs, the log copies them); a prune gathers the
released timelines' IDs from the log in release order on the device and
gives them to the pool in one launch, with no readback. The tree bookkeeping
runs on the host, as in the reference: it is a handful of dictionary updates
per step.

Calls are ordered on one stream, like DeviceSlotPool's.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .decode_slots import DeviceSlotPool

ROLE_ORDER = ("pre", "core", "post")


@dataclass
class Timeline:
    """One (branch, role, depth) timeline: its request row, prefix length,
    whether the row is a leased fork row, the row to copy the prefix mapping
    from before its first decode, and the log positions of the decode KV IDs
    it owns, oldest first."""

    row: int
    seq_len: int
    fork_row: bool = False
    pending_parent_row: int | None = None
    positions: list[int] = field(default_factory=list)


@dataclass
class _Branch:
    branch_id: int
    parent: "_Branch | None"
    live: bool = True
    children: int = 0
    # role -> depth -> timeline, in creation order (release walks this order)
    timelines: dict[str, dict[int, Timeline]] = field(default_factory=lambda: {r: {} for r in ROLE_ORDER})


class DeviceTimelines:
    def __init__(self, pool: DeviceSlotPool, fork_rows) -> None:
        """pool: the device decode-slot pool the IDs come from and go back to;
        fork_rows: the request rows leased for forks (reserve_fork_rows,
        manager.py:118-144), handed out from the end of the list."""
        self.pool = pool
        self.device = pool.device
        self.fork_rows_total = len(fork_rows)
        self._fork_stack = list(fork_rows)
        # every live decode KV ID has one log position; freed positions are reused
        self.log = torch.zeros(pool.capacity, dtype=torch.int64, device=self.device)
        self._free_positions = list(range(pool.capacity - 1, -1, -1))
        self.branches: dict[int, _Branch] = {}
        self.released_rows: list[int] = []  # prefill rows given back (SGLang's pool in the reference)
        self._pending: list[int] = []       # log positions of released IDs, in release order
        self.finished = False

    # ------------------------------------------------------------------
    # tree growth
    # ------------------------------------------------------------------
    def initialize_root(self, timelines: dict[str, dict[int, tuple[int, int]]]) -> None:
        """The root branch 0 with its prefill timelines: role -> depth ->
        (request row, prefix length) (initialize_root, manager.py:310-329)."""
        if self.branches:
            raise RuntimeError("root branch is already initialized")
        root = _Branch(0, None)
        for role in ROLE_ORDER:
            for depth, (row, seq_len) in timelines.get(role, {}).items():
                root.timelines[role][depth] = Timeline(int(row), int(seq_len))
        self.branches[0] = root

    def _branch(self, branch_id: int, parent_id: int | None) -> _Branch:
        found = self.branches.get(branch_id)
        if found is not None:
            return found
        parent = self.branches.get(parent_id)
        if parent is None:
            raise RuntimeError(f"branch {branch_id} has unavailable parent {parent_id}")
        parent.children += 1
        made = _Branch(branch_id, parent)
        self.branches[branch_id] = made
        return made

    def timelines(self, role: str, depths, branch_ids, parent_ids) -> list[Timeline]:
        """The timeline of each (depth, branch) pair, a branch and a fork of
        its parent's timeline made on first use (get_or_create_cursors,
        manager.py:357-388; fork, :207-232)."""
        out = []
        for depth, branch_id, parent_id in zip(depths, branch_ids, parent_ids, strict=True):
            branch = self._branch(branch_id, parent_id)
            tl = branch.timelines[role].get(depth)
            if tl is None:
                if not self._fork_stack:
                    raise RuntimeError("recurrent branch ran out of request-pool rows")
                src = branch.parent.timelines[role][depth]
                tl = Timeline(self._fork_stack.pop(), src.seq_len, fork_row=True, pending_parent_row=src.row)
                branch.timelines[role][depth] = tl
            out.append(tl)
        return out

    # ------------------------------------------------------------------
    # decode: IDs from the pool into the timelines
    # ------------------------------------------------------------------
    def decode(self, timelines: list[Timeline], out_cache_locs: torch.Tensor) -> None:
        """One decode of each timeline (row b of out_cache_locs, int64 [B] on
        the pool's device): the IDs released since the last call go back to
        the pool first, then every row takes the next ID (DeviceSlotPool.step);
        timeline b now owns out_cache_locs[b] (request.py:219 appends it)."""
        n = len(timelines)
        if out_cache_locs.dtype != torch.int64 or out_cache_locs.shape != (n,) or out_cache_locs.device != self.device:
            raise ValueError("decode: out_cache_locs must be int64 [len(timelines)] on the pool's device")
        if n > len(self._free_positions) + len(self._pending):
            raise RuntimeError("recurrent decode ran out of KV cache slots")
        released = self._take_pending()
        markers = torch.arange(n, dtype=torch.int64, device=self.device)
        self.pool.step(released, markers, out_cache_locs)
        # the released positions are free again once their IDs were gathered
        # (the gather above precedes every later write on the stream)
        positions = [self._free_positions.pop() for _ in range(n)]
        idx = self._upload(positions)
        self.log.index_copy_(0, idx, out_cache_locs)
        for tl, pos in zip(timelines, positions):
            tl.positions.append(pos)
            tl.pending_parent_row = None
            tl.seq_len += 1

    def flush(self) -> None:
        """Give the IDs released so far back to the pool now (one launch)."""
        released = self._take_pending()
        if released.numel():
            self.pool.release(released)

    def _upload(self, values: list[int]) -> torch.Tensor:
        # a new pinned tensor per upload: torch's host allocator keeps it until
        # the asynchronous copy has run, so the host never waits here
        host = torch.tensor(values, dtype=torch.int64)
        if self.device.type != "cuda":
            return host
        return host.pin_memory().to(self.device, non_blocking=True)

    def _take_pending(self) -> torch.Tensor:
        if not self._pending:
            return torch.empty(0, dtype=torch.int64, device=self.device)
        idx = self._upload(self._pending)
        ids = self.log.index_select(0, idx)
        self._free_positions.extend(reversed(self._pending))
        self._pending = []
        return ids

    # ------------------------------------------------------------------
    # pruning and the ownership transfer
    # ------------------------------------------------------------------
    def _release_timeline(self, tl: Timeline) -> None:
        # _TimelineManager.release, manager.py:234-251
        self._pending.extend(tl.positions)
        tl.positions = []
        if tl.fork_row:
            self._fork_stack.append(tl.row)
        else:
            self.released_rows.append(tl.row)

    def _drop_if_unused(self, branch: _Branch) -> None:
        # _release_unused_branch, manager.py:390-409: a dead branch with no
        # children gives back every timeline, then so may its parent
        while branch is not None and not branch.live and branch.children == 0:
            for role in ROLE_ORDER:
                for tl in branch.timelines[role].values():
                    self._release_timeline(tl)
            self.branches.pop(branch.branch_id, None)
            up = branch.parent
            if up is not None:
                up.children -= 1
            branch = up

    @staticmethod
    def _inherit(mine: dict[int, Timeline], theirs: dict[int, Timeline]) -> None:
        # _transfer_timeline_ownership, manager.py:410-429
        for depth in list(theirs):
            if depth in mine:
                mine[depth].positions[:0] = theirs[depth].positions
                theirs[depth].positions = []
            else:
                mine[depth] = theirs.pop(depth)

    def _absorb_parent(self, branch: _Branch) -> None:
        # _detach_from_unused_parent, manager.py:431-451
        up = branch.parent
        if up is None or up.live or up.children != 1:
            return
        for role in ROLE_ORDER:
            self._inherit(branch.timelines[role], up.timelines[role])
        branch.parent = None
        up.children -= 1
        self._drop_if_unused(up)

    def retain_branches(self, lanes) -> None:
        """Keep the surviving frontier, (branch, parent branch) per lane, and
        prune the rest (retain_branches, manager.py:453-482). Released IDs go
        back to the pool at the next decode or flush()."""
        lanes = [(int(b), int(p)) for b, p in lanes]
        for branch_id, parent_id in sorted(lanes):
            if branch_id and branch_id not in self.branches:
                self._branch(branch_id, parent_id)
        keep = {b for b, _ in lanes}
        doomed = sorted((br for br in self.branches.values() if br.live and br.branch_id not in keep),
                        key=lambda br: br.branch_id, reverse=True)
        for br in doomed:
            br.live = False
            self._drop_if_unused(br)
        for br in list(self.branches.values()):
            self._absorb_parent(br)
        if not self.branches:
            # finish_request, manager.py:146-158
            if len(self._fork_stack) != self.fork_rows_total:
                raise RuntimeError("cannot finish LoopSpec with active branch rows")
            self.finished = True

    # ------------------------------------------------------------------
    # queries (one device read each; for checks, not the decode loop)
    # ------------------------------------------------------------------
    def owned_slots(self, branch_id: int) -> dict[str, dict[int, list[int]]]:
        br = self.branches[branch_id]
        log = self.log.cpu()
        return {role: {d: [int(log[p]) for p in tl.positions] for d, tl in br.timelines[role].items()}
                for role in ROLE_ORDER}
