"""CPU restatement of BranchManager's timeline ownership bookkeeping (test
infrastructure only; the library has no host-side branch tree).

Follows sglang_recurrent/loopspec/branching/manager.py: TimelineCursor
(:45-63), _TimelineManager.fork / release (:207-251), _BranchNode (:253-270),
_get_or_create_branch (:331-355), get_or_create_cursors (:357-388) and the
pruning path _release_unused_branch / _transfer_timeline_ownership /
_detach_from_unused_parent / retain_branches (:390-482). It keeps only what
decides which decode KV slots are released and who owns the rest: request
rows are plain integers, prefill cursors own no decode slots (their
owned_kv_slots excludes eager-prefill allocations, :61-63), and a decode
appends the new slot to the cursor's ownership list (request.py:219).

`released` logs every slot given back by release(), in call order: the
argument order of release_decode_slots, which the decode-slot pool recycles
in that order (decode_slots.py:153-166).
"""

from __future__ import annotations

from dataclasses import dataclass, field

ROLES = ("pre", "core", "post")


@dataclass
class Cursor:
    row: int
    seq_len: int
    fork_row: bool = False
    pending_parent: int | None = None
    owned: list[int] = field(default_factory=list)


@dataclass
class Node:
    branch_id: int
    parent: "Node | None" = None
    cursors: dict[str, dict[int, Cursor]] = field(default_factory=lambda: {r: {} for r in ROLES})
    child_count: int = 0
    is_live: bool = True


class BranchTimelines:
    def __init__(self, fork_rows: int, first_fork_row: int = 100) -> None:
        # reserve_fork_rows (:118-144): a stack popped from its end, in row order
        self.available_rows = list(reversed(range(first_fork_row, first_fork_row + fork_rows)))
        self.fork_rows_total = fork_rows
        self.nodes: dict[int, Node] = {}
        self.released: list[int] = []
        self.released_rows: list[int] = []
        self.finished = False

    # --- set-up and growth -------------------------------------------------
    def initialize_root(self, cursors: dict[str, dict[int, Cursor]]) -> None:
        # initialize_root, :310-329
        if self.nodes:
            raise RuntimeError("root branch is already initialized")
        root = Node(0)
        for role in ROLES:
            root.cursors[role] = dict(cursors.get(role, {}))
        self.nodes = {0: root}

    def _get_or_create_branch(self, branch_id: int, parent_id: int | None) -> Node:
        # :331-355
        node = self.nodes.get(branch_id)
        if node is not None:
            return node
        parent = self.nodes.get(parent_id)
        if parent is None:
            raise RuntimeError(f"branch {branch_id} has unavailable parent {parent_id}")
        node = Node(branch_id, parent=parent)
        parent.child_count += 1
        self.nodes[branch_id] = node
        return node

    def _fork(self, parent: Cursor) -> Cursor:
        # _TimelineManager.fork, :207-232
        if not self.available_rows:
            raise RuntimeError("recurrent branch ran out of request-pool rows")
        row = self.available_rows.pop()
        return Cursor(row, parent.seq_len, fork_row=True, pending_parent=parent.row)

    def cursors(self, role: str, stage_ids, branch_ids, parent_ids) -> list[Cursor]:
        # get_or_create_cursors, :357-388
        out = []
        for stage, branch, parent in zip(stage_ids, branch_ids, parent_ids, strict=True):
            node = self._get_or_create_branch(branch, parent)
            cur = node.cursors[role].get(stage)
            if cur is None:
                cur = self._fork(node.parent.cursors[role][stage])
                node.cursors[role][stage] = cur
            out.append(cur)
        return out

    @staticmethod
    def decode(cursor: Cursor, slot: int) -> None:
        """One decode on the cursor's timeline: it now owns the new KV slot."""
        cursor.owned.append(int(slot))
        cursor.pending_parent = None
        cursor.seq_len += 1

    # --- release and pruning -----------------------------------------------
    def _release(self, cursor: Cursor) -> None:
        # _TimelineManager.release, :234-251
        self.released.extend(cursor.owned)
        if cursor.fork_row:
            self.available_rows.append(cursor.row)
        else:
            self.released_rows.append(cursor.row)

    def _release_unused_branch(self, node: Node) -> None:
        # :390-409
        if node.is_live or node.child_count:
            return
        for role in ROLES:
            for cursor in node.cursors[role].values():
                self._release(cursor)
        self.nodes.pop(node.branch_id, None)
        if node.parent is not None:
            node.parent.child_count -= 1
            self._release_unused_branch(node.parent)

    @staticmethod
    def _transfer(child: dict[int, Cursor], parent: dict[int, Cursor]) -> None:
        # _transfer_timeline_ownership, :410-429
        for stage in tuple(parent):
            mine = child.get(stage)
            if mine is None:
                child[stage] = parent.pop(stage)
            else:
                mine.owned[:0] = parent[stage].owned
                parent[stage].owned = []

    def _detach_from_unused_parent(self, node: Node) -> None:
        # :431-451
        parent = node.parent
        if parent is None or parent.is_live or parent.child_count != 1:
            return
        for role in ROLES:
            self._transfer(node.cursors[role], parent.cursors[role])
        node.parent = None
        parent.child_count -= 1
        self._release_unused_branch(parent)

    def retain_branches(self, lanes) -> None:
        """lanes: (branch, parent_branch) pairs of the surviving frontier (:453-482)."""
        lanes = tuple(lanes)
        for branch, parent in sorted(lanes, key=lambda lane: lane[0]):
            if branch and branch not in self.nodes:
                self._get_or_create_branch(branch, parent)
        retained = {branch for branch, _ in lanes}
        unused = [n for n in self.nodes.values() if n.is_live and n.branch_id not in retained]
        for node in sorted(unused, key=lambda n: n.branch_id, reverse=True):
            node.is_live = False
            self._release_unused_branch(node)
        for node in tuple(self.nodes.values()):
            self._detach_from_unused_parent(node)
        if not self.nodes:
            # finish_request (:146-158): every fork row must be back
            if len(self.available_rows) != self.fork_rows_total:
                raise RuntimeError("cannot finish LoopSpec with active branch rows")
            self.finished = True

    # --- queries -------------------------------------------------------------
    def owned(self, branch_id: int) -> dict[str, dict[int, list[int]]]:
        node = self.nodes[branch_id]
        return {role: {stage: list(c.owned) for stage, c in node.cursors[role].items()} for role in ROLES}
