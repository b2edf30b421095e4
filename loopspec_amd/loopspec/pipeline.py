"""Logical pipeline of LoopSpec: lanes, results, schedule, and the commit loop.

Host-side data types the decision policies consume, restated from
sglang_recurrent/loopspec/pipeline.py (no tensors are handled here). The loop
``continue_pipelined`` is the reference's acceptance/prune rule
(pipeline.py:254-423): it commits one token per cycle from the lane reaching
final depth, keeps the child whose token and originating readout match the
accepted proposal, and discards every branch that does not descend from it.
Chained over k sequential draft positions this is exactly the accept-prefix
rule the fused verify kernels implement.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Mapping, Protocol, Sequence


@dataclass
class PipelineLane:
    """One input token moving through repeated core iterations (pipeline.py:13-43)."""

    stage: int
    index: int
    token: int
    state: int | None = None
    branch: int = 0
    parent_branch: int | None = None
    origin_stage: int | None = None
    first_token: int | None = None
    first_state: Any = None
    second_token: int | None = None
    second_state: Any = None


@dataclass(frozen=True)
class PipelineResult:
    """One lane's result and optional proposal (pipeline.py:46-59)."""

    state: int
    prediction: int
    proposed: bool = False
    proposal_state: Any = None
    accepted_stage: int | None = None
    proposal_action: str | None = None


class PipelineExecutor(Protocol):
    """Model execution boundary used by continue_pipelined (pipeline.py:62-86)."""

    schedule: "PipelineSchedule"

    def should_stop(self, output_ids: Sequence[int]) -> bool: ...

    def forward(self, lanes: Sequence[PipelineLane]) -> Sequence[PipelineResult]: ...

    def retain_branches(self, lanes: Sequence[PipelineLane], accepted_stage: int | None = None) -> None: ...


@dataclass(frozen=True)
class PipelineSchedule:
    """S total iterations, K per cycle, optional q2 after K*X (pipeline.py:132-207)."""

    stages: int
    step_size: int
    second_step: int | None = None

    def __post_init__(self) -> None:
        if not isinstance(self.stages, int) or self.stages <= 0:
            raise ValueError(f"stages S must be a positive integer, got {self.stages}")
        k = self.step_size
        if not isinstance(k, int) or not 1 <= k < self.stages or self.stages % k:
            raise ValueError(f"step_size K must be a positive divisor of S with K < S; got K={k}, S={self.stages}")
        x = self.second_step
        if x is not None and (not isinstance(x, int) or not 1 < x < self.depth):
            raise ValueError(f"second_step X must satisfy 1 < X < S/K so K*X < S; got X={x}, S/K={self.depth}")

    @property
    def depth(self) -> int:
        return self.stages // self.step_size

    @property
    def proposal_stage(self) -> int:
        return self.step_size - 1

    @property
    def second_stage(self) -> int | None:
        return None if self.second_step is None else self.step_size * self.second_step - 1

    @property
    def endpoint_kinds(self) -> dict[int, str]:
        kinds = {self.proposal_stage: "q1"}
        if self.second_stage is not None:
            kinds[self.second_stage] = "q2"
        kinds[self.stages - 1] = "final"
        return kinds

    @property
    def endpoint_stages(self) -> tuple[int, ...]:
        return tuple(sorted(self.endpoint_kinds))

    @property
    def row_birth_sizes(self) -> list[int]:
        """New stage-zero lanes per time step: 1 each, or b_t = b_(t-1) + b_(t-X) with q2."""
        if self.second_step is None:
            return [1] * self.depth
        births = [1] * self.second_step
        for t in range(self.second_step, self.depth):
            births.append(births[t - 1] + births[t - self.second_step])
        return births

    @property
    def max_rows(self) -> int:
        return sum(self.row_birth_sizes)


def _descends_from(branch: int | None, ancestor: int, parents: Mapping[int, int | None]) -> bool:
    while branch is not None and branch != ancestor:
        branch = parents.get(branch)
    return branch == ancestor


def _prune_ancestry(lanes: Sequence[PipelineLane], root: int,
                    parents: Mapping[int, int | None]) -> dict[int, int | None]:
    live = {root}
    for lane in lanes:
        b = lane.branch
        while b != root:
            if b is None or b not in parents:
                raise RuntimeError("pipeline branch escaped the selected ancestry")
            live.add(b)
            b = parents[b]
    return {b: None if b == root else parents[b] for b in live}


def continue_pipelined(first_token: int, max_new_tokens: int, executor: PipelineExecutor) -> list[int]:
    """Committed completion ids, first token included (pipeline.py:254-423)."""
    if max_new_tokens <= 0:
        raise ValueError("a committed first token requires a positive budget")
    sched = executor.schedule
    proposal_stages = {sched.proposal_stage, sched.second_stage} - {None}
    final_stage = sched.stages - 1
    committed = [first_token]
    if max_new_tokens == 1:
        executor.retain_branches(())
        return committed
    next_branch = 1
    parents: dict[int, int | None] = {0: None}
    lanes = [PipelineLane(stage=0, index=1, token=first_token)]
    while len(committed) < max_new_tokens:
        results = list(executor.forward(lanes))
        if len(results) != len(lanes):
            raise ValueError("executor must return one result per lane")
        following: list[PipelineLane] = []
        children: list[PipelineLane] = []
        final: tuple[PipelineLane, PipelineResult] | None = None
        accepted_stage: int | None = None
        for lane, result in zip(lanes, results):
            end = lane.stage + sched.step_size - 1
            if end == final_stage:
                if final is not None:
                    raise RuntimeError("multiple branches reached the final stage")
                final = (lane, result)
                continue
            lane.stage = end + 1
            lane.state = result.state
            if end in proposal_stages and result.proposed:
                if end == sched.proposal_stage:
                    lane.first_token, lane.first_state = result.prediction, result.proposal_state
                elif result.proposal_action in ("residual", "argmax"):
                    lane.second_token, lane.second_state = result.prediction, result.proposal_state
                else:
                    raise RuntimeError("q2 proposal has no branch action")
                if lane.index + 1 < max_new_tokens:
                    children.append(PipelineLane(stage=0, index=lane.index + 1, token=result.prediction,
                                                 branch=next_branch, parent_branch=lane.branch, origin_stage=end))
                    parents[next_branch] = lane.branch
                    next_branch += 1
            following.append(lane)
        following.extend(children)
        if final is not None:
            lane, result = final
            if lane.index != len(committed):
                raise RuntimeError("pipeline attempted to commit out of order")
            committed.append(result.prediction)
            if executor.should_stop(committed):
                executor.retain_branches(())
                return committed
            if lane.index + 1 < max_new_tokens:
                selected = next((c for c in following if c.parent_branch == lane.branch
                                 and c.token == result.prediction and c.origin_stage == result.accepted_stage), None)
                if selected is None:
                    selected = PipelineLane(stage=0, index=lane.index + 1, token=result.prediction,
                                            branch=next_branch, parent_branch=lane.branch, origin_stage=final_stage)
                    parents[next_branch] = lane.branch
                    next_branch += 1
                    following.append(selected)
                accepted_stage = result.accepted_stage
                keep = selected.branch
                following = [c for c in following if _descends_from(c.branch, keep, parents)]
                parents = _prune_ancestry(following, keep, parents)
            else:
                following = []
        if len(following) > sched.max_rows:
            raise RuntimeError("speculative tree exceeded branch row limit")
        lanes = following
        executor.retain_branches(tuple(lanes), accepted_stage)
        if not lanes and len(committed) < max_new_tokens:
            raise RuntimeError("pipeline drained before generation completed")
    return committed
