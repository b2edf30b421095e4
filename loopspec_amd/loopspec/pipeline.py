"""Interface types of LoopSpec's logical pipeline that the decision policies
take and return (sglang_recurrent/loopspec/pipeline.py:13-207): lanes, lane
results, the executor protocol and the schedule's endpoint geometry.

The pipeline's commit loop itself (pipeline.py:254-423) is host control flow
and is not part of this package: its accept-prefix rule over k sequential
draft positions is what the batched verify entry points compute on the GPU.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Protocol, Sequence


@dataclass
class PipelineLane:
    """A token in flight: its stage, position, branch ancestry and the q1 / q2
    proposals (token and distribution) recorded on its way (pipeline.py:13-43)."""

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
    """What one forward returns for a lane (pipeline.py:46-59)."""

    state: int
    prediction: int
    proposed: bool = False
    proposal_state: Any = None
    accepted_stage: int | None = None
    proposal_action: str | None = None


class PipelineExecutor(Protocol):
    """The model-side boundary a pipeline drives (pipeline.py:62-86)."""

    schedule: "PipelineSchedule"

    def should_stop(self, output_ids: Sequence[int]) -> bool: ...

    def forward(self, lanes: Sequence[PipelineLane]) -> Sequence[PipelineResult]: ...

    def retain_branches(self, lanes: Sequence[PipelineLane], accepted_stage: int | None = None) -> None: ...


@dataclass(frozen=True)
class PipelineSchedule:
    """S recurrent iterations per token (`stages`), K per cycle (`step_size`),
    and an optional second readout after K X iterations (`second_step`);
    pipeline.py:124-207 defines the same quantities."""

    stages: int
    step_size: int
    second_step: int | None = None

    def __post_init__(self) -> None:
        s, k, x = self.stages, self.step_size, self.second_step
        if type(s) is not int or s < 1:
            raise ValueError(f"PipelineSchedule: stages must be an int >= 1 (got {s!r})")
        if type(k) is not int or not (0 < k < s) or s % k != 0:
            raise ValueError(f"PipelineSchedule: step_size must divide stages and be below it (got {k!r} for {s})")
        if x is not None and (type(x) is not int or not (1 < x < s // k)):
            raise ValueError(f"PipelineSchedule: second_step must lie strictly between 1 and "
                             f"stages / step_size = {s // k} (got {x!r})")

    @property
    def depth(self) -> int:
        """Cycles a lane needs to reach its final readout."""
        return self.stages // self.step_size

    @property
    def proposal_stage(self) -> int:
        """Last iteration (0-based) before the q1 readout."""
        return self.step_size - 1

    @property
    def second_stage(self) -> int | None:
        """Last iteration before the q2 readout, if there is one."""
        return None if self.second_step is None else self.second_step * self.step_size - 1

    @property
    def endpoint_kinds(self) -> dict[int, str]:
        """Readout iteration -> 'q1' / 'q2' / 'final'."""
        kinds = {self.proposal_stage: "q1", self.stages - 1: "final"}
        if self.second_step is not None:
            kinds[self.second_stage] = "q2"
        return kinds

    @property
    def endpoint_stages(self) -> tuple[int, ...]:
        return tuple(sorted(self.endpoint_kinds))

    @property
    def row_birth_sizes(self) -> list[int]:
        """Lanes born at stage zero at each time step 0 .. depth-1 in the full
        tree: one per step, and with a second readout after X cycles, from step
        X on, the previous step's births plus those X steps back."""
        x = self.second_step
        births: list[int] = []
        for t in range(self.depth):
            births.append(1 if x is None or t < x else births[t - 1] + births[t - x])
        return births

    @property
    def max_rows(self) -> int:
        """Bound on the lanes alive at once."""
        return sum(self.row_birth_sizes)
