"""CPU tests of the pipeline restatement (loopspec_amd.loopspec.pipeline).

Pinned by what the reference's pipeline must guarantee: whatever the
proposals, the committed sequence equals the autoregressive decode of the
final readout (greedy losslessness), accepted proposals shorten the work, and
the schedule rejects invalid S/K/X exactly as pipeline.py:132-146 states.
"""

import pytest

from loopspec_amd.loopspec.pipeline import (PipelineLane, PipelineResult, PipelineSchedule,
                                            continue_pipelined)


def test_schedule_validation_and_shapes():
    s = PipelineSchedule(8, 2)
    assert (s.depth, s.proposal_stage, s.second_stage) == (4, 1, None)
    assert s.endpoint_kinds == {1: "q1", 7: "final"}
    assert s.max_rows == 4
    q = PipelineSchedule(12, 2, 3)
    assert q.second_stage == 5 and q.endpoint_stages == (1, 5, 11)
    assert q.row_birth_sizes == [1, 1, 1, 2, 3, 4]
    for bad in ((0, 1), (8, 3), (8, 8), (8, 0)):
        with pytest.raises(ValueError):
            PipelineSchedule(*bad)
    for x in (1, 4, 5):
        with pytest.raises(ValueError):
            PipelineSchedule(8, 2, x)


class ToyExecutor:
    """Final readout = model(token) exactly; q1/q2 readouts = model(token) or a
    deliberately wrong token, chosen by a fixed pattern."""

    def __init__(self, schedule, model, wrong_q1, wrong_q2=None):
        self.schedule = schedule
        self.model = model
        self.wrong_q1 = wrong_q1
        self.wrong_q2 = wrong_q2
        self.forwards = 0
        self.retained = []

    def should_stop(self, ids):
        return False

    def forward(self, lanes):
        self.forwards += 1
        out = []
        k = self.schedule.step_size
        for lane in lanes:
            end = lane.stage + k - 1
            truth = self.model(lane.token, lane.index)
            if end == self.schedule.proposal_stage:
                pred = truth if not self.wrong_q1(lane.index) else truth + 1
                out.append(PipelineResult(state=0, prediction=pred, proposed=True))
            elif end == self.schedule.second_stage:
                wrong = self.wrong_q2 is not None and self.wrong_q2(lane.index)
                pred = truth if not wrong else truth + 2
                proposed = pred != lane.first_token
                out.append(PipelineResult(state=0, prediction=pred, proposed=proposed,
                                          proposal_action="argmax" if proposed else None))
            elif end == self.schedule.stages - 1:
                acc = None
                if lane.first_token == truth:
                    acc = self.schedule.proposal_stage
                elif lane.second_token == truth:
                    acc = self.schedule.second_stage
                out.append(PipelineResult(state=0, prediction=truth, accepted_stage=acc))
            else:
                out.append(PipelineResult(state=0, prediction=-1))
        return out

    def retain_branches(self, lanes, accepted_stage=None):
        self.retained.append((len(lanes), accepted_stage))


def model(token, index):
    return (token * 31 + index * 7) % 1000


def reference_decode(first, n):
    seq = [first]
    while len(seq) < n:
        seq.append(model(seq[-1], len(seq)))
    return seq


@pytest.mark.parametrize("pattern", ["all_right", "all_wrong", "alternate", "every_third"])
@pytest.mark.parametrize("sched", [(8, 2, None), (12, 3, None), (12, 2, 3)])
def test_committed_sequence_is_autoregressive(pattern, sched):
    wrong = {"all_right": lambda i: False, "all_wrong": lambda i: True,
             "alternate": lambda i: i % 2 == 0, "every_third": lambda i: i % 3 == 0}[pattern]
    s = PipelineSchedule(*sched)
    ex = ToyExecutor(s, model, wrong, wrong_q2=(lambda i: i % 2 == 1) if sched[2] else None)
    out = continue_pipelined(5, 40, ex)
    assert out == reference_decode(5, 40)
    if pattern == "all_right":
        # Perfect proposals: one committed token per cycle after the pipeline fills.
        assert ex.forwards <= 40 + s.depth
    if pattern == "all_wrong" and sched[2] is None:
        # Every proposal rejected: each token costs a full depth of cycles.
        assert ex.forwards >= 39 * s.depth


def test_budget_of_one_releases_branches():
    s = PipelineSchedule(8, 2)
    ex = ToyExecutor(s, model, lambda i: False)
    assert continue_pipelined(9, 1, ex) == [9]
    assert ex.retained == [(0, None)]
    with pytest.raises(ValueError):
        continue_pipelined(9, 0, ex)


def test_lane_defaults():
    lane = PipelineLane(stage=0, index=1, token=3)
    assert lane.first_token is None and lane.second_state is None and lane.branch == 0
