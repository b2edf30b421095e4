"""CPU tests of the pipeline interface types (loopspec_amd.loopspec.pipeline):
the schedule's endpoint geometry and its rejection of invalid S/K/X as
pipeline.py:132-146 states, and the lane defaults.
"""

import pytest

from loopspec_amd.loopspec.pipeline import PipelineLane, PipelineSchedule


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


def test_lane_defaults():
    lane = PipelineLane(stage=0, index=1, token=3)
    assert lane.first_token is None and lane.second_state is None and lane.branch == 0
