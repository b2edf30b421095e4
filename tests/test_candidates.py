"""The constructed rows of tests/candidates.py take the path they are built
for (CPU restatement of the kernels' candidate rule), and the seeded BASELINE
rows take the fast path."""

import collections

import numpy as np

from loopspec_amd import workloads
from tests import candidates


def test_constructed_rows_take_their_paths():
    for name, (row, top_p) in candidates.path_rows().items():
        assert candidates.row_path(row, top_p) == name
    row, top_p = candidates.path_rows()["refill"]
    assert candidates.row_path(row[::-1].copy(), top_p) == "refill"
    assert candidates.row_path(row, 1.0) == "unfiltered"


def test_all_equal_chunks_overflow():
    x = np.full(8192, 0.25, dtype=np.float32)  # every element ties at every chunk's max
    assert candidates.row_path(x, 0.5) == "slow_dense"


def test_baseline_rows_take_the_fast_path():
    for cfg, epv in ((workloads.C3, 4), (workloads.C4, 8)):
        inp = workloads.sampling_inputs(cfg, 0)
        paths = collections.Counter()
        for b in range(3):
            for r in range(cfg.k + 1):
                paths[candidates.row_path(inp["target"][b, r].float().numpy(), cfg.top_p, cfg.temperature, epv)] += 1
            for r in range(cfg.k):
                paths[candidates.row_path(inp["draft"][b, r].float().numpy(), cfg.top_p, cfg.temperature, epv)] += 1
        assert set(paths) == {"fast"}, (cfg.name, dict(paths))
