"""The constructed rows of tests/candidates.py take the path they are built
for (CPU only; the GPU tests feed the same rows through the kernels)."""

import numpy as np

from tests import candidates


def test_constructed_rows_take_each_path():
    rows = candidates.repair_rows()
    assert candidates.row_path(rows["repair"], 1.0, 0.9) == "repair"
    assert candidates.row_path(rows["slow"], 1.0, 0.9) == "slow"
    assert candidates.row_path(rows["rebuild"], 1.0, 0.9) == "rebuild"
    assert candidates.row_path(rows["rebuild"][::-1].copy(), 1.0, 0.9) == "rebuild"


def test_typical_rows_are_fast():
    rng = np.random.default_rng(0)
    for _ in range(2):
        x = (rng.standard_normal(49152) * 3).astype(np.float32)
        assert candidates.row_path(x, 1.0, 0.7) == "fast"


def test_flat_rows_are_slow():
    x = np.full(8192, 0.25, dtype=np.float32)  # every entry in exponent bin 0: no candidates
    assert candidates.row_path(x, 1.0, 0.5) == "slow"
