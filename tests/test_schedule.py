"""The persistent attention schedule (h3hip_schedule, the lists
h3hip_plan_create uploads) on the host: every (head, q-tile) unit of a plan
is listed exactly once, for the committed CSR lists of every benchmark shape
and for several CU counts, and each XCD's workgroups carry comparable work."""
import os

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")

SHAPES = [("tiles_cfg1_band_4x32x32.npz", 4), ("tiles_cfg2_864x480x7s.npz", 40),
          ("tiles_cfg3_1344x768x5s.npz", 40), ("tiles_cfg3_1344x768x5s_frame0.npz", 40),
          ("tiles_cfg4_dense_864x480x7s.npz", 40), ("tiles_axial_h3_864x480x124.npz", 56)]


def _units(work):
    return (work >> 16).astype(np.int64), (work & 0xFFFF).astype(np.int64)


@pytest.mark.parametrize("name,heads", SHAPES)
@pytest.mark.parametrize("groups", [8, 64, 256, 304])
def test_every_unit_exactly_once(h3, name, heads, groups):
    row_ptr = np.load(os.path.join(GOLDEN, name))["row_ptr"]
    n = len(row_ptr) - 1
    work_ptr, work = h3.schedule(row_ptr, heads, groups)
    assert work_ptr[0] == 0 and work_ptr[-1] == heads * n
    assert np.all(np.diff(work_ptr) >= 0)
    h, qt = _units(work)
    assert np.all((h >= 0) & (h < heads) & (qt >= 0) & (qt < n))
    ids = np.sort(h * n + qt)
    assert np.array_equal(ids, np.arange(heads * n))


@pytest.mark.parametrize("name,heads", SHAPES[1:4])
def test_workgroups_balanced(h3, name, heads):
    """Cost per workgroup (tiles + 2 per unit, the schedule's own model) within
    12% of the mean at the benchmark shapes on 256 workgroups."""
    row_ptr = np.load(os.path.join(GOLDEN, name))["row_ptr"]
    work_ptr, work = h3.schedule(row_ptr, heads, 256)
    lens = np.diff(row_ptr)
    cost = np.array([sum(lens[u & 0xFFFF] + 2 for u in work[work_ptr[b]:work_ptr[b + 1]])
                     for b in range(256)], dtype=np.float64)
    assert cost.max() <= 1.12 * cost.mean(), (cost.max(), cost.mean())


def test_single_row_and_empty_rows(h3):
    row_ptr = np.array([0, 0, 3, 3, 4], dtype=np.int32)
    work_ptr, work = h3.schedule(row_ptr, 3, 8)
    h, qt = _units(work)
    assert sorted(zip(h.tolist(), qt.tolist())) == [(a, b) for a in range(3) for b in range(4)]


def test_refusals(h3):
    with pytest.raises(h3.H3HIPError):
        h3.schedule(np.array([0, 2, 1], dtype=np.int32), 2, 8)      # not monotone
    with pytest.raises(h3.H3HIPError):
        h3.schedule(np.array([0, 1], dtype=np.int32), 2, 12)        # groups % 8
    with pytest.raises(h3.H3HIPError):
        h3.schedule(np.array([1, 2], dtype=np.int32), 2, 8)         # row_ptr[0] != 0
