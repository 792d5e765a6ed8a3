"""The committed tile-list fixtures are what the oracle's brute force gives,
and carry the counts the rules are documented with."""
import glob
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden  # noqa: E402

EXPECTED_NNZ = {
    "cfg1_band_4x32x32": 183,          # closed form: band +-2 + column 0 on 32x32
    "cfg2_864x480x7s": 3204,
    "cfg3_1344x768x5s": 7854,
    "cfg3_1344x768x5s_frame0": 9691,
    "cfg4_dense_864x480x7s": 142 * 142,
    "axial_h3_864x480x124": 10815,
}


def load(name):
    z = np.load(os.path.join(HERE, "golden", f"tiles_{name}.npz"))
    return z["row_ptr"], z["col_idx"].astype(np.int32), int(z["seq_len"])


def test_fixture_set_is_complete():
    names = sorted(os.path.basename(p)[6:-4] for p in glob.glob(os.path.join(HERE, "golden", "tiles_*.npz")))
    assert names == sorted(EXPECTED_NNZ)


@pytest.mark.parametrize("name,kw", list(make_golden.rules()))
def test_fixture_matches_oracle(orc, name, kw):
    row_ptr, col_idx, seq_len = load(name)
    assert seq_len == kw["seq_len"]
    bm = orc.tile_bitmap(orc.Rule(**kw))
    rp, ci = orc.csr(bm)
    assert np.array_equal(rp, row_ptr) and np.array_equal(ci, col_idx)
    assert len(col_idx) == EXPECTED_NNZ[name]
