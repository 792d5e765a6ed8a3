"""The committed fixtures: tile lists are what the oracle's brute force gives
and carry the counts the rules are documented with; the attention and
prologue output vectors are what the oracle computes from their seeded,
bit-stable inputs (so a change to the oracle that moves them is caught)."""
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
    for f in ("attn_h2_s600.npz", "prologue_h2_s300.npz"):
        assert os.path.exists(os.path.join(HERE, "golden", f))


def test_splitmix64_known_answer(orc):
    """splitmix64's published first outputs for seed 0."""
    got = [int(x) for x in orc.splitmix64(0, 3)]
    assert got == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    x = orc.bf16_to_f32(orc.splitmix_normal_bf16((200000,), 3))
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1.0) < 0.01
    assert float(np.abs(x).max()) <= 2.0 * np.sqrt(3.0)


def test_attention_golden_is_what_the_oracle_computes(orc):
    z = np.load(os.path.join(HERE, "golden", "attn_h2_s600.npz"))
    assert np.array_equal(z["bitmap"], make_golden.attn_bitmap())
    want = orc.bf16_to_f32(z["out_bf16"])
    got = make_golden.attn_expected()
    assert np.all(got[:, 256:384] == 0)                      # the empty tile row
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -8 + 1e-7)


def test_prologue_golden_is_bit_identical(orc):
    z = np.load(os.path.join(HERE, "golden", "prologue_h2_s300.npz"))
    q, k = make_golden.prologue_expected()
    assert np.array_equal(q, z["q"]) and np.array_equal(k, z["k"])


@pytest.mark.parametrize("name,kw", list(make_golden.rules()))
def test_fixture_matches_oracle(orc, name, kw):
    row_ptr, col_idx, seq_len = load(name)
    assert seq_len == kw["seq_len"]
    bm = orc.tile_bitmap(orc.Rule(**kw))
    rp, ci = orc.csr(bm)
    assert np.array_equal(rp, row_ptr) and np.array_equal(ci, col_idx)
    assert len(col_idx) == EXPECTED_NNZ[name]
