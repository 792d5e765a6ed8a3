"""Pins the oracle's topology and tile lists (CPU only).

Mirrors Tests/H3AttentionTests/AxialReferenceTests.swift: the known-answer
tokens of topologyIsWhatItClaims (:119-143), the counted-vs-closed-form
density (:145-160), landmark placement (:176-193) and the bulk-vs-pairwise
check (:99-117), carried to tile bitmaps. A pure-Python restatement of each
rule is the independent side of the pairwise checks.
"""
import itertools

import numpy as np
import pytest


def fixture_rule(orc, prefix=7, frames=5, h=3, w=4, landmarks=None, tile=128, kind=None):
    landmarks = [0, frames - 1] if landmarks is None else landmarks
    return orc.Rule(orc.RULE_AXIAL if kind is None else kind, prefix + frames * h * w, tile=tile,
                    prefix_len=prefix, frames=frames, height=h, width=w, landmarks=landmarks)


def py_allows_axial(q, k, prefix, frames, h, w, landmarks):
    s = prefix + frames * h * w
    if not (0 <= q < s and 0 <= k < s):
        return False
    if q < prefix or k < prefix:
        return True
    fq, rq = divmod(q - prefix, h * w)
    fk, rk = divmod(k - prefix, h * w)
    return fq == fk or rq == rk or fk in landmarks


def py_allows_local(q, k, prefix, frames, h, w, fw, sp, sw, landmarks):
    s = prefix + frames * h * w
    if not (0 <= q < s and 0 <= k < s):
        return False
    if q < prefix or k < prefix:
        return True
    fq, rq = divmod(q - prefix, h * w)
    fk, rk = divmod(k - prefix, h * w)
    yq, xq = divmod(rq, w)
    yk, xk = divmod(rk, w)
    if (abs(fq - fk) <= fw and abs(yq // sp[0] - yk // sp[0]) <= sw
            and abs(xq // sp[1] - xk // sp[1]) <= sw):
        return True
    return fk in landmarks


def test_topology_is_what_it_claims(orc):
    # AxialReferenceTests.swift:119-143, token for token.
    t = fixture_rule(orc)
    q = 7 + 2 * 12 + 1 * 4 + 2
    assert q == 37
    assert orc.allows(t, q, 3)                       # prefix
    assert orc.allows(t, q, 7 + 2 * 12 + 0)          # same frame
    assert orc.allows(t, q, 7 + 4 * 12 + 1 * 4 + 2)  # same column
    assert orc.allows(t, q, 7 + 0 * 12 + 5)          # landmark 0
    assert orc.allows(t, q, 7 + 4 * 12 + 5)          # landmark 4
    assert not orc.allows(t, q, 7 + 1 * 12 + 0 * 4 + 0)
    assert all(orc.allows(t, 0, k) for k in range(67))


def test_pairwise_matches_python_restatement(orc):
    t = fixture_rule(orc)
    for q, k in itertools.product(range(67), range(67)):
        assert orc.allows(t, q, k) == py_allows_axial(q, k, 7, 5, 3, 4, [0, 4]), (q, k)
    loc = orc.Rule(orc.RULE_LOCAL, 7 + 6 * 5 * 7, prefix_len=7, frames=6, height=5, width=7,
                   frame_window=1, sp_tile=(2, 3), sp_window=1, landmarks=[2])
    for q, k in itertools.product(range(loc.seq_len), range(loc.seq_len)):
        assert orc.allows(loc, q, k) == py_allows_local(q, k, 7, 6, 5, 7, 1, (2, 3), 1, [2]), (q, k)


def test_density_is_counted_not_estimated(orc):
    # AxialReferenceTests.swift:145-160: closed form vs counted, < 1e-9.
    t = fixture_rule(orc, frames=6)
    assert abs(orc.token_density_counted(t) - orc.axial_density_closed(t)) < 1e-9
    t3 = fixture_rule(orc, prefix=11, frames=9, h=4, w=5, landmarks=orc.landmarks(9, 3))
    assert abs(orc.token_density_counted(t3) - orc.axial_density_closed(t3)) < 1e-9


def test_landmark_placement(orc):
    # AxialReferenceTests.swift:176-193 (37 latent frames at 864x480x124).
    assert orc.landmarks(37, 3) == [0, 18, 36]
    assert orc.landmarks(37, 1) == [0, 36]
    assert orc.landmarks(37, 999) == list(range(37))
    lm = orc.landmarks(10, 4)
    assert lm[0] == 0 and lm[-1] == 9 and len(set(lm)) == len(lm)
    # Half-way rounding is away from zero (Swift .rounded()): 35/2 = 17.5 -> 18.
    assert orc.landmarks(36, 3) == [0, 18, 35]


@pytest.mark.parametrize("tile", [4, 8, 16])
def test_tile_bitmap_is_or_of_pairs(orc, tile):
    """Bulk (tile bitmap) vs the per-pair definition, as the reference checks
    maskRows against allows, at tiles that cut frames and the prefix."""
    for kind in (orc.RULE_AXIAL, orc.RULE_LOCAL):
        if kind == orc.RULE_AXIAL:
            t = fixture_rule(orc, tile=tile)
            pred = lambda q, k: py_allows_axial(q, k, 7, 5, 3, 4, [0, 4])
        else:
            t = orc.Rule(orc.RULE_LOCAL, 7 + 6 * 5 * 7, tile=tile, prefix_len=7, frames=6,
                         height=5, width=7, frame_window=1, sp_tile=(2, 3), sp_window=1)
            pred = lambda q, k: py_allows_local(q, k, 7, 6, 5, 7, 1, (2, 3), 1, [])
        bm = orc.tile_bitmap(t)
        n = bm.shape[0]
        S = t.seq_len
        want = np.zeros((n, n), dtype=np.uint8)
        for q in range(S):
            for k in range(S):
                if pred(q, k):
                    want[q // tile, k // tile] = 1
        assert np.array_equal(bm, want)


def test_band_rule_closed_form(orc):
    """cfg1: band +-2 plus column 0 on 32x32 tiles is exactly 183 tiles, row r
    = {0} U [max(0, r-2), min(31, r+2)]."""
    r = orc.Rule(orc.RULE_BAND, 4096, band=2, global_cols=[0])
    bm = orc.tile_bitmap(r)
    assert bm.sum() == 183
    row_ptr, col_idx = orc.csr(bm)
    for i in range(32):
        want = sorted({0} | set(range(max(0, i - 2), min(31, i + 2) + 1)))
        assert list(col_idx[row_ptr[i]:row_ptr[i + 1]]) == want


def test_csr_invariants(orc):
    rng = np.random.default_rng(3)
    bm = (rng.random((37, 41)) < 0.2).astype(np.uint8)
    bm[5] = 0  # an empty row
    row_ptr, col_idx = orc.csr(bm)
    assert row_ptr[0] == 0 and row_ptr[-1] == bm.sum() == len(col_idx)
    for i in range(37):
        cols = col_idx[row_ptr[i]:row_ptr[i + 1]]
        assert np.all(np.diff(cols) > 0)
        assert np.array_equal(cols, np.nonzero(bm[i])[0])


def test_local_rule_structure(orc):
    """The cfg2/cfg3 local rule: prefix rows and columns dense, symmetric
    without landmarks, diagonal always present; frame-0 landmark only adds."""
    import h3hip.configs as C
    for shape in (C.CFG2,):
        r = orc.Rule(**shape.oracle_rule_kwargs())
        bm = orc.tile_bitmap(r)
        n = bm.shape[0]
        p_tiles = (shape.prefix_len + 127) // 128
        assert bm[:p_tiles].all() and bm[:, :p_tiles].all()
        assert np.array_equal(bm, bm.T)
        assert np.all(np.diag(bm) == 1)
        kw = shape.oracle_rule_kwargs()
        kw["landmarks"] = [0]
        bm0 = orc.tile_bitmap(orc.Rule(**kw))
        assert np.all(bm0 >= bm) and bm0.sum() > bm.sum()
        assert bm.sum() == 3204 and n == 142
