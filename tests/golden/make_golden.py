"""Writes the committed tile-list fixtures under tests/golden/.

Each fixture is the oracle's brute-force tile list (OR over token pairs) for
one benchmark shape and mask rule, plus the reference topology at H3's real
shape. Run from the repo root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "minimax-h3-swift_amd")]
import oracle as O  # noqa: E402
from h3hip import configs as C  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))

# The reference's topology at its production shape: 864x480x124 with the
# 746-token prefix of AxialReferenceTests.mismatchedGeometryRefused (:162-174),
# 37 x 15 x 27 video lattice, landmarks [0, 18, 36] (:176-193).
AXIAL_H3 = dict(kind=O.RULE_AXIAL, seq_len=15731, prefix_len=746, frames=37, height=15,
                width=27, landmarks=[0, 18, 36])


def rules():
    for name in ("cfg1_band_4x32x32", "cfg2_864x480x7s", "cfg3_1344x768x5s",
                 "cfg3_1344x768x5s_frame0", "cfg4_dense_864x480x7s"):
        yield name, C.ALL[name].oracle_rule_kwargs()
    yield "axial_h3_864x480x124", AXIAL_H3


def main():
    for name, kw in rules():
        r = O.Rule(**kw)
        bm = O.tile_bitmap(r)
        row_ptr, col_idx = O.csr(bm)
        path = os.path.join(OUT, f"tiles_{name}.npz")
        np.savez_compressed(path, row_ptr=row_ptr, col_idx=col_idx.astype(np.int16),
                            seq_len=np.int32(kw["seq_len"]))
        print(f"{name}: S={kw['seq_len']} tiles={bm.shape[0]}^2 nnz={len(col_idx)} "
              f"density={len(col_idx) / bm.size:.4f} -> {os.path.basename(path)}")


if __name__ == "__main__":
    main()
