"""Writes the committed fixtures under tests/golden/.

* tiles_*.npz -- the oracle's brute-force tile list (OR over token pairs) for
  each benchmark shape and mask rule, plus the reference topology at H3's
  real shape.
* attn_h2_s600.npz -- dense-masked attention (AxialReference.attend
  semantics) of 2 heads x 600 tokens (ragged) on a fixed 5x5 tile bitmap with
  an empty row, inputs from the seeded splitmix64 generator; the oracle's
  fp32 output stored rounded to bf16.
* prologue_h2_s300.npz -- the fused Q/K RMSNorm + 3D RoPE of a 300-token,
  2-head fused qkv buffer in reference rounding, bf16 bit patterns.

Inputs are regenerated from their seeds (oracle.splitmix_normal_bf16 is
integer-exact), so only outputs are stored. Run from the repo root:
    python tests/golden/make_golden.py
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


ATTN = dict(heads=2, seq_len=600, seeds=(11, 12, 13))
PROLOGUE = dict(heads=2, prefix_len=12, frames=4, height=6, width=12, seed=21, gamma_seed=22,
                eps=1e-6, theta=1e4, dims=(32, 48, 48))


def attn_bitmap() -> np.ndarray:
    """5x5 tiles: a fixed pattern with every diagonal tile but row 2 empty."""
    n = 5
    bm = np.zeros((n, n), dtype=np.uint8)
    for i in range(n):
        for j in range(n):
            bm[i, j] = 1 if (i == j or (3 * i + 5 * j) % 7 < 3) else 0
    bm[2] = 0
    return bm


def attn_inputs():
    H, S = ATTN["heads"], ATTN["seq_len"]
    return [O.splitmix_normal_bf16((H, S, 128), s) for s in ATTN["seeds"]]


def attn_expected() -> np.ndarray:
    q, k, v = (O.bf16_to_f32(t) for t in attn_inputs())
    return O.attend_masked(q, k, v, 1.0 / np.sqrt(128.0), attn_bitmap(), tile=128)


def prologue_inputs():
    P = PROLOGUE
    S = P["prefix_len"] + P["frames"] * P["height"] * P["width"]
    inner = P["heads"] * 128
    qkv = O.splitmix_normal_bf16((S, 3 * inner), P["seed"])
    u = O.splitmix_uniform((2, 128), P["gamma_seed"])
    gq, gk = (O.f32_to_bf16((0.9 + 0.2 * u[i]).astype(np.float32)) for i in range(2))
    pos = O.positions_grid(P["prefix_len"], P["frames"], P["height"], P["width"])
    ax, inv = O.rope_pairs_axes(P["theta"], *P["dims"])
    return S, inner, qkv, gq, gk, pos, ax, inv


def prologue_expected():
    S, inner, qkv, gq, gk, pos, ax, inv = prologue_inputs()
    H = PROLOGUE["heads"]
    eps = PROLOGUE["eps"]
    q = O.qk_norm_rope(qkv, 3 * inner, S, S, H, 128, gq, eps, pos, ax, inv, 128)
    k = O.qk_norm_rope(np.ascontiguousarray(qkv[:, inner:2 * inner]), inner, S, S, H, 128, gk, eps,
                       pos, ax, inv, 128)
    return q, k


def main():
    out = attn_expected()
    np.savez_compressed(os.path.join(OUT, "attn_h2_s600.npz"), out_bf16=O.f32_to_bf16(out),
                        bitmap=attn_bitmap(), seeds=np.array(ATTN["seeds"], dtype=np.int32))
    print(f"attention golden: {out.shape}, bitmap rows {attn_bitmap().sum(axis=1).tolist()}")
    q, k = prologue_expected()
    np.savez_compressed(os.path.join(OUT, "prologue_h2_s300.npz"), q=q, k=k)
    print(f"prologue golden: q {q.shape} k {k.shape}")
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
