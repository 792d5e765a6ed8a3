"""Seeded random cases of block-sparse attention against the oracle, in full.

Each case draws, from its own seed: the number of 128-row tiles (1-12) and a
sequence length inside the last one (ragged), the head count (1-4), a tile
bitmap of random density with some rows emptied, the score scale, a
magnitude for Q and K (up to 3, so scores span hundreds of units in log2 and
the lazy rescale fires; V stays N(0, 1), the scale the bar is set for),
garbage in the padding rows, and the output layout. Every
output row of every head is compared with the dense-masked fp32 oracle
(AxialReference.attend semantics, AxialReference.swift:89-114) at the
north-star bar, rows with no active tile must be exactly zero, and padding
rows of a head-major output must be zero.
"""
import math

import numpy as np
import pytest
import torch

from _gpu import err_stats, f32, note, randn_bf16_gpu

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def _case(seed):
    rng = np.random.default_rng(1000 + seed)
    n = int(rng.integers(1, 13))
    S = int((n - 1) * 128 + rng.integers(1, 129))
    H = int(rng.integers(1, 5))
    density = float(rng.choice([0.05, 0.2, 0.5, 1.0]))
    bm = (rng.random((n, n)) < density).astype(np.uint8)
    if n > 2:
        bm[rng.choice(n, size=int(rng.integers(0, 3)), replace=False)] = 0
    scale = float(rng.choice([0.05, 1.0 / math.sqrt(128), 0.125, 0.5, 1.0]))
    magnitude = float(rng.choice([1.0, 2.0, 3.0]))
    pad = float(rng.choice([0.0, float("nan"), 1e4]))
    layout = int(rng.integers(0, 2))
    return n, S, H, bm, scale, magnitude, pad, layout


@pytest.mark.parametrize("seed", range(16))
def test_random_case_against_oracle(h3, orc, seed):
    from h3hip import ops
    n, S, H, bm, scale, magnitude, pad, layout = _case(seed)
    note(f"random attention seed={seed} n={n} S={S} H={H} density={bm.mean():.2f} "
         f"scale={scale:.3f} magnitude={magnitude} pad={pad} layout={layout}")
    plan = h3.TilePlan(h3.MaskRule.from_bitmap(S, bm), heads=H)
    S_pad = plan.seq_pad
    q, k = (randn_bf16_gpu((H, S_pad, 128), 50 * seed + i, magnitude) for i in range(2))
    v = randn_bf16_gpu((H, S_pad, 128), 50 * seed + 2)
    if S_pad > S:
        for t in (q, k, v):
            t[:, S:] = pad
    out = ops.bsattn_fwd(plan, q, k, v, scale, out_layout=layout)
    torch.cuda.synchronize()
    o = f32(out)
    if layout == 1:   # token-major [S_pad, H*128] -> [H, S_pad, 128]
        o = o.reshape(S_pad, H, 128).transpose(1, 0, 2)
    assert np.all(np.isfinite(o[:, :S]))
    if layout == 0:
        assert np.all(o[:, S:] == 0)
    empty = np.flatnonzero(bm.sum(axis=1) == 0)
    for t in empty:
        assert np.all(o[:, t * 128:min((t + 1) * 128, S)] == 0), t
    want = orc.attend_masked(f32(q)[:, :S], f32(k)[:, :S], f32(v)[:, :S], scale, bm, tile=128)
    mx, mean = err_stats(o[:, :S], want)
    print(f"seed {seed}: max-abs {mx:.3e} mean-abs {mean:.3e}")
    assert mx < MAX_ABS and mean < MEAN_ABS
