"""Edge cases of the block-sparse attention against the dense-masked oracle
(AxialReference.attend semantics, AxialReference.swift:89-114), at the bar of
the north star (max-abs 2e-2, mean-abs 2e-3 of the fp32 reference):

- sequence lengths at and around the 128-row tile boundary, down to a single
  token, with one and with three heads (padding rows come back zero);
- large-magnitude scores whose running maximum keeps rising from tile to
  tile, so the online softmax (AxialReference.swift:129-171) takes its
  rescale branch over and over, including the lazy raise past 2^8;
- rows whose first (or only) key tile is the ragged last one with <= 64
  valid keys, so one 64-key half of the wave pair sees padding only, at the
  scales the public ABI accepts (a finite padding sentinel turned into an
  infinite weight there for most scales).
"""
import math

import numpy as np
import pytest
import torch

from _gpu import err_stats, f32, head_major_inputs, note

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def _dense_case(h3, orc, S, H, seed, q_scale=1.0, k_ramp=0.0, scale=None, bitmap=None):
    from h3hip import ops
    rule = h3.MaskRule.dense(S) if bitmap is None else h3.MaskRule.from_bitmap(S, bitmap)
    plan = h3.TilePlan(rule, heads=H)
    q, k, v = head_major_inputs(H, S, plan.seq_pad, 128, seed)
    if q_scale != 1.0:
        q = (q.float() * q_scale).to(torch.bfloat16)
        k = (k.float() * q_scale).to(torch.bfloat16)
    if k_ramp:
        # Scores grow with the key index: every later tile holds a larger max.
        ramp = torch.linspace(0, k_ramp, plan.seq_pad, device="cuda")[None, :, None]
        k = (k.float() + ramp * q.float().mean(dim=1, keepdim=True).sign()).to(torch.bfloat16)
        k[:, S:] = 0
    scale = 1.0 / math.sqrt(128) if scale is None else scale
    note(f"edge S={S} H={H} q_scale={q_scale} ramp={k_ramp} scale={scale} "
         f"bitmap={bitmap is not None}")
    out = ops.bsattn_fwd(plan, q, k, v, scale)
    torch.cuda.synchronize()
    n = plan.n_tiles
    bm = np.ones((n, n), dtype=np.uint8) if bitmap is None else bitmap
    qf, kf, vf = (f32(t)[:, :S] for t in (q, k, v))
    want = orc.attend_masked(qf, kf, vf, scale, bm, tile=128)
    o = f32(out)
    assert np.all(np.isfinite(o)) and np.all(o[:, S:] == 0)
    mx, mean = err_stats(o[:, :S], want)
    return mx, mean


@pytest.mark.parametrize("S", [1, 5, 127, 128, 129, 255, 256, 257])
@pytest.mark.parametrize("H", [1, 3])
def test_short_and_boundary_lengths(h3, orc, S, H):
    mx, mean = _dense_case(h3, orc, S, H, seed=S + 10 * H)
    assert mx < MAX_ABS and mean < MEAN_ABS, (S, H, mx, mean)


@pytest.mark.parametrize("q_scale,ramp", [(6.0, 0.0), (1.0, 6.0), (4.0, 4.0)])
def test_rising_maxima_force_rescales(h3, orc, q_scale, ramp):
    """Scores with a spread of hundreds in log2 units and maxima that rise
    across the key tiles: the lazy rescale fires repeatedly and the result
    still matches the fp32 reference."""
    mx, mean = _dense_case(h3, orc, 900, 2, seed=17, q_scale=q_scale, k_ramp=ramp)
    print(f"q_scale {q_scale} ramp {ramp}: max-abs {mx:.2e} mean-abs {mean:.2e}")
    assert mx < MAX_ABS and mean < MEAN_ABS, (mx, mean)


@pytest.mark.parametrize("scale", [0.088, 0.125, 1.0])
@pytest.mark.parametrize("S", [1, 5, 64, 129, 192, 300])
def test_padding_only_key_half(h3, orc, S, scale):
    """Dense rows at S <= 64 have one tile whose upper 64-key half is all
    padding; S = 129, 192 and 300 put <= 64 valid keys in the last tile after
    real ones. Finite everywhere and within the bar at each scale."""
    mx, mean = _dense_case(h3, orc, S, 2, seed=S + 3, scale=scale)
    assert mx < MAX_ABS and mean < MEAN_ABS, (S, scale, mx, mean)


@pytest.mark.parametrize("scale", [0.088, 0.125, 1.0])
def test_row_whose_only_tile_is_the_ragged_last(h3, orc, scale):
    """A bitmap whose last q-tile attends only the last key tile (40 valid
    keys), and an earlier row that attends only that tile too: the padding
    half is the first thing those rows' second half sees."""
    n = 5
    S = (n - 1) * 128 + 40
    bm = np.zeros((n, n), dtype=np.uint8)
    bm[np.arange(n), np.arange(n)] = 1
    bm[0, :] = 1
    bm[n - 1] = 0
    bm[n - 1, n - 1] = 1
    bm[2] = 0
    bm[2, n - 1] = 1
    mx, mean = _dense_case(h3, orc, S, 3, seed=41, scale=scale, bitmap=bm)
    assert mx < MAX_ABS and mean < MEAN_ABS, (scale, mx, mean)
