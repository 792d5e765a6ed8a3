"""Edge cases of the block-sparse attention against the dense-masked oracle
(AxialReference.attend semantics, AxialReference.swift:89-114), at the bar of
the north star (max-abs 2e-2, mean-abs 2e-3 of the fp32 reference):

- sequence lengths at and around the 128-row tile boundary, down to a single
  token, with one and with three heads (padding rows come back zero);
- large-magnitude scores whose running maximum keeps rising from tile to
  tile, so the online softmax (AxialReference.swift:129-171) takes its
  rescale branch over and over, including the lazy raise past 2^8.
"""
import math

import numpy as np
import pytest
import torch

from _gpu import err_stats, f32, head_major_inputs, note

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def _dense_case(h3, orc, S, H, seed, q_scale=1.0, k_ramp=0.0):
    from h3hip import ops
    plan = h3.TilePlan(h3.MaskRule.dense(S), heads=H)
    q, k, v = head_major_inputs(H, S, plan.seq_pad, 128, seed)
    if q_scale != 1.0:
        q = (q.float() * q_scale).to(torch.bfloat16)
        k = (k.float() * q_scale).to(torch.bfloat16)
    if k_ramp:
        # Scores grow with the key index: every later tile holds a larger max.
        ramp = torch.linspace(0, k_ramp, plan.seq_pad, device="cuda")[None, :, None]
        k = (k.float() + ramp * q.float().mean(dim=1, keepdim=True).sign()).to(torch.bfloat16)
        k[:, S:] = 0
    scale = 1.0 / math.sqrt(128)
    note(f"edge S={S} H={H} q_scale={q_scale} ramp={k_ramp}")
    out = ops.bsattn_fwd(plan, q, k, v, scale)
    torch.cuda.synchronize()
    n = plan.n_tiles
    bm = np.ones((n, n), dtype=np.uint8)
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
