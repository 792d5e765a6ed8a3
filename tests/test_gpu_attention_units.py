"""Every work unit of the persistent attention kernel at full size.

The kernel runs each (head, 128-query tile) unit on one persistent workgroup
after that workgroup's previous units, carrying LDS contents (the next unit's
Q and first K tile are loaded during the previous unit's merge) from one unit
to the next in the order the plan's schedule fixes. So at the benchmark shapes
one query row of EVERY unit is compared with the dense-masked oracle
(AxialReference.attend semantics, AxialReference.swift:89-114), on the same
bf16 inputs, to the north star's bar (max-abs 2e-2, mean-abs 2e-3). The row
offset inside the tile advances by 53 (odd, so coprime with 128) from one unit
to the next, so all 128 row positions -- every query group and lane of the
workgroup -- are covered at each shape; each row's softmax runs over both
64-key halves of every active tile.
"""
import math

import numpy as np
import pytest
import torch

from _gpu import err_stats, f32, head_major_inputs, note

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def _bitmap(plan):
    row_ptr, col_idx = plan.tiles()
    bm = np.zeros((plan.n_tiles, plan.n_tiles), dtype=np.uint8)
    for i in range(plan.n_tiles):
        bm[i, col_idx[row_ptr[i]:row_ptr[i + 1]]] = 1
    return bm


def unit_rows(S, n_tiles, head):
    """One row per q-tile of `head`: offset (53 * unit) mod 128, folded into
    the ragged last tile."""
    rows = []
    for qt in range(n_tiles):
        unit = head * n_tiles + qt
        valid = min(128, S - qt * 128)
        rows.append(qt * 128 + (53 * unit) % 128 % valid)
    return np.asarray(rows, dtype=np.int32)


def check_every_unit(h3, orc, shape, seed, strided=False):
    from h3hip import ops
    plan = h3.TilePlan(shape.mask_rule(), heads=shape.heads)
    S, H, n = plan.seq_len, shape.heads, plan.n_tiles
    note(f"{shape.name} every unit: inputs (strided={strided})")
    q, k, v = head_major_inputs(H, S, plan.seq_pad, 128, seed)
    scale = 1.0 / math.sqrt(128)
    note(f"{shape.name} every unit: kernel")
    if strided:
        # The bench's layer layout: V read in place from a token-major buffer
        # [S, H, 128] (here its own), output token-major [S, H*128].
        v_tm = v[:, :S].transpose(0, 1).contiguous()
        out_tm = ops.bsattn_fwd_strided(plan, q, k, v_tm.transpose(0, 1), scale)
        torch.cuda.synchronize()
        out = out_tm.view(S, H, 128).transpose(0, 1)
    else:
        out = ops.bsattn_fwd(plan, q, k, v, scale)
        torch.cuda.synchronize()
        assert torch.all(out[:, S:] == 0)
    assert torch.isfinite(out.float()).all()
    bm = _bitmap(plan)
    worst_max, worst_mean, covered = 0.0, 0.0, set()
    for h in range(H):
        rows = unit_rows(S, n, h)
        covered.update((rows - np.arange(n) * 128).tolist())
        idx = torch.from_numpy(rows.astype(np.int64)).to(q.device)
        want = orc.attend_rows(f32(q[h].index_select(0, idx)), rows, f32(k[h, :S]),
                               f32(v[h, :S]), scale, bm, tile=128)
        got = f32(out[h].index_select(0, idx))
        mx, mean = err_stats(got, want)
        worst_max, worst_mean = max(worst_max, mx), max(worst_mean, mean)
        assert mx < MAX_ABS and mean < MEAN_ABS, (shape.name, h, mx, mean)
    print(f"{shape.name}: {H * n} units, max-abs {worst_max:.3e} mean-abs {worst_mean:.3e}, "
          f"{len(covered)} row positions")
    assert len(covered) == 128
    return plan


def test_cfg2_every_unit(h3, orc):
    from h3hip import configs as C
    check_every_unit(h3, orc, C.CFG2, seed=210)


def test_cfg3_every_unit(h3, orc):
    from h3hip import configs as C
    plan = check_every_unit(h3, orc, C.CFG3, seed=310)
    assert plan.nnz == 7854


def test_cfg3_every_unit_layer_layout(h3, orc):
    """The layout of the benchmarked layer step: V strided in place, output
    token-major."""
    from h3hip import configs as C
    check_every_unit(h3, orc, C.CFG3, seed=311, strided=True)


def test_cfg3_frame0_every_unit(h3, orc):
    from h3hip import configs as C
    plan = check_every_unit(h3, orc, C.CFG3_F0, seed=312)
    assert plan.nnz == 9691


def test_cfg4_every_unit(h3, orc):
    from h3hip import configs as C
    plan = check_every_unit(h3, orc, C.CFG4, seed=410)
    assert plan.nnz == 142 * 142


def test_axial_h3_every_unit(h3, orc):
    from h3hip import configs as C
    plan = check_every_unit(h3, orc, C.AXIAL_H3, seed=510)
    assert plan.nnz == 10815
