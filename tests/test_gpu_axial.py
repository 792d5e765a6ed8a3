"""The reference's own topology (AxialTopology.allows,
Sources/H3Attention/AxialTopology.swift:128-137) as a tile-mask profile on the
GPU, and the per-span error protocol of
AxialMeasureTests.axialErrorOnRealAttention (AxialMeasureTests.swift:54-98)
run through the capture reader.

Attention parity is against the oracle's dense-masked attention on the same
tile bitmap, to the north star's bar (max-abs 2e-2, mean-abs 2e-3). The
per-span checks use what the topology fixes regardless of the data: prefix
queries attend every key, so their rows equal dense attention up to the
kernel's bf16 rounding, and with every frame a landmark the whole topology is
dense.
"""
import math

import numpy as np
import pytest
import torch

from _gpu import err_stats, f32, head_major_inputs, note

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def tile_bitmap(plan):
    row_ptr, col_idx = plan.tiles()
    bm = np.zeros((plan.n_tiles, plan.n_tiles), dtype=np.uint8)
    for i in range(plan.n_tiles):
        bm[i, col_idx[row_ptr[i]:row_ptr[i + 1]]] = 1
    return bm


def test_axial_small_shape_in_full(h3, orc):
    from h3hip import ops
    note("axial small full")
    rule = h3.MaskRule.axial(prefix_len=100, frames=6, height=10, width=12, landmarks=[0, 5])
    plan = h3.TilePlan(rule, heads=2)
    S = plan.seq_len
    q, k, v = head_major_inputs(2, S, plan.seq_pad, 128, 31)
    scale = 1.0 / math.sqrt(128)
    out = ops.bsattn_fwd(plan, q, k, v, scale)
    torch.cuda.synchronize()
    o = orc.Rule(orc.RULE_AXIAL, S, prefix_len=100, frames=6, height=10, width=12, landmarks=[0, 5])
    bm = orc.tile_bitmap(o)
    assert np.array_equal(bm, tile_bitmap(plan))
    want = orc.attend_masked(f32(q)[:, :S], f32(k)[:, :S], f32(v)[:, :S], scale, bm, tile=128)
    mx, mean = err_stats(f32(out)[:, :S], want)
    print(f"axial small: max-abs {mx:.3e} mean-abs {mean:.3e}")
    assert mx < MAX_ABS and mean < MEAN_ABS


def test_axial_production_shape_sampled(h3, orc):
    """864x480x124, 56 heads: 10,815 of 123^2 tiles; sampled rows of the prefix
    tile, the prefix/video boundary tile, a middle tile and the ragged last tile."""
    from h3hip import configs as C, ops
    sh = C.AXIAL_H3
    note("axial production shape")
    plan = h3.TilePlan(sh.mask_rule(), heads=sh.heads)
    assert plan.nnz == 10815
    S = plan.seq_len
    q, k, v = head_major_inputs(sh.heads, S, plan.seq_pad, 128, 500)
    scale = 1.0 / math.sqrt(128)
    out = ops.bsattn_fwd(plan, q, k, v, scale)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all() and torch.all(out[:, S:] == 0)
    bm = tile_bitmap(plan)
    tiles = sorted({0, sh.prefix_len // 128, plan.n_tiles // 2, plan.n_tiles - 1})
    worst = (0.0, 0.0)
    for h in (0, 29, 55):
        rows = np.concatenate([np.arange(t * 128, min(t * 128 + 128, S))[::4] for t in tiles])
        rows = rows.astype(np.int32)
        want = orc.attend_rows(f32(q[h])[rows], rows, f32(k[h, :S]), f32(v[h, :S]), scale, bm,
                               tile=128)
        mx, mean = err_stats(f32(out[h])[rows], want)
        worst = (max(worst[0], mx), max(worst[1], mean))
    print(f"axial production: tile density {plan.density:.4f}, max-abs {worst[0]:.3e}, "
          f"mean-abs {worst[1]:.3e}")
    assert worst[0] < MAX_ABS and worst[1] < MEAN_ABS


def synthetic_capture(path, S, H, seed):
    from h3hip.capture import save_qkv
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    q, k, v = (torch.randn((S, H, 128), generator=g, device="cuda").to(torch.bfloat16)
               for _ in range(3))
    save_qkv(str(path), q, k, v)


def test_per_span_error_invariants(h3, tmp_path):
    from h3hip.capture import capture_name, load_qkv
    from h3hip.measure import per_span_error
    note("per-span error invariants")
    # Frames of 8 tiles: a q-tile sees its own frame, one tile of every other
    # frame and the landmark frames -- sparse at tile granularity.
    prefix, frames, hh, ww = 128, 8, 32, 32
    S = prefix + frames * hh * ww
    path = tmp_path / capture_name(0, 0.5)
    synthetic_capture(path, S, 2, 77)
    q, k, v, s = load_qkv(str(path))
    assert s == S
    rows = per_span_error(q, k, v, S, prefix, frames, hh, ww, landmark_counts=(2, 8))
    by_n = {r["landmarks"]: r for r in rows}
    for r in rows:
        print(f"landmarks {r['landmarks']}: density {r['density']:.3f} tiles {r['tile_density']:.3f} "
              f"total {r['total']:.4f} prefix {r['prefix']:.4f} video {r['video']:.4f}")
        assert r["tile_density"] >= r["density"] - 1e-12
        assert r["prefix"] < 1e-2          # prefix rows are dense: bf16 rounding only
    assert by_n[8]["total"] < 1e-2         # every frame a landmark: dense
    assert abs(by_n[8]["density"] - 1.0) < 1e-12
    assert by_n[2]["tile_density"] < 0.6
    assert by_n[2]["video"] > 10 * by_n[2]["prefix"]


def test_measure_cli_over_a_capture_directory(h3, tmp_path, capsys):
    from h3hip.capture import capture_name
    from h3hip.measure import main
    note("measure cli")
    prefix, frames, hh, ww = 40, 5, 6, 9
    S = prefix + frames * hh * ww
    synthetic_capture(tmp_path / capture_name(24, 0.5), S, 2, 3)
    synthetic_capture(tmp_path / capture_name(24, 0.6), 200, 2, 4)   # shorter than the lattice
    rc = main([str(tmp_path), "--frames", "5", "--height", "6", "--width", "9",
               "--landmarks", "2,5"])
    out = capsys.readouterr().out
    assert rc == 0
    assert "block 24 progress 0.50" in out and "landmarks  density" in out
    assert "S=200 is shorter than the 270-token lattice -- skipped" in out
    table = [ln.split() for ln in out.splitlines() if ln.strip()[:1].isdigit()]
    assert [int(r[0]) for r in table] == [2, 5] and all(len(r) == 6 for r in table)
