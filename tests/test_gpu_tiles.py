"""Tile lists built on the GPU are bit-exact against the oracle's brute force."""
import ctypes
import os

import numpy as np
import pytest
import torch

from _gpu import note

HERE = os.path.dirname(os.path.abspath(__file__))
pytestmark = pytest.mark.gpu


def fixture(name):
    z = np.load(os.path.join(HERE, "golden", f"tiles_{name}.npz"))
    return z["row_ptr"], z["col_idx"].astype(np.int32)


def rule_for(h3, name):
    from h3hip import configs as C
    if name == "axial_h3_864x480x124":
        return h3.MaskRule.axial(prefix_len=746, frames=37, height=15, width=27,
                                 landmarks=[0, 18, 36])
    return C.ALL[name].mask_rule()


@pytest.mark.parametrize("name", ["cfg1_band_4x32x32", "cfg2_864x480x7s", "cfg3_1344x768x5s",
                                  "cfg3_1344x768x5s_frame0", "cfg4_dense_864x480x7s",
                                  "axial_h3_864x480x124"])
def test_plan_lists_are_bit_exact(h3, name):
    note(f"plan {name}")
    plan = h3.TilePlan(rule_for(h3, name), heads=40)
    row_ptr, col_idx = plan.tiles()
    want_rp, want_ci = fixture(name)
    assert np.array_equal(row_ptr, want_rp)
    assert np.array_equal(col_idx, want_ci)
    assert plan.nnz == len(want_ci)
    assert abs(plan.density - len(want_ci) / plan.n_tiles ** 2) < 1e-12


@pytest.mark.parametrize("case", [
    dict(kind="axial", prefix=7, frames=5, h=3, w=4, lm=[0, 4]),
    dict(kind="axial", prefix=300, frames=9, h=20, w=21, lm=[0, 4, 8]),
    dict(kind="local", prefix=129, frames=7, h=24, w=42, lm=[]),
    dict(kind="local", prefix=0, frames=11, h=13, w=17, lm=[3]),
])
def test_token_rules_on_ragged_shapes(h3, orc, case):
    note(f"token rule {case}")
    if case["kind"] == "axial":
        r = h3.MaskRule.axial(case["prefix"], case["frames"], case["h"], case["w"],
                              landmarks=case["lm"])
        o = orc.Rule(orc.RULE_AXIAL, r.seq_len, prefix_len=case["prefix"], frames=case["frames"],
                     height=case["h"], width=case["w"], landmarks=case["lm"])
    else:
        r = h3.MaskRule.local_window(case["prefix"], case["frames"], case["h"], case["w"],
                                     landmarks=case["lm"])
        o = orc.Rule(orc.RULE_LOCAL, r.seq_len, prefix_len=case["prefix"], frames=case["frames"],
                     height=case["h"], width=case["w"], frame_window=1, sp_tile=(8, 8),
                     sp_window=1, landmarks=case["lm"])
    plan = h3.TilePlan(r, heads=2)
    rp, ci = plan.tiles()
    wrp, wci = orc.csr(orc.tile_bitmap(o))
    assert np.array_equal(rp, wrp) and np.array_equal(ci, wci)


def test_bitmap_rule_with_empty_rows(h3, orc):
    note("bitmap rule")
    rng = np.random.default_rng(9)
    n = 37
    bm = (rng.random((n, n)) < 0.15).astype(np.uint8)
    bm[[0, 5, 36]] = 0
    plan = h3.TilePlan(h3.MaskRule.from_bitmap(n * 128 - 77, bm), heads=3)
    rp, ci = plan.tiles()
    wrp, wci = orc.csr(bm)
    assert np.array_equal(rp, wrp) and np.array_equal(ci, wci)


def test_tiles_from_mask_entry_point(h3, orc):
    note("tiles_from_mask")
    from h3hip import _lib
    rng = np.random.default_rng(2)
    nq, nk = 300, 517
    bm = (rng.random((nq, nk)) < 0.3).astype(np.uint8)
    d_bm = torch.from_numpy(bm).cuda()
    d_rp = torch.zeros(nq + 1, dtype=torch.int32, device="cuda")
    nnz = int(bm.sum())
    d_ci = torch.full((nnz,), -1, dtype=torch.int32, device="cuda")
    got = ctypes.c_int64()
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = h3.lib().h3hip_tiles_from_mask(ctypes.c_void_p(d_bm.data_ptr()), nq, nk,
                                        ctypes.c_void_p(d_rp.data_ptr()),
                                        ctypes.c_void_p(d_ci.data_ptr()), nnz, ctypes.byref(got), s)
    assert rc == 0 and got.value == nnz
    torch.cuda.synchronize()
    wrp, wci = orc.csr(bm)
    assert np.array_equal(d_rp.cpu().numpy(), wrp) and np.array_equal(d_ci.cpu().numpy(), wci)
    # Too little room: refused with nnz reported, nothing written past row_ptr.
    small = torch.full((10,), -7, dtype=torch.int32, device="cuda")
    rc = h3.lib().h3hip_tiles_from_mask(ctypes.c_void_p(d_bm.data_ptr()), nq, nk,
                                        ctypes.c_void_p(d_rp.data_ptr()),
                                        ctypes.c_void_p(small.data_ptr()), 10, ctypes.byref(got), s)
    assert rc == _lib.EINVAL and got.value == nnz
    assert torch.all(small == -7)


def test_mask_from_rule_entry_point(h3, orc):
    note("mask_from_rule")
    r = h3.MaskRule.local_window(637, 31, 24, 42)
    n = r.n_tiles
    d = torch.zeros(n * n, dtype=torch.uint8, device="cuda")
    crule = r.to_c()
    rc = h3.lib().h3hip_mask_from_rule(ctypes.byref(crule), ctypes.c_void_p(d.data_ptr()),
                                       ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    torch.cuda.synchronize()
    want_rp, want_ci = fixture("cfg3_1344x768x5s")
    bm = d.cpu().numpy().reshape(n, n)
    rp, ci = orc.csr(bm)
    assert np.array_equal(rp, want_rp) and np.array_equal(ci, want_ci)
