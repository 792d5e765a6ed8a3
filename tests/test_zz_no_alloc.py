"""h3hip_mask_from_rule_noalloc: the allocation-free variant of
h3hip_mask_from_rule (flag tables staged in the library's static per-GPU
scratch). Its bitmap must equal the allocating entry point's, bit for bit, on
two calls in a row where the second has a smaller input, so nothing the first
call left in the shared scratch can leak into the second."""
import ctypes

import numpy as np
import pytest
import torch

from _gpu import note

pytestmark = pytest.mark.gpu


def _bitmap(h3, fn, rule):
    n = rule.n_tiles
    d = torch.full((n * n,), 7, dtype=torch.uint8, device="cuda")
    crule = rule.to_c()
    rc = getattr(h3.lib(), fn)(ctypes.byref(crule), ctypes.c_void_p(d.data_ptr()),
                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, h3.last_error()
    torch.cuda.synchronize()
    return d.cpu().numpy().reshape(n, n)


PAIRS = [
    ("band", lambda h3: h3.MaskRule.band_rule(250 * 128 - 37, band=2, global_cols=(0, 5, 100, 249)),
     lambda h3: h3.MaskRule.band_rule(40 * 128, band=1, global_cols=(3,))),
    ("local", lambda h3: h3.MaskRule.local_window(637, 31, 24, 42, landmarks=(0, 10, 20, 30)),
     lambda h3: h3.MaskRule.local_window(100, 5, 12, 13, spatial_tile=(4, 4), landmarks=(1,))),
    ("axial", lambda h3: h3.MaskRule.axial(746, 37, 15, 27, n_landmarks=5),
     lambda h3: h3.MaskRule.axial(100, 6, 10, 12, landmarks=[0, 5])),
    ("dense", lambda h3: h3.MaskRule.dense(3000), lambda h3: h3.MaskRule.dense(300)),
]


@pytest.mark.parametrize("name,big,small", PAIRS, ids=[p[0] for p in PAIRS])
def test_equals_allocating_entry_point_twice(h3, name, big, small):
    for i, make in enumerate((big, small)):
        rule = make(h3)
        note(f"mask_from_rule_noalloc {name} call {i + 1} (n_tiles {rule.n_tiles})")
        got = _bitmap(h3, "h3hip_mask_from_rule_noalloc", rule)
        want = _bitmap(h3, "h3hip_mask_from_rule", rule)
        assert np.array_equal(got, want), (name, i)
        assert set(np.unique(got)) <= {0, 1}


def test_refuses_rules_beyond_the_scratch(h3):
    """More landmark frames than the scratch holds flags for: refused, nothing launched."""
    from h3hip import _lib
    frames = 40000
    rule = h3.MaskRule.local_window(0, frames, 1, 1, spatial_tile=(1, 1), landmarks=(0,))
    crule = rule.to_c()
    d = torch.zeros(1, dtype=torch.uint8, device="cuda")
    rc = h3.lib().h3hip_mask_from_rule_noalloc(ctypes.byref(crule), ctypes.c_void_p(d.data_ptr()),
                                               None)
    assert rc == _lib.EINVAL and "scratch" in h3.last_error()


def _golden_csr(name):
    import os
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                             f"tiles_{name}.npz"))
    return z["row_ptr"], z["col_idx"].astype(np.int32)


def _csr(bitmap):
    rows = bitmap.astype(bool)
    row_ptr = np.concatenate([[0], np.cumsum(rows.sum(1))]).astype(np.int32)
    col_idx = np.concatenate([np.flatnonzero(r) for r in rows]).astype(np.int32)
    return row_ptr, col_idx


def _call(h3, crule, d):
    return h3.lib().h3hip_mask_from_rule_noalloc(
        ctypes.byref(crule), ctypes.c_void_p(d.data_ptr()),
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


CAPTURED = ["cfg3_1344x768x5s", "cfg3_1344x768x5s_frame0", "cfg1_band_4x32x32"]


@pytest.mark.parametrize("name", CAPTURED)
def test_captured_in_a_graph_and_replayed(h3, name):
    """Rules whose lists travel in the kernel arguments (cfg3: no list; cfg3
    with frame 0 as a landmark: one landmark; cfg1: one global column) are
    captured into a HIP graph, the host lists are overwritten after capture,
    and every replay -- with eager work and synchronisations between them --
    gives the committed tile lists."""
    from h3hip import configs as C
    rule = C.ALL[name].mask_rule()
    n = rule.n_tiles
    crule = rule.to_c()
    d = torch.full((n * n,), 7, dtype=torch.uint8, device="cuda")
    note(f"mask_from_rule_noalloc {name} eager warm-up")
    assert _call(h3, crule, d) == 0, h3.last_error()
    torch.cuda.synchronize()
    want_rp, want_ci = _golden_csr(name)
    graph = torch.cuda.CUDAGraph()
    note(f"mask_from_rule_noalloc {name} capture")
    with torch.cuda.graph(graph):
        rc = _call(h3, crule, d)
    assert rc == 0, h3.last_error()
    # A captured host copy would re-read these at every replay.
    for arr in rule._keep:
        if arr is not None and arr.size:
            arr[...] = 0 if arr.dtype == np.uint8 else n - 1
    for rep in range(3):
        d.fill_(7)                       # eager work between replays
        torch.cuda.synchronize()
        note(f"mask_from_rule_noalloc {name} replay {rep}")
        graph.replay()
        torch.cuda.synchronize()
        rp, ci = _csr(d.cpu().numpy().reshape(n, n))
        assert np.array_equal(rp, want_rp) and np.array_equal(ci, want_ci), (name, rep)
    del graph


@pytest.mark.parametrize("kind", ["long_list", "bitmap"])
def test_host_staging_is_refused_under_capture(h3, kind):
    """A list longer than the kernel arguments carry, and a host bitmap, would
    be staged from host memory: under capture the call returns EINVAL and the
    capture stays valid (the graph ends and replays its other work)."""
    from h3hip import _lib
    if kind == "long_list":
        rule = h3.MaskRule.band_rule(400 * 128, band=1, global_cols=tuple(range(0, 400, 1))[:300])
    else:
        bm = np.eye(8, dtype=np.uint8)
        rule = h3.MaskRule.from_bitmap(8 * 128, bm)
    n = rule.n_tiles
    crule = rule.to_c()
    d = torch.zeros((n * n,), dtype=torch.uint8, device="cuda")
    x = torch.zeros(4, device="cuda")
    graph = torch.cuda.CUDAGraph()
    note(f"mask_from_rule_noalloc refused under capture ({kind})")
    with torch.cuda.graph(graph):
        rc = _call(h3, crule, d)
        x.add_(1.0)
    assert rc == _lib.EINVAL and "capture" in h3.last_error()
    graph.replay()
    torch.cuda.synchronize()
    assert float(x[0]) == 1.0
    # Outside capture the same call stages, synchronises and matches the
    # allocating entry point.
    assert _call(h3, crule, d) == 0, h3.last_error()
    torch.cuda.synchronize()
    got = d.cpu().numpy().reshape(n, n)
    assert np.array_equal(got, _bitmap(h3, "h3hip_mask_from_rule", rule))
