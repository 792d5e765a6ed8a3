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
