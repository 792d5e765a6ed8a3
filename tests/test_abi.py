"""The C ABI without a GPU: the library loads, exports every symbol
include/ch3hip.h declares, its host-side helpers agree with the oracle, and
argument refusals (EINVAL / DECLINED) happen before any device call."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "ch3hip.h")).read()
    return sorted(set(re.findall(r"\b(h3hip_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(h3):
    lib = h3.lib()
    syms = declared_symbols()
    assert len(syms) >= 18
    for name in syms:
        assert hasattr(lib, name), name
    from h3hip import _lib
    assert sorted(_lib.SIGNATURES) == syms


def test_version_and_no_device_here(h3):
    lib = h3.lib()
    assert b"gfx950" in lib.h3hip_version()


def test_rope_tables_match_oracle(h3, orc):
    from h3hip import ops
    ax, inv = ops.rope_pairs_axes(10000.0, (32, 48, 48))
    oax, oinv = orc.rope_pairs_axes(10000.0, 32, 48, 48)
    assert np.array_equal(ax, oax) and np.array_equal(inv, oinv)
    f = (1.0 / 10000.0 ** (np.arange(16) / 16)).astype(np.float32)
    ax3, inv3 = ops.rope_pairs_h3(f)
    oax3, oinv3 = orc.rope_pairs_h3(f)
    assert np.array_equal(ax3, oax3) and np.array_equal(inv3, oinv3)


def test_positions_match_oracle(h3, orc):
    from h3hip import ops
    assert np.array_equal(ops.positions_grid(637, 31, 24, 42), orc.positions_grid(637, 31, 24, 42))
    assert np.array_equal(ops.positions_packed(52, 207, 37, 30, 54),
                          orc.positions_packed(52, 207, 37, 30, 54))
    with pytest.raises(h3.H3HIPError):
        ops.positions_packed(1, 1, 1, 1, 1)          # axis smaller than the patch


def test_landmarks_match_oracle(h3, orc):
    for frames in (1, 2, 3, 5, 10, 36, 37, 100):
        for n in (0, 1, 2, 3, 4, 7, 999):
            assert h3.landmark_frames(frames, n) == orc.landmarks(frames, n), (frames, n)


def test_plan_refuses_bad_rules_before_touching_a_device(h3):
    lib = h3.lib()
    from h3hip import _lib
    out = ctypes.c_void_p()
    bad = _lib.MaskRuleC(kind=9, seq_len=100)
    assert lib.h3hip_plan_create(ctypes.byref(bad), 4, None, None, ctypes.byref(out)) == _lib.EINVAL
    assert "kind" in h3.last_error()
    # A lattice that does not fill the video span is refused, as AxialTopology refuses it
    # (AxialReferenceTests.mismatchedGeometryRefused).
    r = h3.MaskRule.axial(prefix_len=746, frames=37, height=15, width=27)
    assert r.seq_len == 15731
    c = r.to_c()
    c.prefix_len = 700
    assert lib.h3hip_plan_create(ctypes.byref(c), 4, None, None, ctypes.byref(out)) == _lib.EINVAL
    assert "lattice" in h3.last_error()
    assert lib.h3hip_bsattn_fwd(None, None, None, None, 4, 128, 0.1, None, 0, None) == _lib.EINVAL
    assert lib.h3hip_bsattn_fwd_strided(None, None, None, None, 4, 128, 0.1, None,
                                        None) == _lib.EINVAL
    assert "plan is NULL" in h3.last_error()


def test_prologue_declines_unsupported_geometry(h3):
    """QKFusionTests.declinesUnsupportedGeometry (:113-122): head_dim 64 declines."""
    lib = h3.lib()
    from h3hip import _lib
    rc = lib.h3hip_qk_norm_rope(None, None, 384, None, None, None, 1e-5, None, None, None, 64,
                                0, 4, 4, 2, 64, None, None, None, None)
    assert rc == _lib.DECLINED
    assert "declined" in h3.last_error()
    rc = lib.h3hip_qk_norm_rope(None, None, 768, None, None, None, 1e-5, None, None, None, 100,
                                0, 4, 4, 2, 128, None, None, None, None)
    assert rc == _lib.DECLINED


def test_projection_and_rope_table_refusals(h3):
    """h3hip_qkv_proj declines geometry it does not handle (the caller then runs
    its own GEMM + prologue) and refuses bad arguments by name; h3hip_rope_table
    refuses NULL and odd rot -- all before any device call."""
    from h3hip import _lib
    lib = h3.lib()
    D = _lib.DECLINED
    # head_dim 64, rot 80, odd heads, hidden % 64: declined.
    for head_dim, rot, heads, hidden in ((64, 64, 2, 128), (128, 80, 2, 128), (128, 128, 3, 128),
                                         (128, 128, 2, 96)):
        rc = lib.h3hip_qkv_proj(None, hidden, None, hidden, hidden, None, None, 1e-6, None, rot,
                                0, 4, 128, heads, head_dim, None, None, None, None)
        assert rc == D, (head_dim, rot, heads, hidden)
        assert "declined" in h3.last_error()
    # Supported geometry, NULL tensors: refused.
    rc = lib.h3hip_qkv_proj(None, 128, None, 128, 128, None, None, 1e-6, None, 128, 0, 4, 128, 2,
                            128, None, None, None, None)
    assert rc == _lib.EINVAL and "NULL" in h3.last_error()
    # Gammas given without a rotation table: refused.
    buf = ctypes.c_void_p(16)
    rc = lib.h3hip_qkv_proj(buf, 128, buf, 128, 128, buf, buf, 1e-6, None, 128, 0, 4, 128, 2,
                            128, buf, buf, buf, None)
    assert rc == _lib.EINVAL and "rotation table" in h3.last_error()
    # seq_pad not a multiple of 128: refused.
    rc = lib.h3hip_qkv_proj(buf, 128, buf, 128, 128, None, None, 1e-6, None, 128, 0, 4, 144, 2,
                            128, buf, buf, buf, None)
    assert rc == _lib.EINVAL and "seq_pad" in h3.last_error()
    # hidden 0 or a negative multiple of 64: refused, not declined.
    for hidden in (0, -64):
        rc = lib.h3hip_qkv_proj(buf, 128, buf, 128, hidden, None, None, 1e-6, None, 128, 0, 4,
                                128, 2, 128, buf, buf, buf, None)
        assert rc == _lib.EINVAL and "hidden" in h3.last_error(), hidden
    # h3hip_head_major: head_dim 64 declines, NULL and a short row stride are refused.
    assert lib.h3hip_head_major(buf, 256, 4, 128, 4, 64, buf, None) == D
    assert lib.h3hip_head_major(None, 512, 4, 128, 4, 128, buf, None) == _lib.EINVAL
    rc = lib.h3hip_head_major(buf, 256, 4, 128, 4, 128, buf, None)
    assert rc == _lib.EINVAL and "ld_in" in h3.last_error()
    assert lib.h3hip_rope_table(None, None, None, 128, 0, 4, None, None) == _lib.EINVAL
    rc = lib.h3hip_rope_table(buf, buf, buf, 127, 0, 4, buf, None)
    assert rc == _lib.EINVAL and "rot" in h3.last_error()
    rc = lib.h3hip_rope_table(buf, buf, buf, 128, 7, 4, buf, None)
    assert rc == _lib.EINVAL and "rounding" in h3.last_error()
