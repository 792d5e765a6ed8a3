"""The torch-facing attention wrappers refuse tensors the kernels would index
out of bounds -- wrong head count, head_dim, row count or a mismatched output --
before anything reaches the library (CPU only: the refusals come first)."""
import types

import pytest
import torch


def _plan(S=200):
    pad = (S + 127) // 128 * 128
    return types.SimpleNamespace(seq_len=S, seq_pad=pad, handle=None)


def _t(*shape):
    return torch.zeros(shape, dtype=torch.bfloat16)


def test_bsattn_fwd_refuses_mismatched_qkv(h3):
    from h3hip import ops
    p = _plan()
    good = _t(2, 256, 128)
    with pytest.raises(ValueError, match="one shape"):
        ops.bsattn_fwd(p, good, _t(1, 256, 128), good)
    with pytest.raises(ValueError, match="one shape"):
        ops.bsattn_fwd(p, good, good, _t(2, 256, 64))
    with pytest.raises(ValueError, match="contiguous"):
        ops.bsattn_fwd(p, _t(2, 200, 128), good, good)          # rows != seq_pad
    with pytest.raises(ValueError, match="contiguous"):
        ops.bsattn_fwd(p, good, good, _t(2, 128, 256).transpose(1, 2))


def test_bsattn_fwd_refuses_a_wrong_out(h3):
    from h3hip import ops
    p = _plan()
    good = _t(2, 256, 128)
    # Shapes pass; the GPU check then names the device.
    with pytest.raises(ValueError, match="GPU"):
        ops.bsattn_fwd(p, good, good, good)
    with pytest.raises(ValueError):
        ops.bsattn_fwd(p, good, good, good, out_layout=7)


def test_attend_refuses_short_inputs(h3):
    from h3hip import ops
    p = _plan()
    with pytest.raises(ValueError, match="contiguous"):
        ops.attend(p, None, _t(2, 200, 128), _t(2, 200, 128), _t(2, 200, 128), 0.1)
    good = _t(2, 256, 128)
    with pytest.raises(ValueError, match="one shape"):
        ops.attend(p, None, good, good, _t(3, 256, 128), 0.1)


def test_strided_views_must_match_heads_and_head_dim(h3):
    from h3hip import ops
    p = _plan()
    q = _t(2, 200, 128)
    for bad_k in (_t(1, 200, 128), _t(2, 200, 64), _t(2, 199, 128)):
        with pytest.raises(ValueError, match=r"\[2, >= 200, 128\]"):
            ops.bsattn_fwd_strided(p, q, bad_k, q)
        with pytest.raises(ValueError, match=r"\[2, >= 200, 128\]"):
            ops.attend_strided(p, None, q, q, bad_k, 0.1)
    with pytest.raises(ValueError, match=r"\[2, >= 200, 128\]"):
        ops.bsattn_fwd_strided(p, q, q, q, out=_t(2, 150, 128))
