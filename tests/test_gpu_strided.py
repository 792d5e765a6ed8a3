"""Attention on strided views (h3hip_bsattn_fwd_strided): the lazily
transposed [B, H, S, D] arrays AttentionLayer hands SDPABackend.attend
(Sources/H3Modules/DiTBlock.swift:323-327, 346-352;
Sources/H3Attention/AttentionBackend.swift:141-154).

The kernel is the same as h3hip_bsattn_fwd's, so on the same values the
output must be bit-identical to the head-major call. The fused buffers here
hold exactly S token rows followed by NaN guard rows, so a read past row S
would show up as NaN or a changed bit, and the output buffers carry a
sentinel that rows the call must not write keep."""
import ctypes
import math

import pytest
import torch

from _gpu import head_major_inputs, note

pytestmark = pytest.mark.gpu

GUARD = 16


def fuse_token_major(tensors, S, guard=GUARD):
    """[S + guard, n*H*D] token-major buffer holding the first S rows of each
    [H, >= S, D] tensor side by side (Q | K | V order); guard rows are NaN."""
    H, _, D = tensors[0].shape
    buf = torch.full((S + guard, len(tensors) * H * D), float("nan"), dtype=torch.bfloat16,
                     device=tensors[0].device)
    for i, t in enumerate(tensors):
        buf[:S, i * H * D:(i + 1) * H * D] = t[:, :S].transpose(0, 1).reshape(S, H * D)
    return buf


def head_views(buf, H, D, n):
    """[H, rows, D] views of the n column blocks of a fused token-major buffer."""
    rows = buf.shape[0]
    return [buf[:, i * H * D:(i + 1) * H * D].view(rows, H, D).transpose(0, 1) for i in range(n)]


def same_bits(a, b):
    return torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16))


@pytest.fixture(scope="module")
def ragged(h3):
    # S = 60 + 3*8*12 = 348: the last of 3 tiles is ragged.
    H = 3
    plan = h3.TilePlan(h3.MaskRule.local_window(prefix_len=60, frames=3, height=8, width=12),
                       heads=H)
    from h3hip import ops
    q, k, v = head_major_inputs(H, plan.seq_len, plan.seq_pad, 128, 71, pad_value=float("nan"))
    ref = ops.bsattn_fwd(plan, q, k, v)
    yield plan, q, k, v, ref
    plan.close()


def test_fused_qkv_views_match_head_major(h3, ragged):
    from h3hip import ops
    note("strided: fused qkv views, ragged S=348")
    plan, q, k, v, ref = ragged
    S, (H, _, D) = plan.seq_len, q.shape
    qkv = fuse_token_major([q, k, v], S)
    qv, kv, vv = head_views(qkv, H, D, 3)
    out = ops.bsattn_fwd_strided(plan, qv, kv, vv)
    torch.cuda.synchronize()
    assert out.shape == (S, H * D)
    assert torch.isfinite(out.float()).all()
    assert same_bits(out.view(S, H, D).transpose(0, 1), ref[:, :S])


def test_only_v_strided_and_strided_output_rows(h3, ragged):
    """Head-major Q and K, V from the fused buffer, and an output view with a
    row stride of 2*H*D whose other columns and rows >= S keep a sentinel."""
    from h3hip import ops
    note("strided: V view + strided output view")
    plan, q, k, v, ref = ragged
    S, (H, _, D) = plan.seq_len, q.shape
    vv = head_views(fuse_token_major([q, k, v], S), H, D, 3)[2]
    buf = torch.full((S + GUARD, 2 * H * D), 7.0, dtype=torch.bfloat16, device=q.device)
    ov = head_views(buf, H, D, 2)[1]
    got = ops.bsattn_fwd_strided(plan, q, k, vv, out=ov)
    torch.cuda.synchronize()
    assert got is ov
    assert same_bits(ov[:, :S], ref[:, :S])
    assert torch.all(buf[:, :H * D] == 7.0)
    assert torch.all(buf[S:] == 7.0)


def test_strided_refusals_leave_output_untouched(h3, ragged):
    from h3hip import _lib as L
    note("strided: refusals")
    plan, q, k, v, _ = ragged
    S, (H, _, D) = plan.seq_len, q.shape
    lib = h3.lib()
    out = torch.full_like(q, 7.0)
    hm = plan.seq_pad * D

    def view(t, off=0, hs=hm, rs=D):
        return L.ViewC(t.data_ptr() + off, hs, rs)

    def call(heads=H, hd=D, scale=1 / math.sqrt(D), **kw):
        vs = dict(q=view(q), k=view(k), v=view(v), out=view(out))
        vs.update(kw)
        return lib.h3hip_bsattn_fwd_strided(
            plan.handle, ctypes.byref(vs["q"]), ctypes.byref(vs["k"]), ctypes.byref(vs["v"]),
            heads, hd, scale, ctypes.byref(vs["out"]),
            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))

    assert call(heads=H + 1) == L.DECLINED
    assert call(hd=64) == L.DECLINED
    assert call(q=view(q, off=2)) == L.EINVAL and "aligned" in h3.last_error()
    assert call(k=view(k, hs=hm + 4)) == L.EINVAL and "head_stride" in h3.last_error()
    assert call(v=view(v, rs=64)) == L.EINVAL and "row_stride" in h3.last_error()
    assert call(out=view(out, rs=132)) == L.EINVAL
    assert call(v=L.ViewC(None, hm, D)) == L.EINVAL and "NULL" in h3.last_error()
    # 32-bit K/V offsets: seq_pad * row_stride * 2 must stay below 2^31.
    assert call(k=view(k, rs=(1 << 30) // plan.seq_pad * 8)) == L.EINVAL
    assert call(scale=0.0) == L.EINVAL
    assert lib.h3hip_bsattn_fwd_strided(None, None, None, None, H, D, 0.1, None, None) == L.EINVAL
    torch.cuda.synchronize()
    assert torch.all(out == 7.0)
    assert call() == L.OK
    torch.cuda.synchronize()
    assert not torch.all(out == 7.0)


def test_cfg3_v_straight_from_projection(h3):
    """The layer step of the headline shape: Q, K head-major (the prologue's
    output), V read in place from the fused projection output. Whole output
    bit-identical to the head-major call."""
    from h3hip import configs as C, ops
    note("strided: cfg3 V from the fused projection")
    sh = C.CFG3
    plan = h3.TilePlan(sh.mask_rule(), heads=sh.heads)
    try:
        S, H, D = plan.seq_len, sh.heads, 128
        q, k, v = head_major_inputs(H, S, plan.seq_pad, D, 91)
        ref = ops.bsattn_fwd(plan, q, k, v, out_layout=h3.OUT_TOKEN_MAJOR)
        qkv = fuse_token_major([q, k, v], S)
        del v
        vv = head_views(qkv, H, D, 3)[2]
        out = ops.bsattn_fwd_strided(plan, q, k, vv)
        torch.cuda.synchronize()
        assert same_bits(out, ref[:S])
    finally:
        plan.close()
