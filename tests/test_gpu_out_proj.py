"""The out-projection (h3hip_out_proj) on the GPU: y = x . w^T, token-major,
the last GEMM of AttentionLayer.callAsFunction (DiTBlock.swift:359,
matmul(merged, outWeight.T), no bias).

Checks per case:
- against an fp32 product on the CPU: each bf16 output within half a bf16 ulp
  of its fp32 value plus a small term for fp32 accumulation order
  (|d| <= 2^-8 |want| + 1e-3 rms);
- bit-identical to the plain QKV GEMM (h3hip_qkv_proj with both gammas NULL)
  on the same operands, which runs the same main loop and writes head-major:
  the two epilogues differ only in where they store;
- rows past seq_len of the output are never written, and a row stride wider
  than the row leaves the gap untouched.
"""
import numpy as np
import pytest
import torch

from _gpu import note

pytestmark = pytest.mark.gpu


def _operands(S, fin, fout, seed, ldx=None, ldw=None):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    xb = torch.randn((S, ldx or fin), generator=g, device="cuda").to(torch.bfloat16)
    wb = (torch.randn((fout, ldw or fin), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    return xb[:, :fin], wb[:, :fin]


def _check_fp32(y, x, w, rows=None):
    xs = x if rows is None else x[torch.from_numpy(rows).cuda()]
    ys = y if rows is None else y[torch.from_numpy(rows).cuda()]
    want = (xs.float().cpu() @ w.float().cpu().T).numpy()
    got = ys.float().cpu().numpy()
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    d = np.abs(got - want)
    bound = np.abs(want) * 2.0 ** -8 + 1e-3 * rms
    print(f"out_proj: max |d| {d.max():.3e}, worst d/bound {np.max(d / bound):.3f}")
    assert np.all(d <= bound), float(np.max(d / bound))


@pytest.mark.parametrize("S,fin,fout,ldx,ldy", [
    (256, 64, 256, None, None),          # one tile, one reduction step
    (300, 192, 512, 200, None),          # ragged rows, three steps, strided x
    (1000, 512, 768, None, 800),         # strided y: the gap stays untouched
    (1, 128, 256, None, None),           # a single token
])
def test_out_proj_small(S, fin, fout, ldx, ldy):
    from h3hip import ops
    x, w = _operands(S, fin, fout, 3, ldx)
    note(f"out_proj S={S} in={fin} out={fout} ldx={x.stride(0)} ldy={ldy}")
    if ldy:
        buf = torch.full((S + 2, ldy), 7.0, dtype=torch.bfloat16, device="cuda")
        y = ops.out_proj(x, w, out=buf[:S, :fout])
    else:
        buf = None
        y = ops.out_proj(x, w)
    torch.cuda.synchronize()
    assert y is not None
    _check_fp32(y, x, w)
    if buf is not None:
        assert torch.all(buf[:S, fout:] == 7.0) and torch.all(buf[S:] == 7.0)


def test_out_proj_equals_plain_qkv_gemm():
    """Same operands through the plain QKV GEMM (heads = out/384, written
    head-major) and the out-projection (token-major): bit for bit."""
    from h3hip import ops
    S, fin, H = 700, 320, 2
    fout = 3 * H * 128
    x, w = _operands(S, fin, fout, 11)
    note(f"out_proj vs plain qkv_proj S={S} in={fin} out={fout}")
    y = ops.out_proj(x, w)
    q, k, v = ops.qkv_proj(x, w, heads=H)
    torch.cuda.synchronize()
    tm = torch.cat([t[:, :S].permute(1, 0, 2).reshape(S, H * 128) for t in (q, k, v)], dim=1)
    assert torch.equal(y.view(torch.int16), tm.contiguous().view(torch.int16))


def test_out_proj_cfg3_full_size():
    """Config 3's out-projection: [31,885 x 5,120] . [5,120 x 5,120]^T, checked
    on 64 rows spread over the sequence (every channel tile)."""
    from h3hip import configs as C, ops
    S, inner = C.CFG3.seq_len, C.CFG3.heads * 128
    x, w = _operands(S, inner, 5120, 5)
    note(f"out_proj cfg3 S={S}")
    y = ops.out_proj(x, w)
    torch.cuda.synchronize()
    rows = np.linspace(0, S - 1, 64).astype(np.int64)
    _check_fp32(y, x, w, rows)
    assert torch.isfinite(y.float()).all()


def test_out_proj_declines_and_refuses(h3):
    from h3hip import _lib as L, ops
    x, w = _operands(256, 96, 256, 1)          # in_features not a multiple of 64
    assert ops.out_proj(x, w) is None
    x, w = _operands(256, 128, 200, 1)         # out_features not a multiple of 256
    assert ops.out_proj(x, w) is None
    x, w = _operands(256, 128, 256, 1)
    y = torch.empty((256, 256), dtype=torch.bfloat16, device="cuda")
    import ctypes
    rc = h3.lib().h3hip_out_proj(ctypes.c_void_p(x.data_ptr()), 64, ctypes.c_void_p(w.data_ptr()),
                                 128, 128, 256, 256, ctypes.c_void_p(y.data_ptr()), 256, None)
    assert rc == L.EINVAL and "ldx" in h3.last_error()
