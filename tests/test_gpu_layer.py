"""AttentionLayer (DiTBlock.swift:336-359) end to end on the GPU.

Against a float32 restatement of the reference chain computed on the CPU --
x . Wqkv^T, split, H3RMSNorm (Modulation.swift:116-120), SplitHalfRoPE with the
rotation table of H3RoPE (H3Transformer.swift:62-78, DiTBlock.swift:83-103),
scaled-dot-product attention, . Wout^T -- with the attention on the
block-sparse kernel through the backend seam (a dense plan, so every key is
attended). The device chain rounds to bf16 after the projection, the norm,
every RoPE product and sum, the attention and the out-projection; the bar is
relative RMS < 1e-2 of the output and max |d| < 8% of its RMS.
"""
import math

import numpy as np
import pytest
import torch

from _gpu import note

pytestmark = pytest.mark.gpu


def _setup(S=300, hidden=256, H=2, seed=3):
    from h3hip import ops
    from h3hip.layer import RopeState
    D = 128
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn((S, hidden), generator=g, device="cuda").to(torch.bfloat16)
    wqkv = (torch.randn((3 * H * D, hidden), generator=g, device="cuda") * 0.06).to(torch.bfloat16)
    wout = (torch.randn((hidden, H * D), generator=g, device="cuda") * 0.06).to(torch.bfloat16)
    qg = (torch.rand(D, generator=g, device="cuda") * 0.2 + 0.9).to(torch.bfloat16)
    kg = (torch.rand(D, generator=g, device="cuda") * 0.2 + 0.9).to(torch.bfloat16)
    pos = torch.from_numpy(ops.positions_grid(S - 3 * 8 * 9, 3, 8, 9)).cuda()
    ax, inv = (torch.from_numpy(t).cuda() for t in ops.rope_pairs_axes(10000.0, (32, 48, 48)))
    rope = RopeState.build(pos, ax, inv)
    return x, wqkv, wout, qg, kg, rope, H, D


def _reference(x, wqkv, wout, qg, kg, rope, H, D, eps):
    """The reference chain in float32 on the CPU."""
    f = lambda t: t.float().cpu()
    S = x.shape[0]
    qkv = f(x) @ f(wqkv).T
    q, k, v = (qkv[:, i * H * D:(i + 1) * H * D].reshape(S, H, D) for i in range(3))

    def rms(t, g):
        return t * torch.rsqrt((t * t).mean(-1, keepdim=True) + eps) * f(g)

    q, k = rms(q, qg), rms(k, kg)
    half = rope.rot // 2
    ang = f(rope.pos)[:, rope.pair_axis.long().cpu()] * f(rope.pair_inv)[None]   # [S, half]
    c, s = torch.cos(ang.double()).float()[:, None], torch.sin(ang.double()).float()[:, None]

    def rot(t):
        a, b = t[..., :half], t[..., half:rope.rot]
        return torch.cat([c * a - s * b, s * a + c * b, t[..., rope.rot:]], -1)

    q, k = rot(q), rot(k)
    o = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(0, 1)[None], k.transpose(0, 1)[None], v.transpose(0, 1)[None],
        scale=1.0 / math.sqrt(D))[0]
    return o.transpose(0, 1).reshape(S, H * D) @ f(wout).T


def _stats(got, want):
    got = got.float().cpu()
    rms = want.pow(2).mean().sqrt().item()
    d = (got - want).abs()
    return d.pow(2).mean().sqrt().item() / rms, d.max().item() / rms


@pytest.mark.parametrize("projection", ["fused", "hipblaslt"])
def test_layer_matches_fp32_reference(h3, projection):
    from h3hip.backend import AttentionContext, H3HIPBackend
    from h3hip.layer import AttentionLayer
    x, wqkv, wout, qg, kg, rope, H, D = _setup()
    S = x.shape[0]
    plan = h3.TilePlan(h3.MaskRule.dense(S), heads=H)
    layer = AttentionLayer(wqkv, wout, qg, kg, heads=H, eps=1e-6, backend=H3HIPBackend(plan),
                           projection=projection)
    note(f"layer {projection} S={S}")
    y = layer(x, rope, AttentionContext(3, 50, 0.5, S, None))
    torch.cuda.synchronize()
    want = _reference(x, wqkv, wout, qg, kg, rope, H, D, 1e-6)
    rel, mx = _stats(y, want)
    print(f"layer {projection}: rel RMS {rel:.2e}, max |d|/rms {mx:.2e}")
    assert y.shape == (S, wout.shape[0]) and rel < 1e-2 and mx < 8e-2


def test_paths_and_seam(h3):
    """Both projection paths agree; without a context the backend is not
    consulted and the dense path gives the same answer within bf16; with no
    rotation table the layer equals the identity rotation bit for bit."""
    from h3hip.backend import AttentionContext, H3HIPBackend
    from h3hip.layer import AttentionLayer, RopeState
    x, wqkv, wout, qg, kg, rope, H, D = _setup(S=260, seed=4)
    S = x.shape[0]
    plan = h3.TilePlan(h3.MaskRule.dense(S), heads=H)
    calls = []

    class Spy(H3HIPBackend):
        def attend(self, *a, **kw):
            calls.append(1)
            return super().attend(*a, **kw)

    ctx = AttentionContext(3, 50, 0.5, S, None)
    note("layer paths")
    fused = AttentionLayer(wqkv, wout, qg, kg, heads=H, eps=1e-6, backend=Spy(plan),
                           projection="fused")
    unfused = AttentionLayer(wqkv, wout, qg, kg, heads=H, eps=1e-6, backend=Spy(plan))
    y_f = fused(x, rope, ctx)
    y_u = unfused(x, rope, ctx)
    assert len(calls) == 2
    y_dense = unfused(x, rope, None)
    torch.cuda.synchronize()
    assert len(calls) == 2, "no context: the backend must not be consulted"
    ref = y_u.float().cpu()
    rel_fu, _ = _stats(y_f, ref)
    rel_dense, _ = _stats(y_dense, ref)
    print(f"fused vs hipblaslt rel {rel_fu:.2e}, dense vs sparse rel {rel_dense:.2e}")
    assert rel_fu < 1e-2 and rel_dense < 1e-2
    note("layer without a rotation table")
    y0 = fused(x, None, ctx)
    ident = RopeState.identity(S, D, x.device)
    y1 = fused(x, ident, ctx)
    torch.cuda.synchronize()
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
    rel0, mx0 = _stats(y0, _reference(x, wqkv, wout, qg, kg, ident, H, D, 1e-6))
    assert rel0 < 1e-2 and mx0 < 8e-2, (rel0, mx0)
