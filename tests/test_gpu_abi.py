"""The C ABI on real device buffers: refusals instead of traps (the H3Error
style, Sources/H3Foundation/H3Error.swift:26-43), declines for geometry this
path does not take (the nil of H3AttentionBackend.attend,
Sources/H3Attention/AttentionBackend.swift:123-127), stream ordering and
plan reuse. Every refused call leaves its output untouched."""
import ctypes
import math

import numpy as np
import pytest
import torch

from _gpu import head_major_inputs, note

pytestmark = pytest.mark.gpu


def vp(t, byte_offset=0):
    return ctypes.c_void_p(t.data_ptr() + byte_offset)


def cur_stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


@pytest.fixture(scope="module")
def small(h3):
    plan = h3.TilePlan(h3.MaskRule.local_window(prefix_len=60, frames=3, height=8, width=12), heads=2)
    q, k, v = head_major_inputs(2, plan.seq_len, plan.seq_pad, 128, 41)
    yield plan, q, k, v
    plan.close()


def test_attention_declines_and_refusals(h3, small):
    from h3hip import _lib as L
    note("abi attention refusals")
    plan, q, k, v = small
    lib = h3.lib()
    out = torch.full_like(q, 7.0)
    args = lambda **kw: dict(dict(q=vp(q), k=vp(k), v=vp(v), heads=2, hd=128, scale=0.088,
                                  out=vp(out), layout=0), **kw)

    def call(**kw):
        a = args(**kw)
        return lib.h3hip_bsattn_fwd(plan.handle, a["q"], a["k"], a["v"], a["heads"], a["hd"],
                                    a["scale"], a["out"], a["layout"], cur_stream())

    assert call(heads=3) == L.DECLINED and "declined" in h3.last_error()
    assert call(hd=64) == L.DECLINED
    assert call(q=vp(q, 2)) == L.EINVAL and "aligned" in h3.last_error()
    assert call(out=vp(out, 4)) == L.EINVAL
    assert call(scale=0.0) == L.EINVAL and call(scale=-1.0) == L.EINVAL
    assert call(scale=float("nan")) == L.EINVAL and call(scale=float("inf")) == L.EINVAL
    assert call(layout=2) == L.EINVAL and "out_layout" in h3.last_error()
    assert call(v=ctypes.c_void_p(None)) == L.EINVAL
    torch.cuda.synchronize()
    assert torch.all(out == 7.0)
    assert call() == L.OK
    torch.cuda.synchronize()
    assert not torch.all(out == 7.0)


def test_prologue_refusals(h3):
    from h3hip import _lib as L
    from h3hip import ops
    note("abi prologue refusals")
    lib = h3.lib()
    S, H, D = 300, 2, 128
    S_pad = 384
    inner = H * D
    x = torch.randn((S, inner), device="cuda").to(torch.bfloat16)
    g = torch.ones(D, device="cuda", dtype=torch.bfloat16)
    pos = torch.zeros((S, 3), device="cuda", dtype=torch.float32)
    ax_np, inv_np = ops.rope_pairs_axes(1e4, (32, 48, 48))
    ax, inv = torch.from_numpy(ax_np).cuda(), torch.from_numpy(inv_np).cuda()
    qo = torch.full((H, S_pad, D), 3.0, device="cuda", dtype=torch.bfloat16)
    ko = torch.full_like(qo, 3.0)
    vo = torch.full_like(qo, 3.0)

    def call(v_in=None, v_out=None, seq_len=S, seq_pad=S_pad, ld=inner, rounding=0, q_in=None,
             q_out=None):
        return lib.h3hip_qk_norm_rope(q_in if q_in is not None else vp(x), vp(x), ld, v_in, vp(g),
                                      vp(g), 1e-6, vp(pos), vp(ax), vp(inv), 128, rounding,
                                      seq_len, seq_pad, H, D,
                                      q_out if q_out is not None else vp(qo), vp(ko), v_out,
                                      cur_stream())

    assert call(v_in=vp(x)) == L.EINVAL and "v_in and v_out" in h3.last_error()
    assert call(v_out=vp(vo)) == L.EINVAL
    assert call(seq_pad=256) == L.EINVAL                    # seq_pad < seq_len
    assert call(seq_len=0) == L.EINVAL
    assert call(ld=inner - 8) == L.EINVAL and "ld_in" in h3.last_error()
    assert call(ld=inner + 4) == L.EINVAL                   # not a multiple of 8
    assert call(rounding=5) == L.EINVAL
    assert call(q_in=vp(x, 2)) == L.EINVAL and "aligned" in h3.last_error()
    assert call(q_out=vp(qo, 8)) == L.EINVAL
    torch.cuda.synchronize()
    assert torch.all(qo == 3.0) and torch.all(ko == 3.0)
    assert call(v_in=vp(x), v_out=vp(vo)) == L.OK
    torch.cuda.synchronize()
    assert torch.all(qo[:, S:] == 0) and torch.all(vo[:, :S] == x.view(S, H, D).transpose(0, 1))


def test_results_on_a_side_stream_match_the_default_stream(h3, small):
    """Calls are ordered on the stream they are given; a side stream gives the
    same bits as the default one."""
    from h3hip import ops
    note("abi side stream")
    plan, q, k, v = small
    want = ops.bsattn_fwd(plan, q, k, v, 0.088)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        got = ops.bsattn_fwd(plan, q, k, v, 0.088)
        got_tm = ops.bsattn_fwd(plan, q, k, v, 0.088, out_layout=1)
    side.synchronize()
    assert torch.equal(got, want)
    H, Sp, D = want.shape
    assert torch.equal(got_tm.view(Sp, H, D).transpose(0, 1), want)


def test_one_plan_serves_many_calls_and_closes_cleanly(h3, small):
    """A plan is immutable after creation: the same plan answers different
    inputs independently, and a destroyed plan handle is refused by the
    Python side rather than reused."""
    from h3hip import ops
    note("abi plan reuse")
    plan, q, k, v = small
    q2, k2, v2 = head_major_inputs(2, plan.seq_len, plan.seq_pad, 128, 99)
    a1 = ops.bsattn_fwd(plan, q, k, v, 0.088)
    a2 = ops.bsattn_fwd(plan, q2, k2, v2, 0.088)
    a3 = ops.bsattn_fwd(plan, q, k, v, 0.088)
    torch.cuda.synchronize()
    assert torch.equal(a1, a3) and not torch.equal(a1, a2)
    p2 = h3.TilePlan(h3.MaskRule.dense(700), heads=1)
    p2.close()
    p2.close()                       # idempotent
    assert h3.lib().h3hip_plan_destroy(None) == 0
    z = torch.zeros((1, 768, 128), device="cuda", dtype=torch.bfloat16)
    with pytest.raises(h3.H3HIPError, match="plan is NULL"):
        ops.bsattn_fwd(p2, z, z, z, 0.088)


def test_prologue_is_deterministic(h3):
    from h3hip import ops
    note("abi prologue determinism")
    S, H, D = 1000, 3, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(8)
    q = torch.randn((S, H * D), generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn((S, H * D), generator=g, device="cuda").to(torch.bfloat16)
    gam = torch.ones(D, device="cuda", dtype=torch.bfloat16)
    pos = torch.rand((S, 3), generator=g, device="cuda") * 30
    ax_np, inv_np = ops.rope_pairs_axes(1e4, (32, 48, 48))
    ax, inv = torch.from_numpy(ax_np).cuda(), torch.from_numpy(inv_np).cuda()
    r1 = ops.qk_norm_rope(q, k, gam, gam, pos, ax, inv, heads=H)
    r2 = ops.qk_norm_rope(q, k, gam, gam, pos, ax, inv, heads=H)
    torch.cuda.synchronize()
    assert torch.equal(r1[0], r2[0]) and torch.equal(r1[1], r2[1])
