"""The reference's real positions, and the direction of rotation, on the GPU.

PackedLayout.positionIds (Sources/H3Foundation/PackedSequence.swift:185-296)
are float64, area-normalised and advance the time axis in non-integer steps;
prepareRender narrows them to fp32 before the angles are taken
(Sources/H3Modules/H3Transformer.swift:270). Here they feed the three device
paths that rotate -- the prologue, the rotation table and the fused QKV
projection -- at the H3 model geometry: 56 heads x 128, rot 96 (16 inv_freq
per axis, t|h|w duplicated; channels 96..127 pass through), eps 1e-5
(H3Config.swift:32). The checkpoint's inv_freq is not in the reference tree;
a theta-10000 geometric series of 16 stands in for it.

Gates: the prologue against orc_qk_norm_rope with the gate of
QKFusionTests.qkNormRoPECeiling (QKFusionTests.swift:64-110: relative RMS
< 1e-3, worst scaled ulp < 8) and >= 99.9% identical words; the bf16 table
against orc_rope_table (cos/sin in double, rounded once); the fused projection
bit-identical to the prologue over its own plain GEMM.

The rotation direction is pinned by a closed form that no restatement of the
kernel formula enters: a one-hot row e_p (p < rot/2) normalised by RMSNorm
is a * e_p with a = bf16(sqrt(128 / (1 + 128 eps))), and rotating it by +theta
in the (p, p + rot/2) plane gives a cos(theta) in channel p and a sin(theta)
in channel p + rot/2; e_{p + rot/2} gives -a sin(theta) and a cos(theta).
"""
import math

import numpy as np
import pytest
import torch

from _gpu import bits, note, to_gpu_bf16

pytestmark = pytest.mark.gpu

H3_HEADS, H3_ROT, H3_EPS = 56, 96, 1e-5
PACKED = dict(text_tokens=52, audio_t=207, latent_t=37, latent_h=30, latent_w=54)


def _h3_pairs():
    from h3hip import ops
    return ops.rope_pairs_h3((1.0 / 10000.0 ** (np.arange(16) / 16)).astype(np.float32))


def _packed_pos():
    from h3hip import ops
    p64 = ops.positions_packed(**PACKED)
    pos = p64.astype(np.float32)          # Float($0): H3Transformer.swift:270
    # The positions really are non-integer and large.
    frac = np.abs(pos - np.round(pos))
    assert frac.max() > 0.1 and pos.max() > 30
    return pos


def gate(got_bits, want_bits):
    import oracle as O
    a = O.bf16_to_f32(want_bits).astype(np.float64)
    b = O.bf16_to_f32(got_bits).astype(np.float64)
    rms = np.sqrt(np.mean(a * a))
    rel = np.sqrt(np.mean((a - b) ** 2)) / rms
    ulp = np.max(np.abs(a - b) / (np.abs(a) + rms)) / 0.0078125
    return rel, ulp, float(np.mean(got_bits == want_bits))


@pytest.mark.parametrize("rounding", [0, 1])
def test_prologue_on_packed_positions(h3, orc, rounding):
    from h3hip import ops
    pos = _packed_pos()
    S, H, D = pos.shape[0], H3_HEADS, 128
    S_pad = (S + 127) // 128 * 128
    axis, inv = _h3_pairs()
    inner = H * D
    qkv = orc.randn_bf16((S, 3 * inner), 61)
    qg = orc.uniform_bf16((D,), 62, 0.9, 1.1)
    kg = orc.uniform_bf16((D,), 63, 0.9, 1.1)
    g = to_gpu_bf16(qkv)
    note(f"prologue packed positions S={S} H={H} rot={H3_ROT} rounding={rounding}")
    q, k, _ = ops.qk_norm_rope(g[:, :inner], g[:, inner:2 * inner], to_gpu_bf16(qg),
                               to_gpu_bf16(kg), torch.from_numpy(pos).cuda(),
                               torch.from_numpy(axis).cuda(), torch.from_numpy(inv).cuda(),
                               heads=H, eps=H3_EPS, rot=H3_ROT, rounding=rounding)
    torch.cuda.synchronize()
    for name, got, x_bits, gam in (("q", q, np.ascontiguousarray(qkv[:, :inner]), qg),
                                   ("k", k, np.ascontiguousarray(qkv[:, inner:2 * inner]), kg)):
        want = orc.qk_norm_rope(x_bits, inner, S, S_pad, H, D, gam, H3_EPS, pos, axis, inv,
                                H3_ROT, rounding)
        rel, ulp, same = gate(bits(got), want)
        print(f"{name} rounding {rounding}: rel RMS {rel:.2e}, worst ulp {ulp:.2f}, "
              f"identical {same:.6f}")
        assert rel < 1e-3 and ulp < 8
        assert same >= 0.999


def test_rope_table_on_packed_positions(h3, orc):
    from h3hip import ops
    pos = _packed_pos()
    S = pos.shape[0]
    axis, inv = _h3_pairs()
    t_pos, t_ax, t_inv = (torch.from_numpy(a).cuda() for a in (pos, axis, inv))
    note(f"rope_table packed positions S={S}")
    got16 = ops.rope_table(t_pos, t_ax, t_inv, rot=H3_ROT, rounding=0)
    got32 = ops.rope_table(t_pos, t_ax, t_inv, rot=H3_ROT, rounding=1)
    torch.cuda.synchronize()
    want16 = orc.rope_table(pos, axis, inv, H3_ROT, 0)
    want32 = orc.rope_table(pos, axis, inv, H3_ROT, 1)
    gb = got16.reshape(S, H3_ROT // 2, 4).view(torch.int16).cpu().numpy().view(np.uint16)
    same = np.mean(gb == want16)
    d16 = np.abs(gb.astype(np.int32) - want16.astype(np.int32))
    gf = got32.reshape(S, H3_ROT // 2, 4).cpu().numpy()
    ulp = np.abs(gf.view(np.int32).astype(np.int64) - want32.view(np.int32).astype(np.int64))
    print(f"packed table: bf16 identical {same:.6f} (max {d16.max()} ulp), fp32 max {ulp.max()} ulp")
    assert same >= 0.999 and d16.max() <= 1 and ulp.max() <= 2
    # Against the closed form in double for the largest angles: cos and sin of
    # the fp32 angle fp32(pos * inv_freq) that H3RoPE.angles forms.
    ang = (pos[:, axis] * inv[None, :]).astype(np.float32).astype(np.float64)
    big = ang > 50
    assert big.any()
    assert np.allclose(gf[..., 0][big], np.cos(ang[big]), atol=2e-6)
    assert np.allclose(gf[..., 2][big], np.sin(ang[big]), atol=2e-6)


def test_fused_projection_on_packed_positions(h3, orc):
    """h3hip_qkv_proj with the table of the packed positions equals
    h3hip_qk_norm_rope over its own plain GEMM with the same positions, bit
    for bit, at hidden 5,376 and 56 heads."""
    from h3hip import ops
    pos = _packed_pos()[:2000]
    S, H, hidden = pos.shape[0], H3_HEADS, 5376
    axis, inv = _h3_pairs()
    t_pos, t_ax, t_inv = (torch.from_numpy(np.ascontiguousarray(a)).cuda()
                          for a in (pos, axis, inv))
    g = torch.Generator(device="cuda")
    g.manual_seed(64)
    x = torch.randn((S, hidden), generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn((3 * H * 128, hidden), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    qg = to_gpu_bf16(orc.uniform_bf16((128,), 65, 0.9, 1.1))
    kg = to_gpu_bf16(orc.uniform_bf16((128,), 66, 0.9, 1.1))
    for rounding in (0, 1):
        note(f"qkv_proj packed positions S={S} rounding={rounding}")
        plain = ops.qkv_proj(x, w, heads=H)
        table = ops.rope_table(t_pos, t_ax, t_inv, rot=H3_ROT, rounding=rounding)
        fused = ops.qkv_proj(x, w, qg, kg, table, heads=H, eps=H3_EPS, rounding=rounding)
        tm = [p[:, :S].permute(1, 0, 2).reshape(S, H * 128).contiguous() for p in plain[:2]]
        want_q, want_k, _ = ops.qk_norm_rope(tm[0], tm[1], qg, kg, t_pos, t_ax, t_inv, heads=H,
                                             eps=H3_EPS, rot=H3_ROT, rounding=rounding)
        torch.cuda.synchronize()
        assert np.array_equal(bits(fused[0]), bits(want_q))
        assert np.array_equal(bits(fused[1]), bits(want_k))
        assert np.array_equal(bits(fused[2]), bits(plain[2]))


@pytest.mark.parametrize("rounding", [0, 1])
def test_rotation_direction_closed_form(h3, rounding):
    from h3hip import ops
    axis, inv = _h3_pairs()
    half = H3_ROT // 2
    H, D = 2, 128
    # Token s rotates pair p by theta = pos[s, axis[p]] * inv[p]; the angles
    # cover all four quadrants.
    thetas = np.array([0.3, 1.9, 3.0, 4.4, 5.9, 37.25], dtype=np.float32)
    rows = []
    for p in (0, 5, 17, 40):
        for th in thetas:
            pos = np.zeros(3, dtype=np.float32)
            pos[axis[p]] = th / inv[p]
            for hot in (p, p + half):
                rows.append((p, hot, pos))
    S = len(rows)
    x = np.zeros((S, H * D), dtype=np.float32)
    pos = np.zeros((S, 3), dtype=np.float32)
    for s, (p, hot, ps) in enumerate(rows):
        x[s, hot] = 1.0
        x[s, D + hot] = 1.0
        pos[s] = ps
    xb = torch.from_numpy(x).to(torch.bfloat16).cuda()
    ones = torch.ones(D, dtype=torch.bfloat16, device="cuda")
    note(f"rotation direction closed form rounding={rounding}")
    q, _, _ = ops.qk_norm_rope(xb, xb, ones, ones, torch.from_numpy(pos).cuda(),
                               torch.from_numpy(axis).cuda(), torch.from_numpy(inv).cuda(),
                               heads=H, eps=H3_EPS, rot=H3_ROT, rounding=rounding)
    torch.cuda.synchronize()
    out = q.float().cpu().numpy()
    a = float(torch.tensor(math.sqrt(128.0 / (1.0 + 128.0 * H3_EPS))).to(torch.bfloat16).float())
    for s, (p, hot, ps) in enumerate(rows):
        th = float(ps[axis[p]]) * float(inv[p])
        c, sn = math.cos(th), math.sin(th)
        want_p, want_q = (a * c, a * sn) if hot == p else (-a * sn, a * c)
        for h in range(H):
            got = out[h, s]
            assert abs(got[p] - want_p) <= 0.02 * a, (s, p, hot, th, got[p], want_p)
            assert abs(got[p + half] - want_q) <= 0.02 * a, (s, p, hot, th, got[p + half], want_q)
            others = np.delete(got, [p, p + half])
            assert np.all(others == 0)
