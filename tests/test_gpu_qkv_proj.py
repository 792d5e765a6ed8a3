"""The fused QKV projection (GEMM + Q/K norm/RoPE epilogue) on the GPU.

Two checks per case:
- the plain GEMM (both gammas NULL) against an fp32 product computed on the
  CPU: each bf16 output within half a bf16 ulp of its fp32 value plus a small
  term for fp32 accumulation order (|d| <= 2^-8 |want| + 1e-3 rms);
- the fused call, rotating with the table h3hip_rope_table builds, against
  h3hip_qk_norm_rope applied to the plain GEMM's output (converted back to
  the token-major qkv the reference's AttentionLayer.callAsFunction produces,
  DiTBlock.swift:338-345): Q and K bit-identical, V bit-identical to the
  plain V. The prologue kernel is itself pinned to the oracle by
  test_gpu_prologue.py, so this carries the oracle through to the fused
  kernel. The table itself is checked against orc_rope_table.
"""
import numpy as np
import pytest
import torch

from _gpu import bits, note, to_gpu_bf16

pytestmark = pytest.mark.gpu


def _tables(orc, S, rot, h3_tables):
    from h3hip import ops
    frames, hh, ww = 3, 8, 9
    pos = orc.positions_grid(max(S - frames * hh * ww, 0), frames, hh, ww)[:S]
    if h3_tables:
        axis, inv = ops.rope_pairs_h3((1.0 / 10000.0 ** (np.arange(16) / 16)).astype(np.float32))
    else:
        axis, inv = ops.rope_pairs_axes(10000.0, (32, 48, 48))
    axis, inv = axis[:rot // 2], inv[:rot // 2]
    return (torch.from_numpy(np.ascontiguousarray(pos)).cuda(), torch.from_numpy(axis).cuda(),
            torch.from_numpy(inv).cuda())


def _inputs(S, hidden, H, seed, ldx=None, ldw=None):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    ldx, ldw = ldx or hidden, ldw or hidden
    xb = torch.randn((S, ldx), generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn((3 * H * 128, ldw), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    return xb[:, :hidden], w[:, :hidden]


def _token_major(t, S):
    H, _, D = t.shape
    return t[:, :S].permute(1, 0, 2).reshape(S, H * D).contiguous()


def _check_plain(q, k, v, x, w, S, rows=None):
    """Plain GEMM output [3][H, S_pad, 128] against fp32 x . w^T on the CPU."""
    H = q.shape[0]
    xs = x if rows is None else x[torch.from_numpy(rows).cuda()]
    want = (xs.float().cpu() @ w.float().cpu().T).numpy()          # [R, 3*H*128]
    got = torch.cat([_token_major(t, S) for t in (q, k, v)], dim=1)
    if rows is not None:
        got = got[torch.from_numpy(rows).cuda()]
    got = got.float().cpu().numpy()
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    d = np.abs(got - want)
    bound = np.abs(want) * 2.0 ** -8 + 1e-3 * rms
    print(f"plain: max |d| {d.max():.3e}, worst d/bound {np.max(d / bound):.3f}")
    assert np.all(d <= bound), float(np.max(d / bound))
    for t in (q, k, v):
        assert torch.all(t[:, S:] == 0)


def _run(orc, S, hidden, H, rot, rounding, h3_tables=False, ldx=None, seed=7, ldw=None):
    from h3hip import ops
    x, w = _inputs(S, hidden, H, seed, ldx, ldw)
    qg = to_gpu_bf16(orc.uniform_bf16((128,), seed + 1, 0.9, 1.1))
    kg = to_gpu_bf16(orc.uniform_bf16((128,), seed + 2, 0.9, 1.1))
    pos, axis, inv = _tables(orc, S, rot, h3_tables)
    note(f"qkv_proj plain S={S} hidden={hidden} H={H} ldx={x.stride(0)}")
    plain = ops.qkv_proj(x, w, heads=H)
    torch.cuda.synchronize()
    note(f"rope_table S={S} rot={rot} rounding={rounding}")
    table = ops.rope_table(pos, axis, inv, rot=rot, rounding=rounding)
    note(f"qkv_proj fused S={S} hidden={hidden} H={H} rot={rot} rounding={rounding}")
    fused = ops.qkv_proj(x, w, qg, kg, table, heads=H, eps=1e-6, rounding=rounding)
    torch.cuda.synchronize()
    note(f"prologue over the plain GEMM S={S} H={H}")
    q_tm, k_tm = _token_major(plain[0], S), _token_major(plain[1], S)
    want_q, want_k, _ = ops.qk_norm_rope(q_tm, k_tm, qg, kg, pos, axis, inv, heads=H, eps=1e-6,
                                         rot=rot, rounding=rounding)
    torch.cuda.synchronize()
    return x, w, plain, fused, (want_q, want_k)


@pytest.mark.parametrize("S,hidden,H,rot,rounding,h3t", [
    (300, 256, 2, 128, 0, False),     # ragged S (two token tiles, the second part-padding)
    (300, 256, 2, 128, 1, False),     # fp32 rounding
    (256, 512, 4, 96, 0, True),       # the H3 table: rot 96, channels 96..127 pass through
    (130, 128, 6, 96, 1, True),       # S just past one 128-row tile, rot 96 fp32 rounding
    (1000, 5120, 4, 128, 0, False),   # the benchmark configs' hidden width
    (700, 5376, 56, 96, 0, True),     # the H3 model: hidden 5,376, 56 heads, rot 96
    (200, 64, 2, 128, 0, False),      # one reduction step (no second stage loaded up front)
    (260, 192, 2, 128, 0, False),     # three steps: the last step's stage is the first's
    (129, 320, 4, 96, 1, True),       # five steps, S one row past a tile, fp32 rounding
    (1, 128, 2, 128, 0, False),       # a single token: one valid row in the last tile
    # Launch order (tile_order.h): 6 x 3 tiles, XCD lists of 4,4,4,2,2,2,0,0 (a full
    # chunk, short chunks of 2, two XCDs with no tile, 14 empty workgroups) ...
    (1500, 256, 2, 128, 0, False),
    # ... and 7 x 6 tiles, lists of 7,7,7,7,4,4,3,3 (full chunks and short chunks of 3
    # on the same XCD).
    (1700, 320, 4, 96, 1, True),
])
def test_fused_equals_prologue_of_plain(h3, orc, S, hidden, H, rot, rounding, h3t):
    x, w, plain, fused, (want_q, want_k) = _run(orc, S, hidden, H, rot, rounding, h3t)
    _check_plain(*plain, x, w, S)
    q, k, v = fused
    assert np.array_equal(bits(q), bits(want_q))
    assert np.array_equal(bits(k), bits(want_k))
    assert np.array_equal(bits(v), bits(plain[2]))


def test_strided_x_and_w_rows(h3, orc):
    """x and W as views with row stride > hidden (slices of wider buffers)."""
    x, w, plain, fused, (want_q, want_k) = _run(orc, 200, 384, 2, 128, 0, ldx=1024, ldw=448)
    assert x.stride(0) == 1024 and w.stride(0) == 448
    _check_plain(*plain, x, w, 200)
    assert np.array_equal(bits(fused[0]), bits(want_q))
    assert np.array_equal(bits(fused[1]), bits(want_k))


def test_cfg3_full_size(h3, orc):
    """Config 3 (S 31,885, hidden 5,120, 40 heads): fused == prologue(plain)
    everywhere; the plain GEMM checked against fp32 on sampled token rows."""
    from h3hip import configs as C, ops
    shape = C.CFG3
    S, H = shape.seq_len, shape.heads
    x, w = _inputs(S, 5120, H, 21)
    qg = to_gpu_bf16(orc.uniform_bf16((128,), 22, 0.9, 1.1))
    kg = to_gpu_bf16(orc.uniform_bf16((128,), 23, 0.9, 1.1))
    pos = torch.from_numpy(ops.positions_grid(shape.prefix_len, shape.frames, shape.height,
                                              shape.width)).cuda()
    axis, inv = (torch.from_numpy(t).cuda() for t in ops.rope_pairs_axes(10000.0, (32, 48, 48)))
    note("qkv_proj cfg3 plain")
    plain = ops.qkv_proj(x, w, heads=H)
    torch.cuda.synchronize()
    rng = np.random.default_rng(1)
    rows = np.unique(np.concatenate([np.arange(4), np.arange(S - 4, S), rng.integers(0, S, 60)]))
    _check_plain(*plain, x, w, S, rows=rows)
    note("qkv_proj cfg3 fused")
    fused = ops.qkv_proj(x, w, qg, kg, ops.rope_table(pos, axis, inv), heads=H, eps=1e-6)
    torch.cuda.synchronize()
    assert np.array_equal(bits(fused[2]), bits(plain[2]))
    q_tm = _token_major(plain[0], S)
    k_tm = _token_major(plain[1], S)
    del plain
    note("qkv_proj cfg3 prologue over plain")
    want_q, want_k, _ = ops.qk_norm_rope(q_tm, k_tm, qg, kg, pos, axis, inv, heads=H, eps=1e-6)
    torch.cuda.synchronize()
    assert torch.equal(fused[0].view(torch.int16), want_q.view(torch.int16))
    assert torch.equal(fused[1].view(torch.int16), want_k.view(torch.int16))


def test_larger_seq_pad_is_zero_filled(h3, orc):
    """A caller's seq_pad beyond the 128-row round-up: rows seq_len .. seq_pad
    of Q, K and V come out zero, rows below are the same as with the minimal
    seq_pad."""
    from h3hip import ops
    S, H = 150, 2
    x, w = _inputs(S, 256, H, 9)
    qg = to_gpu_bf16(orc.uniform_bf16((128,), 10, 0.9, 1.1))
    kg = to_gpu_bf16(orc.uniform_bf16((128,), 11, 0.9, 1.1))
    pos, axis, inv = _tables(orc, S, 128, False)
    table = ops.rope_table(pos, axis, inv)
    note("qkv_proj seq_pad 512 vs 256")
    big = [torch.full((H, 512, 128), 7.0, dtype=torch.bfloat16, device="cuda") for _ in range(3)]
    ops.qkv_proj(x, w, qg, kg, table, heads=H, seq_pad=512, out=tuple(big))
    small = ops.qkv_proj(x, w, qg, kg, table, heads=H, seq_pad=256)
    torch.cuda.synchronize()
    for b, sm in zip(big, small):
        assert torch.all(b[:, S:] == 0)
        assert torch.equal(b[:, :S].view(torch.int16), sm[:, :S].view(torch.int16))


@pytest.mark.parametrize("rot,rounding,h3t", [(128, 0, False), (128, 1, False), (96, 0, True),
                                               (96, 1, True)])
def test_rope_table_matches_oracle(h3, orc, rot, rounding, h3t):
    """h3hip_rope_table against orc_rope_table (cos/sin in double, rounded
    once): bf16 entries identical; fp32 entries within 2 ulp (the device
    sincosf is not correctly rounded); the [[c, -s], [s, c]] structure exact."""
    from h3hip import ops
    S = 300
    pos, axis, inv = _tables(orc, S, rot, h3t)
    pos = pos + 0.25 * (torch.arange(S, device="cuda", dtype=torch.float32)[:, None] % 3)
    note(f"rope_table vs oracle rot={rot} rounding={rounding}")
    got = ops.rope_table(pos, axis, inv, rot=rot, rounding=rounding)
    torch.cuda.synchronize()
    want = orc.rope_table(pos.cpu().numpy(), axis.cpu().numpy(), inv.cpu().numpy(), rot, rounding)
    assert got.shape == (S, rot // 2, 2, 2)
    g = got.reshape(S, rot // 2, 4)
    if rounding == 0:
        gb = g.view(torch.int16).cpu().numpy().view(np.uint16)
        same = np.mean(gb == want)
        print(f"rope table bf16 identical {same:.6f}")
        assert same >= 0.999
        assert np.array_equal(gb[..., 0], gb[..., 3]) and np.array_equal(gb[..., 1], gb[..., 2] ^ 0x8000)
    else:
        gf = g.cpu().numpy()
        ulp = np.abs(gf.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
        print(f"rope table fp32 max ulp {ulp.max()}")
        assert ulp.max() <= 2
        assert np.array_equal(gf[..., 0], gf[..., 3]) and np.array_equal(gf[..., 1], -gf[..., 2])


def test_declines_and_refusals(h3):
    from h3hip import ops
    from h3hip._lib import H3HIPError
    x = torch.zeros((16, 128), dtype=torch.bfloat16, device="cuda")
    # Odd head count and head_dim 64 decline (None); the caller runs its own GEMM.
    assert ops.qkv_proj(x, torch.zeros((3 * 3 * 128, 128), dtype=torch.bfloat16,
                                       device="cuda"), heads=3) is None
    assert ops.qkv_proj(x, torch.zeros((3 * 2 * 64, 128), dtype=torch.bfloat16, device="cuda"),
                        heads=2, head_dim=64) is None
    # hidden not a multiple of 32 declines.
    x2 = torch.zeros((16, 80), dtype=torch.bfloat16, device="cuda")
    assert ops.qkv_proj(x2, torch.zeros((768, 80), dtype=torch.bfloat16, device="cuda"),
                        heads=2) is None
    # seq_pad not a multiple of 128 is an error.
    with pytest.raises(H3HIPError):
        ops.qkv_proj(x, torch.zeros((768, 128), dtype=torch.bfloat16, device="cuda"), heads=2,
                     seq_pad=144)
