"""h3hip_head_major: the materialised [S, H, D] -> [H, S, D] transpose of
AttentionLayer.sdpa (DiTBlock.swift:297-300). A pure copy, so the check is bit
equality with torch's own transpose of the same bf16 words, rows >= S zero."""
import pytest
import torch

from _gpu import note, randn_bf16_gpu

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("S,H,ld_mult", [(1, 1, 1), (5, 3, 1), (128, 2, 3), (300, 40, 3),
                                         (1000, 7, 2), (31885, 40, 3)])
def test_matches_torch_transpose(h3, S, H, ld_mult):
    from h3hip import ops
    D = 128
    buf = randn_bf16_gpu((S, ld_mult * H * D), seed=S + H)
    x = buf[:, (ld_mult - 1) * H * D:]          # the last H*D columns: V of a fused Q|K|V
    note(f"head_major S={S} H={H} ld={buf.stride(0)}")
    out = ops.head_major(x, heads=H)
    torch.cuda.synchronize()
    S_pad = (S + 127) // 128 * 128
    assert out.shape == (H, S_pad, D)
    want = x.reshape(S, H, D).transpose(0, 1)
    assert torch.equal(out[:, :S].view(torch.int16), want.contiguous().view(torch.int16))
    assert torch.all(out[:, S:].view(torch.int16) == 0)


def test_larger_seq_pad_and_given_out(h3):
    from h3hip import ops
    S, H = 200, 4
    x = randn_bf16_gpu((S, H * 128), seed=3)
    out = torch.full((H, 512, 128), 3.0, dtype=torch.bfloat16, device="cuda")
    note("head_major seq_pad 512")
    r = ops.head_major(x, heads=H, seq_pad=512, out=out)
    torch.cuda.synchronize()
    assert r is out
    assert torch.equal(out[:, :S], x.view(S, H, 128).transpose(0, 1))
    assert torch.all(out[:, S:] == 0)


def test_declines_head_dim_64(h3):
    from h3hip import ops
    x = torch.zeros((16, 256), dtype=torch.bfloat16, device="cuda")
    assert ops.head_major(x, heads=4, head_dim=64) is None
