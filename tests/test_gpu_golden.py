"""The GPU path against the committed golden vectors (tests/golden): inputs
regenerated bit-exactly from their seeds, outputs compared to what the oracle
stored -- attention within the north-star bar, the prologue bit for bit."""
import math
import os
import sys

import numpy as np
import pytest
import torch

from _gpu import bits, f32, note, to_gpu_bf16

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden  # noqa: E402


def test_attention_matches_the_golden_vector(h3, orc):
    from h3hip import ops
    note("golden attention h2 s600")
    z = np.load(os.path.join(HERE, "golden", "attn_h2_s600.npz"))
    S = make_golden.ATTN["seq_len"]
    plan = h3.TilePlan(h3.MaskRule.from_bitmap(S, z["bitmap"]), heads=2)
    q, k, v = (np.zeros((2, plan.seq_pad, 128), dtype=np.uint16) for _ in range(3))
    for dst, src in zip((q, k, v), make_golden.attn_inputs()):
        dst[:, :S] = src
    out = ops.bsattn_fwd(plan, to_gpu_bf16(q), to_gpu_bf16(k), to_gpu_bf16(v), 1.0 / math.sqrt(128))
    torch.cuda.synchronize()
    got = f32(out)[:, :S]
    want = orc.bf16_to_f32(z["out_bf16"])
    err = np.abs(got - want)
    print(f"golden attention: max-abs {err.max():.3e} mean-abs {err.mean():.3e}")
    assert err.max() < 2e-2 and err.mean() < 2e-3
    assert np.all(got[:, 256:384] == 0)


def test_prologue_matches_the_golden_vector_bit_for_bit(h3):
    from h3hip import ops
    note("golden prologue h2 s300")
    z = np.load(os.path.join(HERE, "golden", "prologue_h2_s300.npz"))
    S, inner, qkv, gq, gk, pos, ax, inv = make_golden.prologue_inputs()
    t = to_gpu_bf16(qkv)
    q, k, _ = ops.qk_norm_rope(t[:, :inner], t[:, inner:2 * inner], to_gpu_bf16(gq), to_gpu_bf16(gk),
                               torch.from_numpy(pos).cuda(), torch.from_numpy(ax).cuda(),
                               torch.from_numpy(inv).cuda(), heads=2, eps=make_golden.PROLOGUE["eps"])
    torch.cuda.synchronize()
    assert np.array_equal(bits(q)[:, :S], z["q"]) and np.array_equal(bits(k)[:, :S], z["k"])
