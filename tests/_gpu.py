"""Helpers shared by the GPU tests (bf16 bit-pattern transfer, seeded inputs)."""
import sys

import numpy as np
import torch


def note(msg: str):
    """Names the case before a GPU step, flushed, so a crash log says where."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def dev():
    return torch.device("cuda:0")


def to_gpu_bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(dev())


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def randn_bf16_gpu(shape, seed: int, scale: float = 1.0) -> torch.Tensor:
    g = torch.Generator(device=dev())
    g.manual_seed(seed)
    return (torch.randn(shape, generator=g, device=dev(), dtype=torch.float32) * scale).to(torch.bfloat16)


def head_major_inputs(H, S, S_pad, D, seed, pad_value=0.0):
    """q, k, v [H, S_pad, D] bf16 ~ N(0,1); rows >= S hold pad_value."""
    out = []
    for i in range(3):
        t = randn_bf16_gpu((H, S_pad, D), seed + i)
        if S_pad > S:
            t[:, S:] = pad_value
        out.append(t)
    return out


def err_stats(got: np.ndarray, want: np.ndarray):
    d = np.abs(got.astype(np.float64) - want.astype(np.float64))
    return float(d.max()), float(d.mean())
