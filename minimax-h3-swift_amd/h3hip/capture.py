"""Captured q/k/v of a real render, in the reference's capture format.

AttentionLayer.maybeCapture (Sources/H3Modules/DiTBlock.swift:226-254) writes
one safetensors file per (block, schedule progress), named
``qkv_blockNN_pX.XX.safetensors``, holding ``q``, ``k`` and ``v`` as
``[S, heads, head_dim]``. ``load_qkv`` reads such a file into this path's
head-major device layout, ``[heads, seq_pad, 128]`` bf16 with zero padding
rows, the layout ``ops.bsattn_fwd`` takes. The safetensors loader executes
nothing from the file.
"""
from __future__ import annotations

import os
import re

import torch
from safetensors import safe_open
from safetensors.torch import save_file

from ._lib import TILE

_NAME = re.compile(r"^qkv_block(\d+)_p(\d+\.\d+)\.safetensors$")


def capture_name(block: int, progress: float) -> str:
    """The file name the reference gives a capture (DiTBlock.swift:239-240)."""
    return f"qkv_block{block:02d}_p{progress:.2f}.safetensors"


def parse_capture_name(name: str):
    """(block, progress) of a capture file name, or None for other files."""
    m = _NAME.match(os.path.basename(name))
    return (int(m.group(1)), float(m.group(2))) if m else None


def list_captures(directory: str) -> list[str]:
    """Capture files in a directory, ordered by (block, progress)."""
    names = [n for n in os.listdir(directory) if parse_capture_name(n)]
    names.sort(key=parse_capture_name)
    return [os.path.join(directory, n) for n in names]


def save_qkv(path: str, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """Writes [S, heads, head_dim] tensors in the capture format."""
    for t in (q, k, v):
        if t.dim() != 3 or t.shape != q.shape:
            raise ValueError("q, k, v must share one [S, heads, head_dim] shape")
    save_file({n: t.detach().cpu().clone().contiguous() for n, t in (("q", q), ("k", k), ("v", v))},
              path)


def load_qkv(path: str, device="cuda"):
    """Reads a capture into head-major bf16 [heads, seq_pad, head_dim] tensors on
    `device`, rows >= S zero. Returns (q, k, v, S)."""
    with safe_open(path, framework="pt", device="cpu") as f:
        keys = set(f.keys())
        if not {"q", "k", "v"} <= keys:
            raise ValueError(f"{path}: a capture holds q, k and v; found {sorted(keys)}")
        raw = [f.get_tensor(n) for n in ("q", "k", "v")]
    if raw[0].dim() != 3 or any(t.shape != raw[0].shape for t in raw):
        raise ValueError(f"{path}: q, k, v must share one [S, heads, head_dim] shape")
    S, H, D = raw[0].shape
    s_pad = (S + TILE - 1) // TILE * TILE
    out = []
    for t in raw:
        hm = torch.zeros((H, s_pad, D), dtype=torch.bfloat16, device=device)
        hm[:, :S] = t.to(device=device, dtype=torch.bfloat16).transpose(0, 1)
        out.append(hm)
    return out[0], out[1], out[2], S
