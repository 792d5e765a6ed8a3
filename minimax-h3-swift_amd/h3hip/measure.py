"""Per-span error of the axial topology against dense attention.

The protocol of AxialMeasureTests.axialErrorOnRealAttention
(Tests/H3AttentionTests/AxialMeasureTests.swift:54-98): for each landmark
count, the topology's density and the relative RMS error of the sparse output
against dense fp32 attention, over all rows, the prefix rows and the video
rows -- reported per span, never averaged. Here the sparse output is this
path's block-sparse kernel on the topology's tile plan, so the error also
carries the kernel's bf16 rounding and the tile-level OR-reduction (a tile is
kept if any pair in it is allowed), which only ever adds allowed pairs.

    python -m h3hip.measure CAPTURE_DIR [--frames 37 --height 15 --width 27]

The reference is explicit that synthetic inputs cannot answer the quality
question (AxialMeasureTests.swift:13-20); on them this only exercises the
machinery.
"""
from __future__ import annotations

import argparse
import math

import torch

from . import ops
from .capture import list_captures, load_qkv, parse_capture_name
from .topology import MaskRule, TilePlan, axial_token_density, landmark_frames


def rel_rms(got: torch.Tensor, want: torch.Tensor) -> float:
    """sqrt(mean((got - want)^2)) / sqrt(mean(want^2)) in fp32."""
    g, w = got.float(), want.float()
    return float(torch.sqrt(torch.mean((g - w) ** 2)) / torch.sqrt(torch.mean(w * w)))


def dense_fp32(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, seq_len: int, scale: float,
               chunk: int = 1024) -> torch.Tensor:
    """Unmasked attention in fp32 over the first seq_len rows of head-major
    tensors, computed in query chunks: [heads, seq_len, head_dim] fp32."""
    H, _, D = q.shape
    out = torch.empty((H, seq_len, D), dtype=torch.float32, device=q.device)
    for h in range(H):
        kh = k[h, :seq_len].float()
        vh = v[h, :seq_len].float()
        kt = kh.t().contiguous()
        for c0 in range(0, seq_len, chunk):
            c1 = min(seq_len, c0 + chunk)
            sc = torch.matmul(q[h, c0:c1].float(), kt) * scale
            out[h, c0:c1] = torch.matmul(torch.softmax(sc, dim=-1), vh)
    return out


def span_error(plan: TilePlan, q, k, v, prefix_len: int, want=None) -> dict:
    """Relative RMS of the block-sparse output over ``plan``'s tiles against
    dense fp32 attention, over all rows, the prefix rows and the video rows
    (the spans of AxialMeasureTests.swift:83-96) -- for any tile plan, e.g. the
    local-window rules of the benchmark shapes."""
    seq_len = plan.seq_len
    scale = 1.0 / math.sqrt(q.shape[2])
    if want is None:
        want = dense_fp32(q, k, v, seq_len, scale)
    got = ops.bsattn_fwd(plan, q, k, v, scale)[:, :seq_len]
    torch.cuda.synchronize()
    return dict(tile_density=plan.density, total=rel_rms(got, want),
                prefix=rel_rms(got[:, :prefix_len], want[:, :prefix_len]) if prefix_len else 0.0,
                video=rel_rms(got[:, prefix_len:], want[:, prefix_len:]))


def per_span_error(q, k, v, seq_len: int, prefix_len: int, frames: int, height: int, width: int,
                   landmark_counts=(2, 3, 5, 9), want=None):
    """Rows of (landmarks, token density, tile density, total, prefix, video)
    relative RMS errors of the block-sparse axial output against dense fp32."""
    H, _, D = q.shape
    if prefix_len + frames * height * width != seq_len:
        raise ValueError(f"lattice {frames}x{height}x{width} + prefix {prefix_len} != S {seq_len}")
    scale = 1.0 / math.sqrt(D)
    if want is None:
        want = dense_fp32(q, k, v, seq_len, scale)
    rows = []
    for n in landmark_counts:
        lm = landmark_frames(frames, n)
        plan = TilePlan(MaskRule.axial(prefix_len, frames, height, width, landmarks=lm), heads=H)
        try:
            got = ops.bsattn_fwd(plan, q, k, v, scale)[:, :seq_len]
            torch.cuda.synchronize()
            rows.append(dict(
                landmarks=n, landmark_frames=lm,
                density=axial_token_density(prefix_len, frames, height, width, lm),
                tile_density=plan.density,
                total=rel_rms(got, want),
                prefix=rel_rms(got[:, :prefix_len], want[:, :prefix_len]) if prefix_len else 0.0,
                video=rel_rms(got[:, prefix_len:], want[:, prefix_len:])))
        finally:
            plan.close()
    return rows


def format_rows(rows) -> str:
    lines = ["  landmarks  density  tiles    total    prefix    video"]
    for r in rows:
        lines.append(f"  {r['landmarks']:9d}   {r['density']:.3f}  {r['tile_density']:.3f}   "
                     f"{r['total']:.4f}   {r['prefix']:.4f}   {r['video']:.4f}")
    return "\n".join(lines)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("directory")
    ap.add_argument("--frames", type=int, default=37)
    ap.add_argument("--height", type=int, default=15)
    ap.add_argument("--width", type=int, default=27)
    ap.add_argument("--landmarks", default="2,3,5,9")
    args = ap.parse_args(argv)
    counts = tuple(int(x) for x in args.landmarks.split(","))
    files = list_captures(args.directory)
    if not files:
        print(f"no captures in {args.directory}")
        return 1
    video = args.frames * args.height * args.width
    for path in files:
        q, k, v, S = load_qkv(path)
        block, progress = parse_capture_name(path)
        if S < video:
            print(f"\n{path}: S={S} is shorter than the {video}-token lattice -- skipped")
            continue
        prefix = S - video
        print(f"\n{path}  block {block} progress {progress:.2f}  S={S} D={q.shape[2]}  "
              f"prefix rows 0..<{prefix} ({100.0 * prefix / S:.1f}%)")
        print(format_rows(per_span_error(q, k, v, S, prefix, args.frames, args.height,
                                         args.width, counts)))
        del q, k, v
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
