"""Torch-facing calls into libch3hip.

torch supplies device memory and the current HIP stream; every computation is
one of the library's HIP kernels. Inputs must already be on the GPU: there is
no host or torch fallback, and a declined call returns ``None`` so the caller
can run its own dense path, exactly as the reference's backends decline.
"""
from __future__ import annotations

import ctypes
import math

import numpy as np
import torch

from . import _lib as L
from .topology import TilePlan


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _require_gpu_bf16(name: str, t: torch.Tensor):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (no host fallback exists)")
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16, got {t.dtype}")


# ------------------------------------------------------------------ host tables

def rope_pairs_axes(theta: float = 10000.0, dims=(32, 48, 48)):
    """Per-pair (axis, inv_freq) for three-axis RoPE with the given channel split."""
    n = sum(dims) // 2
    ax = np.zeros(n, dtype=np.int32)
    inv = np.zeros(n, dtype=np.float32)
    got = L.lib().h3hip_rope_pairs_axes(theta, dims[0], dims[1], dims[2],
                                        ax.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                        inv.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    L.check(min(got, 0))
    return ax, inv


def rope_pairs_h3(inv_freq: np.ndarray):
    """H3RoPE's pair table from the checkpoint's inv_freq (H3Transformer.swift:64-78)."""
    f = np.ascontiguousarray(inv_freq, dtype=np.float32)
    ax = np.zeros(3 * len(f), dtype=np.int32)
    inv = np.zeros(3 * len(f), dtype=np.float32)
    got = L.lib().h3hip_rope_pairs_h3(f.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), len(f),
                                      ax.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                      inv.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    L.check(min(got, 0))
    return ax, inv


def positions_grid(prefix_len: int, frames: int, height: int, width: int) -> np.ndarray:
    pos = np.zeros((prefix_len + frames * height * width, 3), dtype=np.float32)
    got = L.lib().h3hip_positions_grid(prefix_len, frames, height, width,
                                       pos.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    L.check(min(got, 0))
    return pos


def positions_packed(text_tokens: int, audio_t: int, latent_t: int, latent_h: int,
                     latent_w: int, patch: int = 2) -> np.ndarray:
    n = text_tokens + 2 * audio_t + latent_t * (latent_h // patch) * (latent_w // patch)
    pos = np.zeros((n, 3), dtype=np.float64)
    got = L.lib().h3hip_positions_packed(text_tokens, audio_t, latent_t, latent_h, latent_w,
                                         patch,
                                         pos.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
    L.check(min(got, 0))
    return pos


# --------------------------------------------------------------------- prologue

def qk_norm_rope(q_in: torch.Tensor, k_in: torch.Tensor, q_gamma: torch.Tensor,
                 k_gamma: torch.Tensor, pos: torch.Tensor, pair_axis: torch.Tensor,
                 pair_inv: torch.Tensor, *, heads: int, head_dim: int = 128,
                 eps: float = 1e-6, rot: int | None = None, seq_pad: int | None = None,
                 v_in: torch.Tensor | None = None, rounding: int = L.ROUND_REFERENCE,
                 out=None):
    """Fused RMSNorm + RoPE + head-major relayout of token-major Q and K.

    q_in/k_in: [S, >= heads*head_dim] bf16 views sharing one row stride (e.g.
    slices of a fused qkv projection). Returns (q_out, k_out, v_out) as
    [heads, seq_pad, head_dim] bf16, or None when the geometry is declined."""
    for name, t in (("q_in", q_in), ("k_in", k_in), ("q_gamma", q_gamma),
                    ("k_gamma", k_gamma)):
        _require_gpu_bf16(name, t)
    if q_in.dim() != 2 or q_in.stride(1) != 1 or k_in.stride() != q_in.stride():
        raise ValueError("q_in and k_in must be row-major 2-D views with the same row stride")
    S = q_in.shape[0]
    seq_pad = seq_pad or ((S + L.TILE - 1) // L.TILE) * L.TILE
    rot = rot if rot is not None else 2 * pair_axis.numel()
    if v_in is not None:
        _require_gpu_bf16("v_in", v_in)
        if v_in.stride() != q_in.stride():
            raise ValueError("v_in must share q_in's row stride")
    for name, t, dt in (("pos", pos, torch.float32), ("pair_axis", pair_axis, torch.int32),
                        ("pair_inv", pair_inv, torch.float32)):
        if not t.is_cuda or t.dtype != dt or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous {dt} GPU tensor")
    if pos.dim() != 2 or pos.shape[0] < S or pos.shape[1] != 3:
        raise ValueError(f"pos must be [>= {S}, 3]")
    if pair_axis.numel() < rot // 2 or pair_inv.numel() < rot // 2:
        raise ValueError(f"pair tables must hold rot/2 = {rot // 2} entries")
    if q_in.shape[1] < heads * head_dim or seq_pad % 4 or seq_pad < S:
        raise ValueError("q_in narrower than heads*head_dim, or bad seq_pad")
    if out is None:
        dev = q_in.device
        shape = (heads, seq_pad, head_dim)
        q_out = torch.empty(shape, dtype=torch.bfloat16, device=dev)
        k_out = torch.empty(shape, dtype=torch.bfloat16, device=dev)
        v_out = torch.empty(shape, dtype=torch.bfloat16, device=dev) if v_in is not None else None
    else:
        q_out, k_out, v_out = out
        for t in (q_out, k_out) + ((v_out,) if v_in is not None else ()):
            if t.shape != (heads, seq_pad, head_dim) or not t.is_contiguous():
                raise ValueError("outputs must be contiguous [heads, seq_pad, head_dim]")
    rc = L.lib().h3hip_qk_norm_rope(_ptr(q_in), _ptr(k_in), q_in.stride(0), _ptr(v_in),
                                    _ptr(q_gamma), _ptr(k_gamma), eps, _ptr(pos),
                                    _ptr(pair_axis), _ptr(pair_inv), rot, rounding, S, seq_pad,
                                    heads, head_dim, _ptr(q_out), _ptr(k_out), _ptr(v_out),
                                    _stream(q_in))
    if L.check(rc, allow_declined=True) == L.DECLINED:
        return None
    return q_out, k_out, v_out


def head_major(x: torch.Tensor, *, heads: int, head_dim: int = 128, seq_pad: int | None = None,
               out: torch.Tensor | None = None):
    """Token-major [S, >= heads*head_dim] bf16 (row stride free, unit column
    stride) -> head-major [heads, seq_pad, head_dim], rows >= S zero: the
    materialised transpose of AttentionLayer.sdpa. Returns None when declined."""
    if x.dim() != 2 or x.stride(1) != 1 or x.shape[1] < heads * head_dim:
        raise ValueError(f"x must be a 2-D view [S, >= {heads * head_dim}] with unit column "
                         f"stride, got shape {tuple(x.shape)} strides {x.stride()}")
    S = x.shape[0]
    seq_pad = seq_pad or ((S + L.TILE - 1) // L.TILE) * L.TILE
    shape = (heads, seq_pad, head_dim)
    if out is not None:
        _require_out(out, shape, x.device)
    _require_gpu_bf16("x", x)
    if out is None:
        out = torch.empty(shape, dtype=torch.bfloat16, device=x.device)
    rc = L.lib().h3hip_head_major(_ptr(x), x.stride(0), S, seq_pad, heads, head_dim, _ptr(out),
                                  _stream(x))
    if L.check(rc, allow_declined=True) == L.DECLINED:
        return None
    return out


def rope_table(pos: torch.Tensor, pair_axis: torch.Tensor, pair_inv: torch.Tensor, *,
               rot: int | None = None, rounding: int = L.ROUND_REFERENCE,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """The render's rotation table (H3RoPE.rotationTable): [S, rot/2, 2, 2]
    holding [[c, -s], [s, c]], bf16 for REFERENCE rounding, fp32 for FP32."""
    for name, t, dt in (("pos", pos, torch.float32), ("pair_axis", pair_axis, torch.int32),
                        ("pair_inv", pair_inv, torch.float32)):
        if not t.is_cuda or t.dtype != dt or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous {dt} GPU tensor")
    rot = rot if rot is not None else 2 * pair_axis.numel()
    if pos.dim() != 2 or pos.shape[1] != 3:
        raise ValueError("pos must be [S, 3]")
    if pair_axis.numel() < rot // 2 or pair_inv.numel() < rot // 2:
        raise ValueError(f"pair tables must hold rot/2 = {rot // 2} entries")
    S = pos.shape[0]
    dt = torch.bfloat16 if rounding == L.ROUND_REFERENCE else torch.float32
    shape = (S, rot // 2, 2, 2)
    if out is None:
        out = torch.empty(shape, dtype=dt, device=pos.device)
    elif out.shape != shape or out.dtype != dt or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous {dt} tensor of shape {shape}")
    L.check(L.lib().h3hip_rope_table(_ptr(pos), _ptr(pair_axis), _ptr(pair_inv), rot, rounding,
                                     S, _ptr(out), _stream(pos)))
    return out


def qkv_proj(x: torch.Tensor, w: torch.Tensor, q_gamma: torch.Tensor | None = None,
             k_gamma: torch.Tensor | None = None, table: torch.Tensor | None = None, *,
             heads: int, head_dim: int = 128, eps: float = 1e-6,
             seq_pad: int | None = None, rounding: int = L.ROUND_REFERENCE, out=None):
    """QKV projection x . w^T with the Q/K norm + RoPE prologue in its epilogue.

    x: [S, hidden] bf16 (row stride free, unit column stride); w: [3*heads*head_dim,
    hidden] bf16 (Q | K | V rows); table: the render's rotation table from
    rope_table() for the same rounding mode ([>= S, rot/2, 2, 2]). With q_gamma =
    k_gamma = None this is the plain GEMM written head-major. Returns (q, k, v)
    as [heads, seq_pad, head_dim] bf16, or None when the geometry is declined."""
    _require_gpu_bf16("x", x)
    _require_gpu_bf16("w", w)
    if x.dim() != 2 or w.dim() != 2 or x.stride(1) != 1 or w.stride(1) != 1:
        raise ValueError("x and w must be 2-D with unit column stride")
    S, hidden = x.shape
    if w.shape != (3 * heads * head_dim, hidden):
        raise ValueError(f"w must be [{3 * heads * head_dim}, {hidden}], got {tuple(w.shape)}")
    seq_pad = seq_pad or ((S + L.TILE - 1) // L.TILE) * L.TILE
    plain = q_gamma is None and k_gamma is None
    if plain:
        rot = head_dim
    else:
        for name, t in (("q_gamma", q_gamma), ("k_gamma", k_gamma)):
            _require_gpu_bf16(name, t)
        dt = torch.bfloat16 if rounding == L.ROUND_REFERENCE else torch.float32
        if (table is None or not table.is_cuda or table.dtype != dt or not table.is_contiguous()
                or table.dim() != 4 or table.shape[0] < S or table.shape[2:] != (2, 2)):
            raise ValueError(f"table must be a contiguous {dt} [>= {S}, rot/2, 2, 2] GPU tensor "
                             "(rope_table() with the same rounding mode)")
        rot = 2 * table.shape[1]
    shape = (heads, seq_pad, head_dim)
    if out is None:
        q_out, k_out, v_out = (torch.empty(shape, dtype=torch.bfloat16, device=x.device)
                               for _ in range(3))
    else:
        q_out, k_out, v_out = out
        for t in (q_out, k_out, v_out):
            if t.shape != shape or not t.is_contiguous() or t.dtype != torch.bfloat16:
                raise ValueError("outputs must be contiguous bf16 [heads, seq_pad, head_dim]")
    rc = L.lib().h3hip_qkv_proj(_ptr(x), x.stride(0), _ptr(w), w.stride(0), hidden,
                                _ptr(q_gamma), _ptr(k_gamma), eps, _ptr(table), rot, rounding,
                                S, seq_pad, heads, head_dim, _ptr(q_out), _ptr(k_out),
                                _ptr(v_out), _stream(x))
    if L.check(rc, allow_declined=True) == L.DECLINED:
        return None
    return q_out, k_out, v_out


def out_proj(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None):
    """Out-projection y = x . w^T (DiTBlock.swift:359, matmul(merged,
    outWeight.T)): x [S, in_features] bf16 (the attention's token-major
    output), w [out_features, in_features] bf16; returns y [S, out_features]
    bf16 (or writes ``out``, any row stride), or None when declined."""
    _require_gpu_bf16("x", x)
    _require_gpu_bf16("w", w)
    if x.dim() != 2 or w.dim() != 2 or x.stride(1) != 1 or w.stride(1) != 1:
        raise ValueError("x and w must be 2-D with unit column stride")
    S, fin = x.shape
    if w.shape[1] != fin:
        raise ValueError(f"w must be [out_features, {fin}], got {tuple(w.shape)}")
    fout = w.shape[0]
    if out is None:
        out = torch.empty((S, fout), dtype=torch.bfloat16, device=x.device)
    elif (out.dim() != 2 or out.shape != (S, fout) or out.stride(1) != 1
          or out.dtype != torch.bfloat16 or not out.is_cuda):
        raise ValueError(f"out must be a bf16 GPU [{S}, {fout}] view with unit column stride")
    rc = L.lib().h3hip_out_proj(_ptr(x), x.stride(0), _ptr(w), w.stride(0), fin, fout, S,
                                _ptr(out), out.stride(0), _stream(x))
    if L.check(rc, allow_declined=True) == L.DECLINED:
        return None
    return out


# -------------------------------------------------------------------- attention

def _head_major_qkv(plan: TilePlan, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
    """q, k, v must be contiguous bf16 GPU tensors of one shape [H, seq_pad, D]:
    the kernel reads all H heads x D columns x seq_len rows of each. Returns (H, D).
    (A head count or head_dim the library does not take is declined by the library
    before anything is read.)"""
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not t.is_contiguous() or t.dim() != 3 or t.shape[1] != plan.seq_pad:
            raise ValueError(f"{name} must be contiguous [heads, {plan.seq_pad}, head_dim], "
                             f"got shape {tuple(t.shape)}")
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q, k and v must have one shape, got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    for name, t in (("q", q), ("k", k), ("v", v)):
        _require_gpu_bf16(name, t)
    return q.shape[0], q.shape[2]


def _require_out(out: torch.Tensor, shape, device):
    if (not isinstance(out, torch.Tensor) or out.dtype != torch.bfloat16 or out.device != device
            or not out.is_contiguous() or tuple(out.shape) != tuple(shape)):
        raise ValueError(f"out must be a contiguous bf16 tensor of shape {tuple(shape)} on "
                         f"{device}, got {getattr(out, 'shape', None)}")


def bsattn_fwd(plan: TilePlan, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
               scale: float | None = None, out_layout: int = L.OUT_HEAD_MAJOR,
               out: torch.Tensor | None = None):
    """Block-sparse attention over the plan's tiles; q/k/v [H, seq_pad, D] bf16.

    Returns the output tensor, or None when the call is declined."""
    H, D = _head_major_qkv(plan, q, k, v)
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    if out_layout not in (L.OUT_HEAD_MAJOR, L.OUT_TOKEN_MAJOR):
        raise ValueError(f"unknown out_layout {out_layout}")
    shape = (H, plan.seq_pad, D) if out_layout == L.OUT_HEAD_MAJOR else (plan.seq_pad, H * D)
    if out is None:
        out = torch.empty(shape, dtype=torch.bfloat16, device=q.device)
    else:
        _require_out(out, shape, q.device)
    rc = L.lib().h3hip_bsattn_fwd(plan.handle, _ptr(q), _ptr(k), _ptr(v), H, D, scale,
                                  _ptr(out), out_layout, _stream(q))
    if L.check(rc, allow_declined=True) == L.DECLINED:
        return None
    return out


def _views(q, k, v, out, S):
    """[heads, rows, head_dim] tensors -> h3hip_views (strides in elements). The
    kernel touches every head and all head_dim columns of rows < S of each, so
    every view must hold q's head count and head_dim and at least S rows."""
    if q.dim() != 3:
        raise ValueError(f"q must be a [heads, rows, head_dim] view, got shape {tuple(q.shape)}")
    H, _, D = q.shape
    named = (("q", q), ("k", k), ("v", v), ("out", out))
    for name, t in named:
        if (t.dim() != 3 or t.stride(2) != 1 or t.shape[0] != H or t.shape[2] != D
                or t.shape[1] < S):
            raise ValueError(f"{name} must be a [{H}, >= {S}, {D}] view with unit stride along "
                             f"head_dim, got shape {tuple(t.shape)} strides {t.stride()}")
    for name, t in named:
        _require_gpu_bf16(name, t)
    return [L.ViewC(t.data_ptr(), t.stride(0), t.stride(1)) for _, t in named]


def bsattn_fwd_strided(plan: TilePlan, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       scale: float | None = None, out: torch.Tensor | None = None):
    """Block-sparse attention on strided [heads, rows, head_dim] views.

    q, k, v may be views straight into a fused token-major projection (e.g.
    ``qkv.view(S, 3, H, D)[:, 2].transpose(0, 1)`` for V); only rows < S are
    read. ``out`` is a [heads, >= S, head_dim] view to write rows < S into;
    by default a token-major [S, heads*head_dim] tensor is allocated and
    returned. Returns None when the call is declined."""
    S = plan.seq_len
    if q.dim() != 3:
        raise ValueError(f"q must be a [heads, rows, head_dim] view, got shape {tuple(q.shape)}")
    H, _, D = q.shape
    ret = None
    if out is None:
        ret = torch.empty((S, H * D), dtype=torch.bfloat16, device=q.device)
        out = ret.view(S, H, D).transpose(0, 1)
    views = _views(q, k, v, out, S)
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    rc = L.lib().h3hip_bsattn_fwd_strided(plan.handle, ctypes.byref(views[0]),
                                          ctypes.byref(views[1]), ctypes.byref(views[2]), H, D,
                                          scale, ctypes.byref(views[3]), _stream(q))
    if L.check(rc, allow_declined=True) == L.DECLINED:
        return None
    return ret if ret is not None else out


def attend_strided(plan: TilePlan, context, q: torch.Tensor, k: torch.Tensor,
                   v: torch.Tensor, scale: float, out: torch.Tensor | None = None):
    """h3hip_attend_strided: policy + geometry checks, then the sparse kernel
    on [heads, rows, head_dim] views (rows >= S; unit stride along head_dim).

    ``out`` is a [heads, >= S, head_dim] view; by default a token-major
    [S, heads*head_dim] buffer is allocated and its [heads, S, head_dim] view
    returned. Returns None when the call is declined."""
    S = plan.seq_len
    if q.dim() != 3:
        raise ValueError(f"q must be a [heads, rows, head_dim] view, got shape {tuple(q.shape)}")
    H, _, D = q.shape
    if out is None:
        out = torch.empty((S, H * D), dtype=torch.bfloat16, device=q.device)
        out = out.view(S, H, D).transpose(0, 1)
    views = _views(q, k, v, out, S)
    cctx = None if context is None else ctypes.byref(context.to_c())
    rc = L.lib().h3hip_attend_strided(plan.handle, cctx, ctypes.byref(views[0]),
                                      ctypes.byref(views[1]), ctypes.byref(views[2]), H, D,
                                      scale, ctypes.byref(views[3]), _stream(q))
    if L.check(rc, allow_declined=True) == L.DECLINED:
        return None
    return out


def attend(plan: TilePlan, context, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
           scale: float, out: torch.Tensor | None = None):
    """h3hip_attend: policy + geometry checks, then the sparse kernel.

    ``context`` is an AttentionContext (or None, which declines). q, k, v are
    contiguous [heads, seq_pad, head_dim] like bsattn_fwd's; a given ``out``
    must be contiguous [heads, seq_pad, head_dim] bf16."""
    H, D = _head_major_qkv(plan, q, k, v)
    if out is None:
        out = torch.empty((H, plan.seq_pad, D), dtype=torch.bfloat16, device=q.device)
    else:
        _require_out(out, (H, plan.seq_pad, D), q.device)
    cctx = None if context is None else ctypes.byref(context.to_c())
    rc = L.lib().h3hip_attend(plan.handle, cctx, _ptr(q), _ptr(k), _ptr(v), H, D, scale,
                              _ptr(out), _stream(q))
    if L.check(rc, allow_declined=True) == L.DECLINED:
        return None
    return out
