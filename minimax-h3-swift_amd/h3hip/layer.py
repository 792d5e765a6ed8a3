"""AttentionLayer of the DiT block on MI355X (Sources/H3Modules/DiTBlock.swift).

Mirrors ``AttentionLayer.callAsFunction(_:ropeTable:context:)`` (:336-359):

    qkv = matmul(x, qkvWeight.T); q, k, v = split(qkv)          (:338-344)
    q = qNorm(q); k = kNorm(k)                                   (:346-347)
    if ropeTable: q, k = SplitHalfRoPE.apply(q/k, ropeTable)     (:348-351)
    merged = sdpa(q, k, v, context)                              (:356-357)
    return matmul(merged, outWeight.T)                           (:358)

with the projection and the norm/RoPE either fused in one kernel
(h3hip_qkv_proj) or run as hipBLASLt's GEMM followed by the prologue kernel
(h3hip_qk_norm_rope), the attention through the backend seam (block-sparse
kernel with a context, the reference's dense SDPA otherwise), and the
out-projection -- a plain GEMM -- on the projection kernel's main loop
(h3hip_out_proj), or on hipBLASLt when that kernel declines the shape. Q and K
come out head-major and V is read in place, so no relayout copy runs between
the stages.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib as L
from . import ops
from .backend import AttentionContext, H3AttentionBackend


@dataclass
class RopeState:
    """The render's rotation state (H3Transformer.swift:263-276, built once per
    render): the rotation table H3RoPE.rotationTable -- the ``ropeTable`` every
    layer takes -- and the (positions, pair) tables it comes from. The fused
    projection rotates with the table, the prologue kernel re-evaluates the same
    entries from the pair tables; both give the same bits."""
    pos: torch.Tensor          # [S, 3] fp32 (t, h, w)
    pair_axis: torch.Tensor    # [rot/2] int32
    pair_inv: torch.Tensor     # [rot/2] fp32
    rot: int
    rounding: int
    table: torch.Tensor        # [S, rot/2, 2, 2], bf16 (REFERENCE) or fp32

    @classmethod
    def build(cls, pos, pair_axis, pair_inv, rot: int | None = None,
              rounding: int = L.ROUND_REFERENCE) -> "RopeState":
        rot = rot if rot is not None else 2 * pair_axis.numel()
        table = ops.rope_table(pos, pair_axis, pair_inv, rot=rot, rounding=rounding)
        return cls(pos, pair_axis, pair_inv, rot, rounding, table)

    @classmethod
    def identity(cls, seq_len: int, head_dim: int, device,
                 rounding: int = L.ROUND_REFERENCE) -> "RopeState":
        """Position 0 everywhere: the rotation is the identity, bit for bit in
        both rounding modes -- the layer without a ropeTable."""
        pos = torch.zeros((seq_len, 3), dtype=torch.float32, device=device)
        half = head_dim // 2
        axis = torch.zeros(half, dtype=torch.int32, device=device)
        inv = torch.ones(half, dtype=torch.float32, device=device)
        return cls.build(pos, axis, inv, head_dim, rounding)


class AttentionLayer:
    """One DiT attention layer (DiTBlock.swift:262-359).

    qkv_weight: [3*heads*head_dim, hidden] bf16 (Q | K | V rows, as stored);
    out_weight: [hidden, heads*head_dim] bf16; q_gamma, k_gamma: [head_dim] bf16
    (qNorm, kNorm). ``projection`` picks the QKV path: "fused" (h3hip_qkv_proj)
    or "hipblaslt" (GEMM + h3hip_qk_norm_rope); either falls back to the other
    when its kernel declines the geometry."""

    def __init__(self, qkv_weight, out_weight, q_gamma, k_gamma, *, heads: int,
                 head_dim: int = 128, eps: float = 1e-5, backend: H3AttentionBackend | None = None,
                 projection: str = "hipblaslt"):
        if projection not in ("fused", "hipblaslt"):
            raise ValueError(f"projection must be 'fused' or 'hipblaslt', got {projection!r}")
        inner = heads * head_dim
        if qkv_weight.shape[0] != 3 * inner or out_weight.shape[1] != inner:
            raise ValueError("weights do not match heads * head_dim")
        self.qkv_weight, self.out_weight = qkv_weight, out_weight
        self.q_gamma, self.k_gamma = q_gamma, k_gamma
        self.heads, self.head_dim, self.eps = heads, head_dim, eps
        self.backend, self.projection = backend, projection

    # ---------------------------------------------------------------- stages

    def _project_fused(self, x, rope: RopeState, seq_pad: int):
        r = ops.qkv_proj(x, self.qkv_weight, self.q_gamma, self.k_gamma, rope.table,
                         heads=self.heads, head_dim=self.head_dim, eps=self.eps,
                         seq_pad=seq_pad, rounding=rope.rounding)
        if r is None:
            return None
        q, k, v = r
        S = x.shape[0]
        return q[:, :S], k[:, :S], v[:, :S]

    def _project_hipblaslt(self, x, rope: RopeState, seq_pad: int):
        S, inner = x.shape[0], self.heads * self.head_dim
        qkv = torch.mm(x, self.qkv_weight.t())
        r = ops.qk_norm_rope(qkv[:, :inner], qkv[:, inner:2 * inner], self.q_gamma,
                             self.k_gamma, rope.pos, rope.pair_axis, rope.pair_inv,
                             heads=self.heads, head_dim=self.head_dim, eps=self.eps, rot=rope.rot,
                             seq_pad=seq_pad, rounding=rope.rounding)
        if r is None:
            return None
        v = qkv[:, 2 * inner:].view(S, self.heads, self.head_dim).transpose(0, 1)
        return r[0][:, :S], r[1][:, :S], v

    def _attend(self, q, k, v, context: AttentionContext | None):
        """AttentionLayer.sdpa (DiTBlock.swift:280-328) on [H, S, D] views:
        the backend only with a context; a decline runs dense SDPA."""
        H, S, D = q.shape
        scale = 1.0 / math.sqrt(D)
        if self.backend is not None and context is not None:
            o = self.backend.attend(q, k, v, scale, None, context)
            if o is not None:
                return o.transpose(0, 1).reshape(S, H * D)
        # Dense: computed in fp32 one head at a time (at least as accurate as
        # a bf16 SDPA, which accumulates in fp32; keeps torch off its bf16
        # batched-product path; one [S, S] score matrix at a time), rounded to
        # the input dtype as the reference's sdpa returns it.
        out = torch.empty((S, H, D), dtype=q.dtype, device=q.device)
        for h in range(H):
            o = torch.nn.functional.scaled_dot_product_attention(
                q[h][None].float(), k[h][None].float(), v[h][None].float(), scale=scale)
            out[:, h] = o[0].to(q.dtype)
        return out.reshape(S, H * D)

    # ------------------------------------------------------------------ call

    def __call__(self, x: torch.Tensor, rope: RopeState | None,
                 context: AttentionContext | None = None) -> torch.Tensor:
        """x: [S, hidden] bf16 -> [S, hidden] bf16."""
        if x.dim() != 2:
            raise ValueError("x must be [S, hidden] (the packed-row layout)")
        S = x.shape[0]
        if rope is None:
            rope = RopeState.identity(S, self.head_dim, x.device)
        seq_pad = ((S + L.TILE - 1) // L.TILE) * L.TILE
        first, second = ((self._project_fused, self._project_hipblaslt)
                         if self.projection == "fused"
                         else (self._project_hipblaslt, self._project_fused))
        qkv = first(x, rope, seq_pad) or second(x, rope, seq_pad)
        if qkv is None:
            raise NotImplementedError(
                f"no kernel takes head_dim {self.head_dim} / rot {rope.rot} / heads {self.heads}")
        merged = self._attend(*qkv, context)
        y = ops.out_proj(merged, self.out_weight)
        if y is None:       # a width the kernel declines: hipBLASLt's GEMM
            y = torch.mm(merged, self.out_weight.t())
        return y
