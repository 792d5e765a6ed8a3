"""The attention seam, mirrored from the reference so callers and tests read
the same: AttentionContext, the H3AttentionBackend protocol, the dense
fallback, the registry, and AttentionLayer.sdpa's dispatch
(Sources/H3Attention/AttentionBackend.swift:37-283,
Sources/H3Modules/DiTBlock.swift:293-328).

``H3HIPBackend`` is the product backend: every call goes to libch3hip. The
dense ``SDPABackend`` stands for the *caller's* fallback (MLX SDPA in the
reference) and is what a declined call lands on; it is never used by the
sparse path itself.
"""
from __future__ import annotations

import enum
import math
from dataclasses import dataclass
from typing import Optional, Sequence

import torch

from . import _lib as L
from .topology import TilePlan


@dataclass(frozen=True)
class AttentionContext:
    """Where in the render a call sits (AttentionBackend.swift:37-59)."""
    block_index: int
    block_count: int
    schedule_progress: float
    sequence_length: int
    video_span: Optional[range] = None

    def to_c(self) -> L.AttentionContextC:
        vs = self.video_span
        return L.AttentionContextC(self.block_index, self.block_count, self.schedule_progress,
                                   self.sequence_length, vs.start if vs is not None else -1,
                                   vs.stop if vs is not None else -1)


@dataclass(frozen=True)
class Machine:
    """The argument of isAvailable(on:) (Sources/H3Hardware/Machine.swift:12-40)."""
    chip: str
    device: int = 0


class TokenOrdering(enum.Enum):
    """AttentionBackend.swift:174-181."""
    none = "none"
    morton3D = "3d"
    mortonPerFrame = "2d_frame"


class H3AttentionBackend:
    """Protocol of AttentionBackend.swift:81-128. ``attend`` takes and returns
    [heads, S, headDim]; returning None declines and the caller runs dense."""
    identifier: str = ""
    equivalence_class: float = 0.0
    materialises_scores: bool = True
    prefers_morton_order: bool = False

    @classmethod
    def is_available(cls, machine: Machine) -> bool:
        raise NotImplementedError

    def attend(self, queries, keys, values, scale: float, mask, context: AttentionContext):
        raise NotImplementedError


class SDPABackend(H3AttentionBackend):
    """The dense fallback every decline lands on (AttentionBackend.swift:132-155).
    Never declines."""
    identifier = "sdpa"
    equivalence_class = 0.0
    materialises_scores = True
    prefers_morton_order = False

    @classmethod
    def is_available(cls, machine: Machine) -> bool:
        return True

    def attend(self, queries, keys, values, scale, mask, context):
        o = torch.nn.functional.scaled_dot_product_attention(
            queries.unsqueeze(0), keys.unsqueeze(0), values.unsqueeze(0), attn_mask=mask,
            scale=scale)
        return o.squeeze(0)


class H3HIPBackend(H3AttentionBackend):
    """Block-sparse attention on MI355X through libch3hip.

    ``equivalence_class`` (the relative-RMS band of AttentionBackend.swift:96-98)
    is the kernel's own class: its output against fp32 attention over the same
    tiles -- AxialReference.attend's definition of the sparse answer, and dense
    SDPA itself when every tile is active. 5e-3 is the gate; measured on seeded
    bf16 inputs at the benchmark shapes it is 2.3e-3 (bf16 rounding of the
    weights and of the output; tests/test_gpu_equivalence.py asserts it at
    cfg2, cfg3, cfg4 and the reference's axial shape, and against torch SDPA on
    a dense plan). How far a SPARSE plan lies from dense SDPA is a property of
    the topology and of the data, not of this kernel: on seeded N(0,1) inputs,
    whose attention is nearly uniform, it is of order 1, while the reference
    measures its own topology only on captured attention (AxialMeasureTests).
    ``topology_class`` holds that distance once it has been measured on
    captures (``python -m h3hip.measure``); until then a sparse plan's class
    against dense is unknown and ``class_against_dense`` says so (None).

    ``materialises_scores`` is False: no [S, S] buffer ever exists. The plan
    fixes the shape; any other shape is declined by the library, so the caller
    falls back to dense."""
    identifier = "h3hip"
    equivalence_class = 5e-3
    materialises_scores = False
    prefers_morton_order = False

    def __init__(self, plan: TilePlan | None = None, topology_class: float | None = None):
        self.plan = plan
        self.topology_class = topology_class

    def class_against_dense(self) -> float | None:
        """Relative-RMS band against dense SDPA: the kernel class for a dense
        plan, kernel + measured topology class for a sparse one, None when the
        topology has not been measured on real attention."""
        if self.plan is not None and self.plan.nnz == self.plan.n_tiles ** 2:
            return self.equivalence_class
        if self.topology_class is None:
            return None
        return self.equivalence_class + self.topology_class

    @classmethod
    def is_available(cls, machine: Machine) -> bool:
        try:
            return bool(L.lib().h3hip_device_supported(machine.device))
        except ImportError:
            return False

    def attend(self, queries, keys, values, scale, mask, context):
        """[H, S, D] bf16 views in (the transposed [S, H, D] arrays sdpa hands
        over, used in place), [H, S, D] view of a token-major [S, H*D] buffer
        out; None declines (another dtype, a mask, another shape, the policy)."""
        if (self.plan is None or mask is not None or not queries.is_cuda
                or queries.dtype != torch.bfloat16):
            return None
        from . import ops
        H, S, D = queries.shape
        if S != self.plan.seq_len:
            return None

        def in_place(t):
            # Rows must be 16-byte aligned with unit stride along D; anything
            # else is made contiguous first.
            ok = (t.dtype == torch.bfloat16 and t.stride(2) == 1 and t.stride(1) >= D
                  and t.stride(1) % 8 == 0 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0)
            return t if ok else t.contiguous()

        return ops.attend_strided(self.plan, context, in_place(queries), in_place(keys),
                                  in_place(values), scale)


@dataclass
class Selection:
    identifier: str
    equivalence_class: float
    materialises_scores: bool
    ordering: TokenOrdering
    backend: H3AttentionBackend
    reason: str


class NotImplementedBackend(Exception):
    """H3Error.notImplemented for the attention backend (AttentionBackend.swift:267-281)."""


class AttentionRegistry:
    """AttentionBackend.swift:188-283. Dense stays the default under 'auto';
    the sparse backend is an explicit request."""
    available: Sequence[type] = (SDPABackend, H3HIPBackend)

    @classmethod
    def resolve(cls, requested: str, machine: Machine, ordering: TokenOrdering | None = None,
                backends: Sequence[type] | None = None) -> Selection:
        backends = cls.available if backends is None else backends

        def make(t, reason):
            order = ordering if ordering is not None else (
                TokenOrdering.mortonPerFrame if t.prefers_morton_order else TokenOrdering.none)
            return Selection(t.identifier, t.equivalence_class, t.materialises_scores, order, t(),
                             reason)

        if requested == "auto":
            for t in backends:
                if t.is_available(machine):
                    return make(t, "auto-selected; highest-preference backend available here")
            return make(SDPABackend, "auto: nothing else available")
        match = [t for t in backends if t.identifier == requested]
        if not match:
            known = ", ".join(t.identifier for t in backends)
            raise NotImplementedBackend(
                f"attention backend '{requested}': this build registers: {known}")
        t = match[0]
        if not t.is_available(machine):
            raise NotImplementedBackend(
                f"attention backend '{requested}': not available on {machine.chip}; ask for "
                "'auto' to fall back explicitly rather than silently")
        return make(t, "requested explicitly")


def sampling_activation_bytes(packed_tokens: int, materialises_scores: bool = True) -> int:
    """MemoryPlan.samplingActivationBytes (Sources/H3Hardware/MemoryPlan.swift:105-118)
    with the backend's ``materialises_scores`` applied, as that comment asks: the
    linear term (residual stream, qkv, MLP working set: 1.6e6 B per packed token)
    always, the quadratic attention-score term (29 B per score) only for a backend
    that builds the [S, S] matrix. The reference fits both coefficients to MLX's
    measured peak; they are kept as fitted."""
    s = float(packed_tokens)
    linear = 1.6e6 * s
    quadratic = 2.9e1 * s * s if materialises_scores else 0.0
    return int(max(0.0, linear + quadratic))


def h3hip_resident_bytes(seq_len: int, heads: int, blocks: int, nnz: int, n_tiles: int,
                         head_dim: int = 128) -> int:
    """What the sparse backend itself keeps resident for a render: two
    token-major bf16 outputs [S, heads*head_dim] per block, used alternately
    by the block's successive calls (each consumed inside its sampling step's
    graph), and the plan's device lists -- row_ptr, col_idx and the persistent
    schedule, int32. Linear in S; no [S, S] term."""
    outputs = 2 * blocks * seq_len * heads * head_dim * 2
    lists = 4 * (n_tiles + 1 + nnz + heads * n_tiles + 257)
    return outputs + lists


def sdpa(q, k, v, head_dim: int, fp32: bool = False, backend: H3AttentionBackend | None = None,
         context: AttentionContext | None = None):
    """AttentionLayer.sdpa (DiTBlock.swift:293-328): [S, H, D] or [B, S, H, D]
    in, [S, H*D] or [B, S, H*D] out. The backend is consulted only with a
    context and no batch axis; a None answer falls back to dense."""
    at = torch.float32 if fp32 else q.dtype
    has_batch = q.dim() == 4
    if has_batch:
        qh, kh, vh = (t.transpose(1, 2).to(at) for t in (q, k, v))
    else:
        qh, kh, vh = (t.transpose(0, 1).unsqueeze(0).to(at) for t in (q, k, v))
    scale = 1.0 / math.sqrt(head_dim)
    o = None
    if backend is not None and context is not None and not has_batch:
        r = backend.attend(qh[0], kh[0], vh[0], scale, None, context)
        o = None if r is None else r.unsqueeze(0)
    if o is None:
        o = torch.nn.functional.scaled_dot_product_attention(qh, kh, vh, scale=scale)
    if has_batch:
        return o.transpose(1, 2).to(q.dtype).reshape(q.shape[0], q.shape[1], q.shape[2] * head_dim)
    return o.squeeze(0).transpose(0, 1).to(q.dtype).reshape(q.shape[0], q.shape[1] * head_dim)
