"""Hierarchy manager output step in one C call (``hclsm_event_top_down``).

Counterpart of ``HierarchyManager.forward`` (hclsm/dynamics/hierarchy_manager.py:120-162) after the
Level-1 pass: the scatter of the Level-1 rows into the Level-0 states, the Level-2 top-down gate
(sigmoid of a Linear over [combined; l2_to_l1(mean context)]) with its blend, and the alive mask, fused
into one pass over the (B, T, N, D) rows plus a per-clip prologue.  The concatenation is never formed
(the Level-2 half of the gate is one bias vector per clip) and the scattered states are never written.
Inference only, fp32 states; the gate GEMM runs in fp32, or in bf16 / fp16 operands.
"""

from __future__ import annotations

import torch

from hclsm_amd import _lib
from hclsm_amd.kernels._common import require_gpu
from hclsm_amd.kernels.sparse_event_attn import EventIndex

_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


class TopDownWeights:
    """A HierarchyManager's parameters as hclsm_event_top_down takes them: l2_to_l1.weight [D, DL2] and
    gate_l2_l0.0.weight [D, 2D] / bias [D] in fp32, plus the gate's combined half W[:, :D] in the operand
    dtype (for fp32 the full matrix with row stride 2D)."""

    def __init__(self, w_l2, w_gate, b_gate, w_x, ldw, dtype, d_slot):
        self.w_l2, self.w_gate, self.b_gate, self.w_x, self.ldw = w_l2, w_gate, b_gate, w_x, ldw
        self.dtype, self.d_slot = dtype, d_slot

    @staticmethod
    def _key(m, dtype):
        return (dtype,) + tuple((p.data_ptr(), p._version) for p in m.parameters())

    @classmethod
    def from_tensors(cls, w_l2: torch.Tensor, w_gate: torch.Tensor, b_gate: torch.Tensor | None,
                     dtype: torch.dtype = torch.float32) -> "TopDownWeights":
        """From l2_to_l1.weight (D, d_l2), gate_l2_l0.0.weight (D, 2D) and its bias (D,) or None."""
        D = w_gate.shape[0]
        if tuple(w_gate.shape) != (D, 2 * D) or w_l2.dim() != 2 or w_l2.shape[0] != D:
            raise ValueError(f"gate weight must be (D, 2D) and l2_to_l1 (D, d_l2); got {tuple(w_gate.shape)}, "
                             f"{tuple(w_l2.shape)}")
        w_gate = w_gate.detach().float().contiguous()
        b_gate = None if b_gate is None else b_gate.detach().float().contiguous()
        w_l2 = w_l2.detach().float().contiguous()
        if dtype == torch.float32:
            w_x, ldw = w_gate, 2 * D
        else:
            w_x, ldw = w_gate[:, :D].to(dtype).contiguous(), D
        return cls(w_l2, w_gate, b_gate, w_x, ldw, dtype, D)

    @classmethod
    def from_module(cls, m, dtype: torch.dtype = torch.float32) -> "TopDownWeights":
        """From a HierarchyManager-shaped module (attribute names of hierarchy_manager.py:27-40); cached on the
        module until a parameter changes."""
        key = cls._key(m, dtype)
        hit = getattr(m, "_hclsm_top_down_weights", None)
        if hit is not None and hit[0] == key:
            return hit[1]
        lin = m.gate_l2_l0[0]
        W = cls.from_tensors(m.l2_to_l1.weight, lin.weight, lin.bias, dtype)
        m._hclsm_top_down_weights = (key, W)
        return W


def top_down_supported(d_slot: int, level2_dim: int | None = None) -> bool:
    """Shapes hclsm_event_top_down takes: d_slot a multiple of 32 up to 384, d_l2 up to 16384."""
    if d_slot % 32 != 0 or not 0 < d_slot <= 384:
        return False
    return level2_dim is None or 0 < level2_dim <= 16384


def event_top_down(level0: torch.Tensor, events: torch.Tensor, idx: EventIndex, W: TopDownWeights | None,
                   level2_context: torch.Tensor | None = None, obj_mask: torch.Tensor | None = None,
                   kpad: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    """level0 (B, T, N, D) fp32; events the Level-1 rows, packed (capacity, N, D) as gather_events_packed lays
    them out (kpad = 0) or padded (B, kpad, N, D); idx the event index of the mask; level2_context
    (B, S2, d_l2) or None; obj_mask (B, N) or None.  Returns the (B, T, N, D) fp32 output of
    HierarchyManager.forward.  No host sync."""
    require_gpu("event_top_down", level0, events, level2_context, obj_mask)
    B, T, N, D = level0.shape
    if (idx.B, idx.T) != (B, T):
        raise ValueError(f"event index is for ({idx.B}, {idx.T}) frames, level0 has ({B}, {T})")
    want = (B, kpad, N, D) if kpad > 0 else None
    if kpad > 0 and tuple(events.shape) != want:
        raise ValueError(f"padded Level-1 rows must be {want}, got {tuple(events.shape)}")
    if kpad == 0 and (events.dim() != 3 or tuple(events.shape[1:]) != (N, D) or events.shape[0] < 1):
        raise ValueError(f"packed Level-1 rows must be (capacity, {N}, {D}), got {tuple(events.shape)}")
    x = level0.contiguous().float()
    ev = events.contiguous().float()
    om = None if obj_mask is None else obj_mask.contiguous().float()
    if om is not None and tuple(om.shape) != (B, N):
        raise ValueError(f"obj_mask must be ({B}, {N}), got {tuple(om.shape)}")
    if out is None:
        out = torch.empty_like(x)
    ctx = ws = None
    S2 = DL2 = 0
    dtype = _lib.F32
    if level2_context is not None:
        if W is None:
            raise ValueError("event_top_down: a level2_context needs the gate weights")
        ctx = level2_context.contiguous().float()
        if ctx.dim() != 3 or ctx.shape[0] != B or ctx.shape[2] != W.w_l2.shape[1]:
            raise ValueError(f"level2_context must be ({B}, S2, {W.w_l2.shape[1]}), got {tuple(ctx.shape)}")
        S2, DL2 = ctx.shape[1], ctx.shape[2]
        nb = _lib.lib().hclsm_event_top_down_workspace(B, D)
        _lib.check(0 if nb >= 0 else int(nb), "hclsm_event_top_down_workspace")
        ws = torch.empty(max(nb // 4, 1), dtype=torch.float32, device=x.device)
        dtype = _DT[W.dtype]
    rc = _lib.lib().hclsm_event_top_down(
        _lib.ptr(x), _lib.ptr(ev), idx.ptr("offsets"), idx.ptr("slot_of"), kpad, _lib.ptr(ctx), S2, DL2,
        _lib.ptr(W.w_l2) if ctx is not None else None, _lib.ptr(W.w_gate) if ctx is not None else None,
        _lib.ptr(W.b_gate) if ctx is not None else None, _lib.ptr(W.w_x) if ctx is not None else None,
        W.ldw if ctx is not None else 0, _lib.ptr(om), _lib.ptr(out), B, T, N, D, dtype, _lib.ptr(ws),
        0 if ws is None else ws.numel() * 4, _lib.stream_of(x))
    _lib.check(rc, "hclsm_event_top_down")
    return out
