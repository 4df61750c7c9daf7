"""Hierarchy manager on MI355X: counterpart of hclsm/dynamics/hierarchy_manager.py.

gather_events / scatter_events run on the device-built int32 event index and the byte-exact
gather / scatter kernels (rule mask > 0.5, ascending event order, exact zero padding).  Without
autograd, forward() and forward_packed() on fp32 states are one hclsm_event_top_down call: the
scatter, the Level-2 top-down gate and its blend, and the alive mask in one pass over the rows, the
gate GEMM in fp32, or in bf16 / fp16 operands under an autocast of that type.  With autograd (or
shapes outside that kernel) the gating is the reference's torch math.  gather_events still returns
K_max as a Python int, as the reference does (:63), which costs one host read of the index
statistics; the packed counterparts (gather_events_packed, forward_packed, level1_events_packed)
need none.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from hclsm_amd.kernels._common import warn_fallback
from hclsm_amd.kernels.sparse_event_attn import (EventIndex, build_event_index, gather_events_packed,
                                                 gather_events_padded, pad_mask_from_index,
                                                 scatter_events_packed, scatter_events_padded)
from hclsm_amd.kernels.top_down import TopDownWeights, event_top_down, top_down_supported


class HierarchyManager(nn.Module):
    def __init__(self, d_slot: int, d_l2: int) -> None:
        super().__init__()
        self.d_slot = d_slot
        self.l2_to_l1 = nn.Linear(d_l2, d_slot, bias=False)
        self.gate_l0 = nn.Sequential(nn.Linear(d_slot * 2, d_slot), nn.Sigmoid())
        self.gate_l2_l0 = nn.Sequential(nn.Linear(d_slot * 2, d_slot), nn.Sigmoid())

    def gather_events(self, states: torch.Tensor, event_mask: torch.Tensor):
        """(B, T, N, D) -> (event_states (B, K_max, N, D), pad mask (B, K_max) float, K_max) (:42-77)."""
        idx = build_event_index(event_mask, "gt_half")
        K_max = max(idx.kmax(), 1)
        ev = gather_events_padded(states, idx, K_max)
        return ev, pad_mask_from_index(idx, K_max, torch.float32), K_max

    def scatter_events(self, base_states: torch.Tensor, event_updates: torch.Tensor,
                       event_mask: torch.Tensor) -> torch.Tensor:
        """Level-1 outputs override Level-0 at event timesteps (:79-118)."""
        idx = build_event_index(event_mask, "gt_half")
        return scatter_events_padded(base_states, event_updates, idx)

    def forward(self, level0_states, level1_states, level2_context, event_mask, obj_mask=None):
        if self._fused_ok(level0_states, level1_states, level2_context, obj_mask):
            idx = build_event_index(event_mask, "gt_half")
            return self._fused(level0_states, level1_states, idx, level2_context, obj_mask,
                               kpad=max(level1_states.shape[1], 1))
        combined = self.scatter_events(level0_states, level1_states, event_mask)      # :143
        return self._top_down(combined, level2_context, obj_mask)

    # ---- fused output step (hclsm_event_top_down)

    def _fused_ok(self, level0_states, level1_states, level2_context, obj_mask) -> bool:
        xs = (level0_states, level1_states, level2_context, obj_mask)
        if torch.is_grad_enabled() and (any(x is not None and x.requires_grad for x in xs) or
                                        any(p.requires_grad for p in self.parameters())):
            warn_fallback("HierarchyManager", "autograd (the fused top-down output step has no backward)")
            return False
        if not level0_states.is_cuda:
            return False   # the torch path runs HIP kernels only on the GPU; CPU tensors raise there
        if level0_states.dtype != torch.float32:
            warn_fallback("HierarchyManager", f"{level0_states.dtype} Level-0 states (the fused top-down output "
                                              "step takes float32)")
            return False
        if level1_states.shape[1] == 0:
            warn_fallback("HierarchyManager", "no event rows (the fused top-down output step takes at least one)")
            return False
        dl2 = None if level2_context is None else level2_context.shape[-1]
        if not top_down_supported(level0_states.shape[-1], dl2):
            warn_fallback("HierarchyManager", "a shape outside the fused top-down output step")
            return False
        return True

    def _fused(self, level0_states, level1_states, idx, level2_context, obj_mask, kpad):
        dtype = torch.float32
        if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") in (torch.bfloat16, torch.float16):
            dtype = torch.get_autocast_dtype("cuda")
        W = TopDownWeights.from_module(self, dtype) if level2_context is not None else None
        return event_top_down(level0_states, level1_states, idx, W, level2_context, obj_mask, kpad=kpad)

    def _top_down(self, combined, level2_context, obj_mask):
        if level2_context is not None:                                                # :146-156
            l2_proj = self.l2_to_l1(level2_context.mean(dim=1))
            l2b = l2_proj[:, None, None, :].expand_as(combined)
            gate = self.gate_l2_l0(torch.cat([combined, l2b], dim=-1))
            combined = gate * l2b + (1 - gate) * combined
        if obj_mask is not None:                                                      # :159-160
            combined = combined * obj_mask[:, None, :, None]
        return combined

    # ---- packed, sync-free counterparts (no K_max host read)

    def gather_events_packed(self, states: torch.Tensor, event_mask: torch.Tensor):
        """(B, T, N, D) -> (packed event states (B*T, N, D), index): event e < index.total() in row e; the rows
        after are zero in grad mode, unspecified otherwise.  Differentiable; no host sync."""
        idx = build_event_index(event_mask, "gt_half")
        return gather_events_packed(states, idx), idx

    def forward_packed(self, level0_states, level1_packed, index: EventIndex, level2_context=None,
                       obj_mask=None):
        """forward() with Level-1 outputs in the packed layout of gather_events_packed."""
        if self._fused_ok(level0_states, level1_packed, level2_context, obj_mask):
            return self._fused(level0_states, level1_packed, index, level2_context, obj_mask, kpad=0)
        combined = scatter_events_packed(level0_states, level1_packed, index)
        return self._top_down(combined, level2_context, obj_mask)


def level1_events_packed(hierarchy: HierarchyManager, level1, level0_states: torch.Tensor,
                         event_mask: torch.Tensor, obj_mask: torch.Tensor | None = None,
                         level2_context: torch.Tensor | None = None) -> torch.Tensor:
    """The Level-1 step of the reference model (model.py:298-310: gather_events, level1_event,
    hierarchy_manager) on packed events, without host synchronisation: event index on the device,
    packed gather, Level-1 over the live events only, packed scatter plus the top-down gating.
    Returns the combined (B, T, N, D) states.  (Level-2 consumes the padded gather and is not on
    this path.)"""
    ev, idx = hierarchy.gather_events_packed(level0_states, event_mask)
    out = level1.forward_packed(ev, idx, obj_mask)
    return hierarchy.forward_packed(level0_states, out, idx, level2_context, obj_mask)
