"""Hierarchy manager on MI355X: counterpart of hclsm/dynamics/hierarchy_manager.py.

gather_events / scatter_events run on the device-built int32 event index and the byte-exact
gather / scatter kernels (rule mask > 0.5, ascending event order, exact zero padding); the
top-down gating of forward() is unchanged torch math.  gather_events still returns K_max as a
Python int, as the reference does (:63), which costs one host read of the index statistics.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from hclsm_amd.kernels.sparse_event_attn import (build_event_index, gather_events_padded,
                                                 pad_mask_from_index, scatter_events_padded)


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
        combined = self.scatter_events(level0_states, level1_states, event_mask)      # :143
        if level2_context is not None:                                                # :146-156
            l2_proj = self.l2_to_l1(level2_context.mean(dim=1))
            l2b = l2_proj[:, None, None, :].expand_as(combined)
            gate = self.gate_l2_l0(torch.cat([combined, l2b], dim=-1))
            combined = gate * l2b + (1 - gate) * combined
        if obj_mask is not None:                                                      # :159-160
            combined = combined * obj_mask[:, None, :, None]
        return combined
