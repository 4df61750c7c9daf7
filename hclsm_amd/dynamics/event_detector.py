"""Event mask rule of the reference EventDetector (hclsm/dynamics/event_detector.py:160-170).

The detector network (multi-scale features, dilated convolutions, MLP head) is upstream of the
hot path; this is only the rule that turns probabilities into the (B, T) mask the event index
consumes, written without the reference's host synchronisation (`if ... .min() == 0`, :168).
"""

from __future__ import annotations

import torch


def event_mask_rule(event_probs: torch.Tensor, threshold_logit: torch.Tensor) -> torch.Tensor:
    """hard = probs > sigmoid(threshold_logit) (:163-164); straight-through mask
    hard - probs.detach() + probs (:165); if any row has no event, column 0 of EVERY row is set
    to 1 (:168-170).  Returns the (B, T) float mask."""
    threshold = torch.sigmoid(threshold_logit)
    hard = (event_probs > threshold).float()
    mask = hard - event_probs.detach() + event_probs
    if mask.shape[1] == 0:
        return mask
    any_empty = (hard.sum(dim=1).min() == 0)                    # stays on the device
    col0 = torch.where(any_empty, torch.ones_like(mask[:, 0]), mask[:, 0])
    return torch.cat([col0[:, None], mask[:, 1:]], dim=1)
