"""SlotTracker on MI355X: counterpart of hclsm/objects/slot_tracker.py.

Same parameters, names and initialisation as the reference module (:53-72), so its state dict loads
unchanged.

* Without autograd: the hclsm_slot_track_* C entries (pair MLP on MFMA pair tiles without the
  (B, N, N, 3D) pair tensor, Sinkhorn in registers, fused gather + GRU gates); compute in fp32, or bf16
  under a bf16 autocast.  ``track`` runs the whole frame loop of hclsm/model.py:229-252 in one call.
* With autograd, or for shapes outside those kernels (d_slot not a multiple of 64 or above 384, more than
  128 slots): the reference's math in torch ops on the GPU, with a HipFallbackWarning.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from hclsm_amd.kernels._common import require_gpu, warn_fallback
from hclsm_amd.kernels.slot_tracker import (SINKHORN_ITERS, SINKHORN_TEMPERATURE, TrackerWeights, track_cost,
                                            track_match, track_reorder_update, track_sequence, track_supported)


def sinkhorn_matching(cost: torch.Tensor, n_iters: int = SINKHORN_ITERS, temperature: float = SINKHORN_TEMPERATURE):
    """(perm, confidence) of the Sinkhorn-normalised exp(-cost / temperature) in torch ops
    (slot_tracker.py:15-43)."""
    log_alpha = -cost / max(temperature, 1e-6)
    for _ in range(n_iters):
        log_alpha = log_alpha - torch.logsumexp(log_alpha, dim=2, keepdim=True)
        log_alpha = log_alpha - torch.logsumexp(log_alpha, dim=1, keepdim=True)
    assignment = log_alpha.exp()
    return assignment.argmax(dim=2), assignment.max(dim=2).values


class SlotTracker(nn.Module):
    def __init__(self, config) -> None:
        super().__init__()
        self.d_slot = config.d_slot
        self.n_max_slots = config.n_max_slots
        d = config.d_slot
        self.match_mlp = nn.Sequential(nn.Linear(d * 3, d), nn.ReLU(), nn.Linear(d, d // 4), nn.ReLU(),
                                       nn.Linear(d // 4, 1))
        self.hidden_gru = nn.GRUCell(d, d)
        nn.init.orthogonal_(self.hidden_gru.weight_ih)
        nn.init.orthogonal_(self.hidden_gru.weight_hh)
        nn.init.zeros_(self.hidden_gru.bias_ih)
        nn.init.zeros_(self.hidden_gru.bias_hh)

    # ---- helpers
    @staticmethod
    def _dtype() -> torch.dtype:
        return torch.bfloat16 if (torch.is_autocast_enabled("cuda") and
                                  torch.get_autocast_dtype("cuda") == torch.bfloat16) else torch.float32

    def _needs_grad(self, *xs) -> bool:
        if not torch.is_grad_enabled():
            return False
        return any(x is not None and x.requires_grad for x in xs) or any(p.requires_grad for p in self.parameters())

    def _fused(self, N: int, *xs, sequence: bool = False) -> TrackerWeights | None:
        """The kernels' weights, or None (with a HipFallbackWarning) when this call runs torch ops."""
        dtype = self._dtype()
        if self._needs_grad(*xs):
            warn_fallback("SlotTracker", "autograd (the fused cost, match and GRU kernels have no backward)")
            return None
        if not track_supported(N, self.d_slot, dtype, sequence):
            warn_fallback("SlotTracker", f"shape outside the fused kernels (N={N}, d_slot={self.d_slot}, {dtype}"
                                         f"{', sequence' if sequence else ''})")
            return None
        return TrackerWeights.from_module(self, dtype)

    # ---- reference methods
    def _torch_cost(self, slots_t, slots_t1, alive_t, alive_t1):
        B, N, D = slots_t.shape
        s_t = torch.clamp(slots_t, -50, 50)
        s_t1 = torch.clamp(slots_t1, -50, 50)
        a = s_t[:, :, None, :].expand(B, N, N, D)
        b = s_t1[:, None, :, :].expand(B, N, N, D)
        score = self.match_mlp(torch.cat([a, b, (a - b).abs()], dim=-1)).squeeze(-1)
        score = score - 1e4 * (alive_t < 0.5).float()[:, :, None]
        score = score - 1e4 * (alive_t1 < 0.5).float()[:, None, :]
        return -score

    def compute_cost_matrix(self, slots_t, slots_t1, alive_t, alive_t1) -> torch.Tensor:
        """(B, N, N) matching cost, lower = better (slot_tracker.py:74-107)."""
        require_gpu("SlotTracker", slots_t, slots_t1, alive_t, alive_t1)
        W = self._fused(slots_t.shape[1], slots_t, slots_t1)
        if W is None:
            return self._torch_cost(slots_t, slots_t1, alive_t, alive_t1)
        return track_cost(slots_t, slots_t1, alive_t, alive_t1, W)

    def forward(self, slots_t, slots_t1, alive_t, alive_t1):
        """-> (perm (B, N) int64 indices into slots_t1, matched (B, N) in {0, 1}) (slot_tracker.py:109-135)."""
        cost = self.compute_cost_matrix(slots_t, slots_t1, alive_t, alive_t1)
        if not cost.requires_grad and cost.shape[1] <= 128:
            perm, matched, _ = track_match(cost, alive_t, alive_t1)
            return perm, matched
        warn_fallback("SlotTracker", "Sinkhorn matching as torch ops (autograd through the cost, or more than "
                                     "128 slots)")
        perm, confidence = sinkhorn_matching(torch.clamp(cost, -1e4, 1e4))
        matched = ((alive_t > 0.5).float() * (alive_t1 > 0.5).float().gather(1, perm) *
                   (confidence > 0.3).float())
        return perm, matched

    def reorder_and_update(self, slots_t1, perm, hidden_t, matched):
        """-> (slots_t1 reordered by perm, next hidden state) (slot_tracker.py:137-158)."""
        require_gpu("SlotTracker", slots_t1, perm, hidden_t, matched)
        B, N, D = slots_t1.shape
        W = self._fused(N, slots_t1, hidden_t)
        if W is not None:
            re, h1 = track_reorder_update(slots_t1, perm, hidden_t, matched, W)
            return re.to(slots_t1.dtype), h1.to(hidden_t.dtype)
        reordered = slots_t1.gather(1, perm.unsqueeze(-1).expand(B, N, D))
        h1 = self.hidden_gru(reordered.reshape(-1, D), hidden_t.reshape(-1, D)).reshape(B, N, D)
        m = matched.unsqueeze(-1)
        return reordered, m * h1 + (1 - m) * reordered

    def track(self, slots: torch.Tensor, alive: torch.Tensor, return_hidden: bool = False):
        """The tracking loop of hclsm/model.py:229-252: slots (B, T, N, D), alive (B, T, N) -> (tracked slots
        (B, T, N, D), alive reordered alongside (B, T, N)[, final hidden state (B, N, D)])."""
        require_gpu("SlotTracker", slots, alive)
        B, T, N, D = slots.shape
        W = self._fused(N, slots, sequence=True)
        if W is not None:
            r = track_sequence(slots, alive, W, with_hidden=return_hidden)
            out = (r["tracked"].to(slots.dtype), r["alive"].to(alive.dtype))
            return out + (r["hidden"],) if return_hidden else out
        hidden = torch.zeros(B, N, D, device=slots.device)
        tracked, alive_frames = [slots[:, 0]], [alive[:, 0]]
        for t in range(1, T):
            perm, matched = self(tracked[t - 1], slots[:, t], alive_frames[t - 1], alive[:, t])
            reordered, hidden = self.reorder_and_update(slots[:, t], perm, hidden, matched)
            tracked.append(reordered)
            alive_frames.append(alive[:, t].gather(1, perm.long()))
        out = (torch.stack(tracked, dim=1), torch.stack(alive_frames, dim=1))
        return out + (hidden,) if return_hidden else out
