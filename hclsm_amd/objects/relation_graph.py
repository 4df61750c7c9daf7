"""RelationGraph on MI355X: counterpart of hclsm/objects/relation_graph.py.

Same parameters and names as the reference module (:23-66), so its state dict loads unchanged.

* Without autograd: one call of ``hclsm_relation_graph_forward`` (pair LayerNorm folded into the first
  edge layer, the edge MLP / weight / messages / causal head fused per pair tile on MFMA, node update on
  the MFMA linear kernels); compute in fp32, or bf16 under a bf16 autocast.  Shapes outside that kernel
  (fp32 operands with more than 64 slots, D or d_edge not multiples of 32, d_edge > 192) run the torch
  path below on the GPU, with a HipFallbackWarning.
* With autograd: the reference's math in torch ops on the GPU (both of its paths: all pairs for N <= 32,
  :171-188, source-chunked for N > 32, :150-170), with a HipFallbackWarning.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from hclsm_amd.kernels._common import require_gpu, warn_fallback
from hclsm_amd.kernels.relation_graph import GnnWeights, fused_supported, relation_graph_forward


class RelationGraph(nn.Module):
    def __init__(self, config) -> None:
        super().__init__()
        self.d_slot = config.d_slot
        self.d_edge = config.d_edge
        self.n_rounds = config.gnn_rounds
        self.n_max_slots = config.n_max_slots
        d, e = config.d_slot, config.d_edge
        self.pair_norm = nn.LayerNorm(d * 4)
        self.edge_mlp = nn.Sequential(nn.Linear(d * 4, e * 2), nn.ReLU(), nn.Linear(e * 2, e), nn.ReLU())
        self.edge_weight = nn.Linear(e, 1)
        self.msg_mlp = nn.Sequential(nn.Linear(e, d), nn.ReLU())
        self.update_mlp = nn.Sequential(nn.Linear(d * 2, d), nn.ReLU(), nn.Linear(d, d))
        self.causal_mlp = nn.Sequential(nn.Linear(e, e // 2), nn.ReLU(), nn.Linear(e // 2, 1))

    # ---- differentiable path (torch ops)
    def _edges(self, a, b):
        """Edge features and weights of the pairs (i in a's rows, j in b's rows)."""
        B, Ni, D = a.shape
        Nj = b.shape[1]
        ni = a[:, :, None, :].expand(B, Ni, Nj, D)
        nj = b[:, None, :, :].expand(B, Ni, Nj, D)
        pf = self.pair_norm(torch.cat([ni, nj, ni - nj, ni * nj], dim=-1))
        e = self.edge_mlp(pf)
        return e, torch.sigmoid(self.edge_weight(e).squeeze(-1))

    def _torch_forward(self, nodes, alive_mask):
        B, N, D = nodes.shape
        pair_mask = (alive_mask[:, :, None] * alive_mask[:, None, :] if alive_mask is not None
                     else torch.ones(B, N, N, device=nodes.device))
        if N > 32:   # source chunks of 16, as the reference (:97-126)
            for _ in range(self.n_rounds):
                agg = torch.zeros_like(nodes)
                for j0 in range(0, N, 16):
                    e, w = self._edges(nodes, nodes[:, j0:j0 + 16])
                    w = w * pair_mask[:, :, j0:j0 + 16]
                    agg = agg + (self.msg_mlp(e) * w.unsqueeze(-1)).sum(dim=2)
                nodes = nodes + self.update_mlp(torch.cat([nodes, agg], dim=-1))
            parts = []
            for j0 in range(0, N, 16):
                e, _ = self._edges(nodes, nodes[:, j0:j0 + 16])
                parts.append(torch.sigmoid(self.causal_mlp(e).squeeze(-1)))
            causal = torch.cat(parts, dim=2) * pair_mask
        else:
            e, w = self._edges(nodes, nodes)
            w = w * pair_mask
            for _ in range(self.n_rounds):
                agg = (self.msg_mlp(e) * w.unsqueeze(-1)).sum(dim=2)
                nodes = nodes + self.update_mlp(torch.cat([nodes, agg], dim=-1))
                if self.n_rounds > 1:
                    e, w = self._edges(nodes, nodes)
                    w = w * pair_mask
            causal = torch.sigmoid(self.causal_mlp(e).squeeze(-1)) * pair_mask
        if alive_mask is not None:
            nodes = nodes * alive_mask.unsqueeze(-1)
        return nodes, causal

    def _needs_grad(self, nodes) -> bool:
        if not torch.is_grad_enabled():
            return False
        return nodes.requires_grad or any(p.requires_grad for p in self.parameters())

    def forward(self, nodes: torch.Tensor, alive_mask: torch.Tensor | None = None):
        """nodes (B, N, d_slot), alive_mask (B, N) -> (updated nodes (B, N, d_slot), causal edges (B, N, N))."""
        require_gpu("RelationGraph", nodes, alive_mask)
        dtype = torch.bfloat16 if (torch.is_autocast_enabled("cuda") and
                                   torch.get_autocast_dtype("cuda") == torch.bfloat16) else torch.float32
        if self._needs_grad(nodes):
            warn_fallback("RelationGraph", "autograd (the fused edge and node kernels have no backward)")
            return self._torch_forward(nodes, alive_mask)
        if not fused_supported(nodes.shape[1], self.d_slot, self.d_edge, dtype):
            warn_fallback("RelationGraph", f"shape outside the fused kernels (N={nodes.shape[1]}, d_slot={self.d_slot}, "
                                           f"d_edge={self.d_edge}, {dtype})")
            return self._torch_forward(nodes, alive_mask)
        W = GnnWeights.from_module(self, dtype)
        out, causal = relation_graph_forward(nodes, alive_mask, W, self.n_rounds, chunked=nodes.shape[1] > 32)
        return out.to(nodes.dtype), causal
