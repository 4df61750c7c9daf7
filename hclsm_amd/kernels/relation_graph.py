"""Relation graph (GNN over object slots) in one C call (``hclsm_relation_graph_forward``).

Counterpart of ``RelationGraph.forward`` (hclsm/objects/relation_graph.py:68-193) for frames of N slots:
the pair tensor (frames, N, N, 4D) is never materialised; the pair LayerNorm is folded into the first
edge layer (per-node projections plus one contraction of length D per pair), and the edge MLP, edge
weight, messages and causal head run per pair tile in one kernel.  Inference only.
"""

from __future__ import annotations

import ctypes

import torch

from hclsm_amd import _lib
from hclsm_amd.kernels._common import require_gpu
from hclsm_amd.kernels.slot_iteration import _workspace

# parameter order of the C entry = the module's state-dict order (relation_graph.py:30-66)
GNN_PARAM_ORDER = ("pair_norm.weight", "pair_norm.bias", "edge_mlp.0.weight", "edge_mlp.0.bias",
                   "edge_mlp.2.weight", "edge_mlp.2.bias", "edge_weight.weight", "edge_weight.bias",
                   "msg_mlp.0.weight", "msg_mlp.0.bias", "update_mlp.0.weight", "update_mlp.0.bias",
                   "update_mlp.2.weight", "update_mlp.2.bias", "causal_mlp.0.weight", "causal_mlp.0.bias",
                   "causal_mlp.2.weight", "causal_mlp.2.bias")
_MATRICES = {"edge_mlp.0.weight", "edge_mlp.2.weight", "msg_mlp.0.weight", "update_mlp.0.weight",
             "update_mlp.2.weight", "causal_mlp.0.weight"}


class GnnWeights:
    """Device copies of a RelationGraph's parameters in GNN_PARAM_ORDER: matrices in the compute dtype,
    the rest fp32 (edge_weight.weight and causal_mlp.2.weight as vectors)."""

    def __init__(self, tensors: list, dtype: torch.dtype, d_slot: int, d_edge: int, eps: float) -> None:
        self.tensors = tensors
        self.ptrs = (ctypes.c_void_p * len(tensors))(*[t.data_ptr() for t in tensors])
        self.dtype, self.d_slot, self.d_edge, self.eps = dtype, d_slot, d_edge, eps

    @classmethod
    def from_dict(cls, w: dict, dtype: torch.dtype, eps: float = 1e-5, device="cuda") -> "GnnWeights":
        t = []
        for name in GNN_PARAM_ORDER:
            v = torch.as_tensor(w[name]).detach()
            v = v.to(device=device, dtype=dtype if name in _MATRICES else torch.float32)
            t.append(v.reshape(-1).contiguous() if name not in _MATRICES else v.contiguous())
        d_edge = t[4].shape[0]
        return cls(t, dtype, t[2].shape[1] // 4, d_edge, eps)

    @classmethod
    def from_module(cls, m, dtype: torch.dtype) -> "GnnWeights":
        key = (dtype,) + tuple((p.data_ptr(), p._version) for p in m.parameters())
        hit = getattr(m, "_hclsm_gnn_weights", None)
        if hit is not None and hit[0] == key:
            return hit[1]
        W = cls.from_dict(dict(m.named_parameters()), dtype, m.pair_norm.eps, m.pair_norm.weight.device)
        m._hclsm_gnn_weights = (key, W)
        return W


def fused_supported(N: int, d_slot: int, d_edge: int, dtype: torch.dtype) -> bool:
    """Whether hclsm_relation_graph_forward takes this shape (D, E multiples of 32, E <= 192, N <= 128, or
    64 with fp32 operands, within the kernel's LDS budget)."""
    return int(_lib.lib().hclsm_relation_graph_workspace(1, N, d_slot, d_edge, _lib.dtype_code(dtype))) >= 0


def relation_graph_forward(nodes: torch.Tensor, alive: torch.Tensor | None, W: GnnWeights, n_rounds: int,
                           chunked: bool | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """nodes (F, N, d_slot), alive (F, N) or None -> (nodes' (F, N, d_slot) fp32, causal (F, N, N) fp32).
    ``chunked`` selects the reference's path semantics (default: N > 32, relation_graph.py:149); they
    differ only for one round (where the causal edges come from)."""
    require_gpu("relation_graph_forward", nodes, alive)
    F, N, D = nodes.shape
    if D != W.d_slot:
        raise ValueError(f"nodes have d_slot {D}, the weights {W.d_slot}")
    if chunked is None:
        chunked = N > 32
    x = nodes.detach().to(torch.float32).contiguous()
    al = None if alive is None else alive.detach().to(torch.float32).contiguous()
    out = torch.empty_like(x)
    causal = torch.empty((F, N, N), dtype=torch.float32, device=x.device)
    L = _lib.lib()
    code = _lib.dtype_code(W.dtype)
    wsb = L.hclsm_relation_graph_workspace(F, N, D, W.d_edge, code)
    _lib.check(wsb if wsb < 0 else 0, "hclsm_relation_graph_workspace")
    ws = _workspace(int(wsb), x.device)
    rc = L.hclsm_relation_graph_forward(_lib.ptr(x), _lib.ptr(al), _lib.ptr(out), _lib.ptr(causal), F, N, D, W.d_edge,
                                        int(n_rounds), int(bool(chunked)), W.ptrs, float(W.eps), code, _lib.ptr(ws),
                                        ws.numel(), _lib.stream_of(x))
    _lib.check(rc, "hclsm_relation_graph_forward")
    return out, causal
