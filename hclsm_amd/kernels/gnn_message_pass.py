"""GNN message passing on MI355X -- drop-in for ``hclsm/kernels/gnn_message_pass.py``.

Reference names kept (same positional signatures, defaults and return structures):

    naive_gnn_message_pass(nodes, alive_mask, edge_mlp, edge_weight_linear, msg_mlp, update_mlp, n_rounds=1)
                                                                                            (:38-100)
    optimized_gnn_message_pass(... same ...)                                                (:107-161)
    chunked_gnn_message_pass(... , n_rounds=1, chunk_size=16)                               (:168-243)
    gnn_message_pass_fn(... , n_rounds=1, backend="auto", chunk_size=16)                    (:250-282)

Each returns (updated nodes (B, N, D), edge features): the last round's (B, N, N, d_edge) for the naive and
optimized forms, the last target chunk's (B, N, C, d_edge) for the chunked form (:225-227), None when
n_rounds == 0.  "auto" takes the chunked form for N > 32 (:274-279), as the reference does.

Per round: e_ij = edge_mlp([n_i; n_j; n_i - n_j; n_i * n_j]), w_ij = sigmoid(edge_weight_linear(e_ij)) *
alive_i * alive_j, agg_i = sum_j msg_mlp(e_ij) w_ij, n_i += update_mlp([n_i; agg_i]); then n * alive.

The modules are the caller's.  With the structure of the reference's tests and benchmark
(tests/test_kernels.py:242-251, scripts/benchmark_kernels.py:179-187) -- edge_mlp = Sequential(Linear(4D, 2E),
ReLU, Linear(2E, E), ReLU), edge_weight_linear = Linear(E, 1), msg_mlp = Sequential(Linear(E, D), ReLU),
update_mlp = Sequential(Linear(2D, D), ReLU, Linear(D, D)) -- and without autograd the call is one
``hclsm_gnn_message_pass`` (the pair tensor is never formed: the first edge layer is split into per-node
projections plus one contraction of length D per pair; edges, weights and messages run per pair tile on MFMA),
in fp32, or with bf16 operands under a bf16 autocast.  Any other structure or shape, and autograd, run the
reference's math as torch ops on the GPU and say so with a ``HipFallbackWarning``.
"""

from __future__ import annotations

import ctypes

import torch
import torch.nn as nn

from hclsm_amd import _lib
from hclsm_amd.kernels._common import require_gpu, warn_fallback
from hclsm_amd.kernels.slot_iteration import _workspace


# ---------------------------------------------------------------------------
# the reference's math in torch ops (autograd, and structures the kernel does not take)
# ---------------------------------------------------------------------------

def _pair_features(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    B, Ni, D = a.shape
    Nj = b.shape[1]
    ni = a[:, :, None, :].expand(B, Ni, Nj, D)
    nj = b[:, None, :, :].expand(B, Ni, Nj, D)
    return torch.cat([ni, nj, ni - nj, ni * nj], dim=-1)


def _torch_message_pass(nodes, alive_mask, edge_mlp, edge_weight_linear, msg_mlp, update_mlp, n_rounds,
                        chunk_size=None):
    B, N, D = nodes.shape
    pair_mask = alive_mask[:, :, None] * alive_mask[:, None, :] if alive_mask is not None else None
    edge_feat = None
    for _ in range(n_rounds):
        starts = [0] if chunk_size is None else list(range(0, N, chunk_size))
        agg = torch.zeros_like(nodes) if chunk_size is not None else None
        for j0 in starts:
            j1 = N if chunk_size is None else min(j0 + chunk_size, N)
            e = edge_mlp(_pair_features(nodes, nodes[:, j0:j1]))
            w = torch.sigmoid(edge_weight_linear(e).squeeze(-1))
            if pair_mask is not None:
                w = w * pair_mask[:, :, j0:j1]
            part = (msg_mlp(e) * w.unsqueeze(-1)).sum(dim=2)
            agg = part if agg is None else agg + part
            edge_feat = e
        nodes = nodes + update_mlp(torch.cat([nodes, agg], dim=-1))
    if alive_mask is not None:
        nodes = nodes * alive_mask.unsqueeze(-1)
    return nodes, edge_feat


# ---------------------------------------------------------------------------
# the fused C path
# ---------------------------------------------------------------------------

def _is_linear(m, din, dout) -> bool:
    return isinstance(m, nn.Linear) and m.in_features == din and m.out_features == dout


def _structure(D, edge_mlp, edge_weight_linear, msg_mlp, update_mlp):
    """d_edge if the modules have the structure the kernel runs, else a reason string."""
    if not (isinstance(edge_mlp, nn.Sequential) and len(edge_mlp) == 4 and isinstance(edge_mlp[1], nn.ReLU)
            and isinstance(edge_mlp[3], nn.ReLU) and isinstance(edge_mlp[0], nn.Linear)):
        return "edge_mlp is not Sequential(Linear, ReLU, Linear, ReLU)"
    E2 = edge_mlp[0].out_features
    if E2 % 2 or not _is_linear(edge_mlp[0], 4 * D, E2) or not _is_linear(edge_mlp[2], E2, E2 // 2):
        return "edge_mlp is not Linear(4D, 2E), ReLU, Linear(2E, E), ReLU"
    E = E2 // 2
    if not _is_linear(edge_weight_linear, E, 1):
        return "edge_weight_linear is not Linear(d_edge, 1)"
    if not (isinstance(msg_mlp, nn.Sequential) and len(msg_mlp) == 2 and _is_linear(msg_mlp[0], E, D)
            and isinstance(msg_mlp[1], nn.ReLU)):
        return "msg_mlp is not Sequential(Linear(d_edge, D), ReLU)"
    if not (isinstance(update_mlp, nn.Sequential) and len(update_mlp) == 3 and _is_linear(update_mlp[0], 2 * D, D)
            and isinstance(update_mlp[1], nn.ReLU) and _is_linear(update_mlp[2], D, D)):
        return "update_mlp is not Sequential(Linear(2D, D), ReLU, Linear(D, D))"
    return E


_LINEARS = lambda em, ew, mm, um: (em[0], em[2], ew, mm[0], um[0], um[2])   # noqa: E731


class _MpWeights:
    """Device copies in the C entry's parameter order: matrices in the compute dtype, vectors fp32 (a missing
    bias as zeros)."""

    def __init__(self, linears, dtype, device):
        self.tensors = []
        for lin in linears:
            w = lin.weight.detach()
            w = w.reshape(-1) if lin.out_features == 1 else w
            self.tensors.append(w.to(device=device, dtype=torch.float32 if lin.out_features == 1 else dtype)
                                .contiguous())
            b = lin.bias.detach() if lin.bias is not None else torch.zeros(lin.out_features, device=device)
            self.tensors.append(b.to(device=device, dtype=torch.float32).contiguous())
        self.ptrs = (ctypes.c_void_p * len(self.tensors))(*[t.data_ptr() for t in self.tensors])


def _weights(linears, dtype, device) -> _MpWeights:
    holder = linears[0]
    key = (dtype, str(device)) + tuple((p.data_ptr(), p._version) for lin in linears for p in lin.parameters())
    hit = getattr(holder, "_hclsm_mp_weights", None)
    if hit is not None and hit[0] == key:
        return hit[1]
    W = _MpWeights(linears, dtype, device)
    holder._hclsm_mp_weights = (key, W)
    return W


def _compute_dtype():
    if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16:
        return torch.bfloat16
    return torch.float32


def _message_pass(nodes, alive_mask, edge_mlp, edge_weight_linear, msg_mlp, update_mlp, n_rounds, chunk_size,
                  name):
    require_gpu(name, nodes, alive_mask)
    if nodes.dim() != 3:
        raise ValueError(f"{name}: nodes must be (B, N, D), got {tuple(nodes.shape)}")
    B, N, D = nodes.shape
    if alive_mask is not None and tuple(alive_mask.shape) != (B, N):
        raise ValueError(f"{name}: alive_mask must be ({B}, {N}), got {tuple(alive_mask.shape)}")
    mods = (edge_mlp, edge_weight_linear, msg_mlp, update_mlp)
    grad = torch.is_grad_enabled() and (nodes.requires_grad or
                                        any(p.requires_grad for m in mods for p in m.parameters()))
    E = _structure(D, *mods)
    dtype = _compute_dtype()
    reason = None
    if grad:
        reason = "autograd (the fused kernel is forward-only)"
    elif isinstance(E, str):
        reason = E
    else:
        wsb = int(_lib.lib().hclsm_gnn_message_pass_workspace(B, N, D, E, _lib.dtype_code(dtype)))
        if wsb < 0:
            reason = f"shape N={N}, D={D}, d_edge={E} in {dtype} is outside the fused kernel ({_lib.strerror(wsb)})"
    if reason is not None:
        warn_fallback(name, reason)
        return _torch_message_pass(nodes, alive_mask, *mods, n_rounds, chunk_size)
    n_rounds = int(n_rounds)
    j0 = 0 if chunk_size is None else ((N - 1) // chunk_size) * chunk_size if N > 0 else 0
    enj = N - j0
    x = nodes.detach().to(torch.float32).contiguous()
    al = None if alive_mask is None else alive_mask.detach().to(torch.float32).contiguous()
    out = torch.empty_like(x)
    edges = torch.empty((B, N, enj, E), dtype=torch.float32, device=x.device) if n_rounds > 0 else None
    W = _weights(_LINEARS(*mods), dtype, x.device)
    ws = _workspace(wsb, x.device)
    rc = _lib.lib().hclsm_gnn_message_pass(_lib.ptr(x), _lib.ptr(al), _lib.ptr(out), _lib.ptr(edges), B, N, D, E,
                                           n_rounds, j0, enj, W.ptrs, _lib.dtype_code(dtype), _lib.ptr(ws), ws.numel(),
                                           _lib.stream_of(x))
    _lib.check(rc, "hclsm_gnn_message_pass")
    if edges is not None and dtype != torch.float32:
        edges = edges.to(dtype)   # the dtype autocast gives the reference's edge_mlp output
    return out.to(nodes.dtype), edges


def naive_gnn_message_pass(nodes: torch.Tensor, alive_mask: torch.Tensor | None, edge_mlp: nn.Module,
                           edge_weight_linear: nn.Module, msg_mlp: nn.Module, update_mlp: nn.Module,
                           n_rounds: int = 1) -> tuple[torch.Tensor, torch.Tensor | None]:
    """All pairs every round; returns (nodes (B, N, D), last round's edge features (B, N, N, d_edge))."""
    return _message_pass(nodes, alive_mask, edge_mlp, edge_weight_linear, msg_mlp, update_mlp, n_rounds, None,
                         "naive_gnn_message_pass")


def optimized_gnn_message_pass(nodes: torch.Tensor, alive_mask: torch.Tensor | None, edge_mlp: nn.Module,
                               edge_weight_linear: nn.Module, msg_mlp: nn.Module, update_mlp: nn.Module,
                               n_rounds: int = 1) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Same result as naive_gnn_message_pass (the reference's two forms differ only in how they build pairs)."""
    return _message_pass(nodes, alive_mask, edge_mlp, edge_weight_linear, msg_mlp, update_mlp, n_rounds, None,
                         "optimized_gnn_message_pass")


def chunked_gnn_message_pass(nodes: torch.Tensor, alive_mask: torch.Tensor | None, edge_mlp: nn.Module,
                             edge_weight_linear: nn.Module, msg_mlp: nn.Module, update_mlp: nn.Module,
                             n_rounds: int = 1, chunk_size: int = 16) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Same nodes; the edge features returned are those of the last chunk of chunk_size targets
    (B, N, C, d_edge), as the reference keeps them (:225-227)."""
    if int(chunk_size) < 1:
        raise ValueError(f"chunk_size must be >= 1, got {chunk_size}")
    return _message_pass(nodes, alive_mask, edge_mlp, edge_weight_linear, msg_mlp, update_mlp, n_rounds,
                         int(chunk_size), "chunked_gnn_message_pass")


def gnn_message_pass_fn(nodes: torch.Tensor, alive_mask: torch.Tensor | None, edge_mlp: nn.Module,
                        edge_weight_linear: nn.Module, msg_mlp: nn.Module, update_mlp: nn.Module,
                        n_rounds: int = 1, backend: str = "auto", chunk_size: int = 16):
    """Dispatch as the reference (:250-282): "naive", "chunked", else chunked for N > 32 and optimized otherwise."""
    args = (nodes, alive_mask, edge_mlp, edge_weight_linear, msg_mlp, update_mlp, n_rounds)
    if backend == "naive":
        return naive_gnn_message_pass(*args)
    if backend == "chunked" or nodes.shape[1] > 32:
        return chunked_gnn_message_pass(*args, chunk_size)
    return optimized_gnn_message_pass(*args)
