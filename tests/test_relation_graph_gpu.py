"""GPU parity of the relation graph (hclsm_relation_graph_forward and the RelationGraph module) against
oracle/objects.py::relation_graph_ref: fp32 normwise 1e-5 (nodes and causal edges), bf16 operands 2e-2;
both path semantics, ragged slot counts (padding to 16), dead slots, 1-3 rounds; the module's
differentiable torch path against the same oracle and its gradients against float64 autograd."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import objects as ob
from oracle.ssm_scan import normwise_rel_err

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().double().cpu().numpy()


def _module(D, E, rounds, N, seed):
    from hclsm_amd.objects import RelationGraph
    torch.manual_seed(seed)
    m = RelationGraph(SimpleNamespace(d_slot=D, d_edge=E, gnn_rounds=rounds, n_max_slots=N)).cuda()
    with torch.no_grad():   # non-trivial LayerNorm affine
        m.pair_norm.weight.add_(0.2 * torch.randn_like(m.pair_norm.weight))
        m.pair_norm.bias.add_(0.1 * torch.randn_like(m.pair_norm.bias))
    return m


def _inputs(F, N, D, seed, dead=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(F, N, D, generator=g)
    alive = (torch.rand(F, N, generator=g) > 0.25).float() if dead else torch.ones(F, N)
    return x.cuda(), alive.cuda()


CASES = [  # F, N, D, E, rounds, chunked
    (6, 16, 128, 64, 1, False),     # tiny preset (config.py:199-203)
    (4, 32, 192, 96, 2, False),     # small preset
    (3, 24, 64, 32, 1, True),       # ragged N, chunked semantics with one round
    (2, 48, 128, 64, 3, True),      # N > 32: the reference's chunked path
    (2, 64, 96, 64, 2, True),
]


@pytest.mark.parametrize("F,N,D,E,rounds,chunked", CASES)
def test_relation_graph_fp32_matches_oracle(F, N, D, E, rounds, chunked):
    from hclsm_amd.kernels.relation_graph import GnnWeights, relation_graph_forward
    m = _module(D, E, rounds, N, F + N)
    x, alive = _inputs(F, N, D, seed=N + D)
    W = GnnWeights.from_module(m, torch.float32)
    out, causal = relation_graph_forward(x, alive, W, rounds, chunked=chunked)
    p = {k: _np(v) for k, v in m.state_dict().items()}
    ref, rc = ob.relation_graph_ref(_np(x), _np(alive), p, rounds, chunked=chunked)
    assert normwise_rel_err(_np(out), ref) <= 1e-5
    assert normwise_rel_err(_np(causal), rc) <= 1e-5


@pytest.mark.parametrize("F,N,D,E,rounds,chunked", CASES + [(1, 128, 384, 192, 3, True), (2, 40, 192, 96, 1, False),
                                                     (2, 64, 256, 128, 2, True)])
def test_relation_graph_bf16_matches_oracle(F, N, D, E, rounds, chunked):
    from hclsm_amd.kernels.relation_graph import GnnWeights, relation_graph_forward
    m = _module(D, E, rounds, N, F + N + 1)
    x, alive = _inputs(F, N, D, seed=N + D + 1)
    W = GnnWeights.from_module(m, torch.bfloat16)
    out, causal = relation_graph_forward(x, alive, W, rounds, chunked=chunked)
    p = {k: _np(v) for k, v in m.state_dict().items()}
    ref, rc = ob.relation_graph_ref(_np(x), _np(alive), p, rounds, chunked=chunked)
    assert normwise_rel_err(_np(out), ref) <= 2e-2
    assert normwise_rel_err(_np(causal), rc) <= 2e-2


def test_module_paths_and_gradients():
    """The module: C path under no_grad, torch path with autograd, both against the oracle; gradients of the
    torch path against float64 autograd of the same module on the CPU."""
    m = _module(64, 32, 2, 16, 9)
    x, alive = _inputs(3, 16, 64, seed=10)
    p = {k: _np(v) for k, v in m.state_dict().items()}
    ref, rc = ob.relation_graph_ref(_np(x), _np(alive), p, 2)
    with torch.no_grad():
        o1, c1 = m(x, alive)
    xa = x.clone().requires_grad_()
    o2, c2 = m(xa, alive)
    for o, c in ((o1, c1), (o2, c2)):
        assert normwise_rel_err(_np(o), ref) <= 1e-5 and normwise_rel_err(_np(c), rc) <= 1e-5
    w = torch.randn_like(o2)
    ((o2 * w).sum() + c2.sum()).backward()
    m64 = _module(64, 32, 2, 16, 9).cpu().double()
    m64.load_state_dict({k: v.double().cpu() for k, v in m.state_dict().items()})
    xb = x.double().cpu().requires_grad_()
    ob_, cb_ = m64._torch_forward(xb, alive.double().cpu())
    ((ob_ * w.double().cpu()).sum() + cb_.sum()).backward()
    assert normwise_rel_err(_np(xa.grad), xb.grad.numpy()) <= 1e-5


def test_fused_shape_limits():
    from hclsm_amd.kernels.relation_graph import fused_supported
    assert fused_supported(128, 384, 192, torch.bfloat16)        # large preset (config.py:270): 32-column chunks
    assert not fused_supported(128, 384, 192, torch.float32)     # fp32 tiles hold 64 pairs
    assert not fused_supported(32, 200, 96, torch.bfloat16)      # D not a multiple of 32


@pytest.mark.parametrize("F,N,D,E,rounds,chunked", [CASES[0], CASES[1], (2, 64, 256, 128, 2, True), CASES[4]])
def test_relation_graph_fp16_matches_oracle(F, N, D, E, rounds, chunked):
    """fp16 operands through the same kernels (resident, streamed and chunked variants)."""
    from hclsm_amd.kernels.relation_graph import GnnWeights, relation_graph_forward
    m = _module(D, E, rounds, N, F + N + 2)
    x, alive = _inputs(F, N, D, seed=N + D + 2)
    W = GnnWeights.from_module(m, torch.float16)
    out, causal = relation_graph_forward(x, alive, W, rounds, chunked=chunked)
    p = {k: _np(v) for k, v in m.state_dict().items()}
    ref, rc = ob.relation_graph_ref(_np(x), _np(alive), p, rounds, chunked=chunked)
    assert normwise_rel_err(_np(out), ref) <= 1e-2
    assert normwise_rel_err(_np(causal), rc) <= 1e-2
