"""GPU parity of hclsm_amd.kernels.gnn_message_pass (hclsm_gnn_message_pass) against
oracle/objects.py::gnn_message_pass_ref, and the reference's own assertions (tests/test_kernels.py:239-300)
on the HIP path.

Tolerances (normwise relative): fp32 1e-5 (nodes and edge features); bf16 operands under autocast 2e-2
(oracle fed the bf16-rounded weights).  Shapes: the reference test's D=32, d_edge=16 (fp32 generic kernel),
the tiny and small presets' (64, 32) / (192, 96) (the weight-resident kernel with bf16 operands), the base
preset's (256, 128) with 64 slots (the chunk-streamed kernel), ragged slot counts and dead slots."""

from __future__ import annotations

import warnings

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import objects as ob
from oracle.ssm_scan import normwise_rel_err

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().double().cpu().numpy()


def _modules(D, E, seed, dtype=torch.float32):
    torch.manual_seed(seed)
    edge_mlp = nn.Sequential(nn.Linear(D * 4, E * 2), nn.ReLU(), nn.Linear(E * 2, E), nn.ReLU())
    edge_weight_linear = nn.Linear(E, 1)
    msg_mlp = nn.Sequential(nn.Linear(E, D), nn.ReLU())
    update_mlp = nn.Sequential(nn.Linear(D * 2, D), nn.ReLU(), nn.Linear(D, D))
    mods = [m.cuda() for m in (edge_mlp, edge_weight_linear, msg_mlp, update_mlp)]
    if dtype != torch.float32:   # weights exactly representable in the operand dtype
        with torch.no_grad():
            for m in mods:
                for p in m.parameters():
                    p.copy_(p.to(dtype).float())
    return mods


def _params(mods):
    em, ew, mm, um = mods
    p = {}
    for name, lin in (("edge_mlp.0", em[0]), ("edge_mlp.2", em[2]), ("edge_weight", ew), ("msg_mlp.0", mm[0]),
                      ("update_mlp.0", um[0]), ("update_mlp.2", um[2])):
        p[name + ".weight"] = _np(lin.weight)
        p[name + ".bias"] = _np(lin.bias)
    return p


def _inputs(B, N, D, seed, dead=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, N, D, generator=g)
    alive = (torch.rand(B, N, generator=g) > 0.25).float() if dead else torch.ones(B, N)
    return x.cuda(), alive.cuda()


CASES = [  # B, N, D, E, rounds
    (2, 16, 32, 16, 1),      # the reference test's modules (tests/test_kernels.py:243-251)
    (3, 8, 32, 16, 2),
    (4, 21, 64, 32, 1),      # ragged N
    (2, 32, 192, 96, 2),     # small preset shape
    (2, 48, 128, 64, 1),
]


@pytest.mark.parametrize("B,N,D,E,rounds", CASES)
def test_fp32_matches_oracle_all_forms(B, N, D, E, rounds):
    from hclsm_amd.kernels import (chunked_gnn_message_pass, gnn_message_pass_fn, naive_gnn_message_pass,
                                   optimized_gnn_message_pass)
    mods = _modules(D, E, B + N)
    x, alive = _inputs(B, N, D, seed=N + D)
    p = _params(mods)
    with torch.no_grad(), warnings.catch_warnings():
        warnings.simplefilter("error")          # the HIP path must run: no fallback warning
        for fn in (naive_gnn_message_pass, optimized_gnn_message_pass):
            out, e = fn(x, alive, *mods, n_rounds=rounds)
            ref, re = ob.gnn_message_pass_ref(_np(x), _np(alive), p, rounds)
            assert out.shape == (B, N, D) and e.shape == (B, N, N, E)
            assert normwise_rel_err(_np(out), ref) <= 1e-5
            assert normwise_rel_err(_np(e), re) <= 1e-5
        out, e = chunked_gnn_message_pass(x, alive, *mods, n_rounds=rounds, chunk_size=5)
        ref, re = ob.gnn_message_pass_ref(_np(x), _np(alive), p, rounds, chunk_size=5)
        assert e.shape == re.shape
        assert normwise_rel_err(_np(out), ref) <= 1e-5
        assert normwise_rel_err(_np(e), re) <= 1e-5
        out, e = gnn_message_pass_fn(x, None, *mods, n_rounds=rounds)   # auto: chunked (16) for N > 32
        ref, re = ob.gnn_message_pass_ref(_np(x), None, p, rounds, chunk_size=16 if N > 32 else None)
        assert normwise_rel_err(_np(out), ref) <= 1e-5
        assert normwise_rel_err(_np(e), re) <= 1e-5


@pytest.mark.parametrize("B,N,D,E,rounds", [(3, 16, 64, 32, 1), (2, 32, 192, 96, 2), (1, 64, 256, 128, 2),
                                            (2, 40, 96, 64, 1)])
def test_bf16_autocast_matches_oracle(B, N, D, E, rounds):
    """bf16 operands: the weight-resident kernel at (64, 32) / (192, 96), the chunk-streamed kernel at
    (256, 128), the generic kernel elsewhere."""
    from hclsm_amd.kernels import naive_gnn_message_pass
    mods = _modules(D, E, 3 * N + D, torch.bfloat16)
    x, alive = _inputs(B, N, D, seed=D + 1)
    p = _params(mods)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16), warnings.catch_warnings():
        warnings.simplefilter("error")
        out, e = naive_gnn_message_pass(x, alive, *mods, n_rounds=rounds)
    assert out.dtype == torch.float32 and e.dtype == torch.bfloat16
    ref, re = ob.gnn_message_pass_ref(_np(x), _np(alive), p, rounds)
    assert normwise_rel_err(_np(out), ref) <= 2e-2
    assert normwise_rel_err(_np(e), re) <= 2e-2


def test_reference_assertions_on_the_hip_path():
    """tests/test_kernels.py:253-300 with the tensors on the GPU."""
    from hclsm_amd.kernels import (chunked_gnn_message_pass, gnn_message_pass_fn, naive_gnn_message_pass,
                                   optimized_gnn_message_pass)
    mods = _modules(32, 16, 0)
    torch.manual_seed(1)
    with torch.no_grad():
        B, N, D = 2, 16, 32
        out, ef = naive_gnn_message_pass(torch.randn(B, N, D, device="cuda"), torch.ones(B, N, device="cuda"), *mods)
        assert out.shape == (B, N, D) and ef is not None
        alive = torch.ones(B, N, device="cuda")
        alive[:, -4:] = 0
        out, _ = naive_gnn_message_pass(torch.randn(B, N, D, device="cuda"), alive, *mods)
        assert torch.allclose(out[:, -4:], torch.zeros(B, 4, D, device="cuda"), atol=1e-6)
        B, N = 2, 8
        nodes, alive = torch.randn(B, N, D, device="cuda"), torch.ones(B, N, device="cuda")
        a, _ = naive_gnn_message_pass(nodes, alive, *mods, n_rounds=1)
        b, _ = optimized_gnn_message_pass(nodes, alive, *mods, n_rounds=1)
        c, _ = chunked_gnn_message_pass(nodes, alive, *mods, n_rounds=1, chunk_size=4)
        assert torch.allclose(a, b, atol=1e-5) and torch.allclose(a, c, atol=1e-4)
        out, _ = gnn_message_pass_fn(nodes, alive, *mods)
        assert out.shape == (B, N, D)
        out, _ = naive_gnn_message_pass(nodes, None, *mods)
        assert out.shape == (B, N, D)
        out, e = naive_gnn_message_pass(nodes, alive, *mods, n_rounds=0)
        assert e is None and torch.equal(out, nodes)


def test_fallbacks_warn_and_match():
    """Autograd and a module structure the kernel does not take run torch ops, with a HipFallbackWarning; the
    values equal the fused kernel's (fp32) and the gradients reach the nodes and the weights."""
    from hclsm_amd.kernels import HipFallbackWarning, _common, naive_gnn_message_pass
    _common._WARNED.clear()          # each reason warns once per process
    mods = _modules(32, 16, 5)
    x, alive = _inputs(2, 12, 32, seed=9)
    with torch.no_grad():
        ref, ref_e = naive_gnn_message_pass(x, alive, *mods, n_rounds=2)
    xg = x.clone().requires_grad_()
    with pytest.warns(HipFallbackWarning, match="autograd"):
        out, e = naive_gnn_message_pass(xg, alive, *mods, n_rounds=2)
    assert normwise_rel_err(_np(out), _np(ref)) <= 1e-5 and normwise_rel_err(_np(e), _np(ref_e)) <= 1e-5
    out.sum().backward()
    assert torch.isfinite(xg.grad).all() and mods[0][0].weight.grad is not None
    gelu = [nn.Sequential(nn.Linear(128, 32), nn.GELU(), nn.Linear(32, 16), nn.ReLU()).cuda()] + mods[1:]
    with torch.no_grad(), pytest.warns(HipFallbackWarning, match="edge_mlp"):
        out, _ = naive_gnn_message_pass(x, alive, *gelu)
    assert out.shape == x.shape
