"""GPU parity of the HIP reverse scan against the finite-difference-pinned oracle
(oracle.ssm_scan.ssm_scan_bwd_ref).  Tolerances normwise: fp32 1e-5 (A_log, D: 2e-5, sums over
every sequence and step); bf16 2e-2."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.ssm_scan import normwise_rel_err, ssm_scan_bwd_ref

pytestmark = pytest.mark.gpu


def _inputs(N, T, Dn, S, seed, dtype=torch.float32, kind="config"):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, T, Dn, generator=g)
    if kind == "config":
        dt = torch.nn.functional.softplus(-2 + 0.5 * torch.randn(N, T, Dn, generator=g))
        A_log = torch.rand(Dn, S, generator=g) * math.log(16)
    else:   # tests/test_kernels.py:120-128 distribution: exercises the model-mode clamps
        dt = torch.rand(N, T, Dn, generator=g) + 0.01
        A_log = torch.randn(Dn, S, generator=g)
    B = torch.randn(N, T, S, generator=g) / math.sqrt(S)
    C = torch.randn(N, T, S, generator=g) / math.sqrt(S)
    D = torch.randn(Dn, generator=g)
    gy = torch.randn(N, T, Dn, generator=g)
    return [t.to(dtype) for t in (x, dt)] + [A_log] + [t.to(dtype) for t in (B, C)] + [D, gy.to(dtype)]


def _np(t):
    return t.detach().double().cpu().numpy()


@pytest.mark.parametrize("N,T,Dn,S", [(2, 16, 32, 8), (1, 8, 64, 16), (4, 32, 16, 4), (3, 37, 384, 16),
                                      (2, 19, 70, 5), (1, 12, 40, 32), (1, 9, 24, 64), (2, 70, 300, 16),
                                      (2, 11, 40, 96), (1, 70, 24, 128)])   # up to the large preset's d_state
@pytest.mark.parametrize("mode", ["raw", "model"])
def test_backward_fp32(N, T, Dn, S, mode):
    from hclsm_amd.kernels.ssm_scan_kernel import fused_ssm_scan_hip
    x, dt, A_log, B, C, D, gy = _inputs(N, T, Dn, S, seed=N * 100 + T + S, kind="config" if mode == "raw" else "ref")
    leaves = [t.cuda().requires_grad_() for t in (x, dt, A_log, B, C, D)]
    y = fused_ssm_scan_hip(*leaves[:5], D=leaves[5], clamp_mode=mode)
    y.backward(gy.cuda())
    ref = ssm_scan_bwd_ref(*(_np(t) for t in (x, dt, A_log, B, C)), _np(gy), D=_np(D), clamp_mode=mode)
    for name, leaf in zip(("x", "dt", "A_log", "B", "C", "D"), leaves):
        tol = 2e-5 if name in ("A_log", "D") else 1e-5
        err = normwise_rel_err(_np(leaf.grad), ref[name])
        assert err <= tol, f"{name} ({mode}): {err:.3e}"


def test_backward_bf16_config1_subset():
    from hclsm_amd.kernels.ssm_scan_kernel import fused_ssm_scan_hip
    x, dt, A_log, B, C, D, gy = _inputs(64, 64, 384, 16, seed=5, dtype=torch.bfloat16)
    leaves = [t.cuda().requires_grad_() for t in (x, dt, A_log, B, C, D)]
    y = fused_ssm_scan_hip(*leaves[:5], D=leaves[5], clamp_mode="raw")
    y.backward(gy.cuda())
    ref = ssm_scan_bwd_ref(*(_np(t) for t in (x, dt, A_log, B, C)), _np(gy), D=_np(D), clamp_mode="raw")
    for name, leaf in zip(("x", "dt", "A_log", "B", "C", "D"), leaves):
        err = normwise_rel_err(_np(leaf.grad), ref[name])
        assert err <= 2e-2, f"{name}: {err:.3e}"
        assert leaf.grad.dtype == leaf.dtype


def test_reference_sequential_backward_runs():
    """tests/test_kernels.py:147-159: backward through the sequential (model) scan on the HIP path."""
    from hclsm_amd.kernels import sequential_ssm_scan
    x = torch.randn(2, 8, 16, device="cuda", requires_grad=True)
    dt = torch.rand(2, 8, 16, device="cuda").abs() + 0.01
    A_log = torch.randn(16, 4, device="cuda", requires_grad=True)
    Bp = torch.randn(2, 8, 4, device="cuda")
    C = torch.randn(2, 8, 4, device="cuda")
    y = sequential_ssm_scan(x, dt, A_log, Bp, C)
    y.sum().backward()
    assert x.grad is not None and A_log.grad is not None
    assert torch.isfinite(x.grad).all() and torch.isfinite(A_log.grad).all()
