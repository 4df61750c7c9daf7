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


@pytest.mark.parametrize("N,T,Dn", [(3, 37, 384), (2, 70, 300), (4, 64, 35), (1, 8, 128), (2, 5, 64)])
@pytest.mark.parametrize("mode", ["raw", "model", "block"])
def test_checkpointing_pair_matches_plain_pair(N, T, Dn, mode):
    """bf16, d_state 16: the forward that leaves the checkpoints (hclsm_ssm_scan_fwd_ckpt / the block form) gives
    the plain forward's output bit for bit, and the backward that starts from those checkpoints
    (hclsm_ssm_scan_bwd_ckpt) gives the plain backward's gradients: fp32 ones within 1e-5, bf16 ones within a
    bf16 rounding (the checkpointed states differ from the recomputed ones by fp32 rounding), both against the
    oracle at the bf16 bar.  T not a multiple of 8 leaves a partial last checkpoint interval; odd d_inner takes the
    one-channel-per-lane kernel."""
    from hclsm_amd import _lib
    from hclsm_amd.kernels.ssm_scan_bwd import scan_backward
    from hclsm_amd.kernels.ssm_scan_kernel import _block_forward, _scan_forward
    x, dt, A_log, B, C, D, gy = _inputs(N, T, Dn, 16, seed=N * 7 + T + Dn, dtype=torch.bfloat16,
                                        kind="config" if mode == "raw" else "ref")
    x, dt, A_log, B, C, D, gy = (t.cuda() for t in (x, dt, A_log, B, C, D, gy))
    if mode == "block":
        gate = torch.randn(N, T, Dn, generator=torch.Generator().manual_seed(T)).to(torch.bfloat16).cuda()
        dt_in = (dt.float() - 1.0).to(torch.bfloat16)       # softplus input
        y0, pre0, ws0 = _block_forward(x, dt_in, A_log, B, C, gate, True)
        y1, pre1, ws1 = _block_forward(x, dt_in, A_log, B, C, gate, True, for_grad=True)
        assert ws0 is None and ws1 is not None
        assert torch.equal(y0, y1) and torch.equal(pre0, pre1)
        args, code, Dk = (x, dt_in, A_log, B, C, None, gy), _lib.SCAN_BLOCK, None
    else:
        code = _lib.SCAN_RAW if mode == "raw" else _lib.SCAN_MODEL
        y0, _, ws0 = _scan_forward(x, dt, A_log, B, C, D, code, False)
        y1, _, ws1 = _scan_forward(x, dt, A_log, B, C, D, code, False, for_grad=True)
        assert ws0 is None and ws1 is not None
        assert torch.equal(y0, y1)
        args, Dk = (x, dt, A_log, B, C, D, gy), D
    plain = scan_backward(*args, code)
    ck = scan_backward(*args, code, ws=ws1)
    for name in plain:
        a, b = _np(ck[name]), _np(plain[name])
        tol = 1e-5 if name in ("A_log", "D") else 1e-2
        err = normwise_rel_err(a, b)
        assert err <= tol, f"{mode} {name}: checkpointed vs plain {err:.3e}"
    if mode != "block":
        ref = ssm_scan_bwd_ref(*(_np(t) for t in (x, dt, A_log, B, C)), _np(gy), D=_np(Dk), clamp_mode=mode)
        for name in ck:
            err = normwise_rel_err(_np(ck[name]), ref[name])
            assert err <= 2e-2, f"{mode} {name}: {err:.3e}"


def test_checkpointing_autograd_takes_the_pair_and_repeats():
    """The autograd path of a bf16, d_state 16 scan keeps the backward workspace from the forward, and a second
    backward through the same graph (retain_graph) gives the same gradients (the checkpoints are not consumed)."""
    from hclsm_amd.kernels.ssm_scan_kernel import fused_ssm_scan_hip
    x, dt, A_log, B, C, D, gy = _inputs(4, 24, 256, 16, seed=77, dtype=torch.bfloat16)
    leaves = [t.cuda().requires_grad_() for t in (x, dt, A_log, B, C, D)]
    y = fused_ssm_scan_hip(*leaves[:5], D=leaves[5], clamp_mode="raw")
    assert y.grad_fn is not None and getattr(y.grad_fn, "ws", None) is not None
    y.backward(gy.cuda(), retain_graph=True)
    first = [leaf.grad.clone() for leaf in leaves]
    for leaf in leaves:
        leaf.grad = None
    y.backward(gy.cuda())
    for a, leaf in zip(first, leaves):
        assert torch.equal(a, leaf.grad)
