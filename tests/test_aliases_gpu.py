"""Every reference-named alias of the kernel API, called by its own name on the GPU, gives the result of the
canonical entry it stands for (the same kernel, so bitwise equal), and that result matches the oracle:
compiled_slot_attention and backend="compiled" (slot_attention_kernel.py:298-317, naive semantics),
fused_slot_attention_triton (:239-258, the +1e-8 denominator), fused_ssm_scan_triton (ssm_scan_kernel.py:379-387)
and parallel_ssm_scan_pytorch (:168-218, raw recurrence), sequential_ssm_scan (:42-86, clamped)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import slot_attention as sa
from oracle.ssm_scan import normwise_rel_err, ssm_scan_ref

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().double().cpu().numpy()


def test_slot_attention_aliases():
    from hclsm_amd.kernels import (compiled_slot_attention, fused_slot_attention_triton, naive_slot_attention,
                                   slot_attention_fn)
    g = torch.Generator().manual_seed(17)
    Q, K, V = (torch.randn(s, generator=g).cuda() for s in ((3, 16, 64), (3, 50, 64), (3, 50, 64)))
    naive = naive_slot_attention(Q, K, V)
    for got in (compiled_slot_attention(Q, K, V), slot_attention_fn(Q, K, V, backend="compiled"),
                slot_attention_fn(Q, K, V, backend="naive")):
        assert torch.equal(got[0], naive[0]) and torch.equal(got[1], naive[1])
    ref_o, ref_a = sa.slot_attention_core(_np(Q), _np(K), _np(V))
    assert normwise_rel_err(_np(naive[0]), ref_o) <= 1e-5 and normwise_rel_err(_np(naive[1]), ref_a) <= 1e-5
    trit = fused_slot_attention_triton(Q, K, V)
    for backend in ("auto", "triton", "hip"):
        got = slot_attention_fn(Q, K, V, backend=backend)
        assert torch.equal(got[0], trit[0]) and torch.equal(got[1], trit[1])
    ref_o, _ = sa.slot_attention_core(_np(Q), _np(K), _np(V), denom_eps=1e-8)
    assert normwise_rel_err(_np(trit[0]), ref_o) <= 1e-5


def test_scan_aliases():
    from hclsm_amd.kernels import (fused_ssm_scan_hip, fused_ssm_scan_triton, parallel_ssm_scan_pytorch,
                                   sequential_ssm_scan, ssm_scan_fn)
    from hclsm_amd.workloads import scan_inputs
    d = scan_inputs(4, 19, 96, 16, seed=23)
    g = torch.Generator().manual_seed(5)
    d["dt"] = torch.rand(4, 19, 96, generator=g) + 0.01          # the model clamps bind on this draw
    d["A_log"] = torch.randn(96, 16, generator=g)
    args = [d[k].cuda() for k in ("x", "dt", "A_log", "B", "C")]
    raw = fused_ssm_scan_hip(*args, clamp_mode="raw")
    model = fused_ssm_scan_hip(*args, clamp_mode="model")
    assert torch.equal(fused_ssm_scan_triton(*args), raw)
    assert torch.equal(parallel_ssm_scan_pytorch(*args), raw)
    assert torch.equal(sequential_ssm_scan(*args), model)
    for backend, want in (("triton", raw), ("parallel", raw), ("hip", raw), ("auto", raw),
                          ("sequential", model), ("something-else", model)):
        assert torch.equal(ssm_scan_fn(*args, backend=backend), want), backend
    np_args = [_np(t) for t in args]
    assert normwise_rel_err(_np(raw), ssm_scan_ref(*np_args, clamp_mode="raw")) <= 1e-5
    assert normwise_rel_err(_np(model), ssm_scan_ref(*np_args, clamp_mode="model")) <= 1e-5
