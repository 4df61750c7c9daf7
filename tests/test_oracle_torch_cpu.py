"""The torch CPU restatements used for bench.py's CPU baseline agree with the pinned numpy oracle."""

from __future__ import annotations

import numpy as np
import torch

from oracle import events as oe
from oracle import slot_attention as osa
from oracle import torch_cpu as tc
from oracle.ssm_scan import normwise_rel_err, ssm_scan_ref


def test_scan_torch_matches_oracle():
    from hclsm_amd.workloads import scan_inputs
    d = scan_inputs(3, 12, 20, 8, seed=4)
    for mode in ("raw", "model"):
        y = tc.scan_torch(d["x"], d["dt"], d["A_log"], d["B"], d["C"], D=d["D"], clamp_mode=mode)
        ref = ssm_scan_ref(*(d[k].numpy() for k in ("x", "dt", "A_log", "B", "C")), D=d["D"].numpy(), clamp_mode=mode)
        assert normwise_rel_err(y.numpy(), ref) <= 1e-5


def test_slot_forward_torch_matches_oracle():
    from hclsm_amd.workloads import slot_config
    tokens, slots0, w = slot_config(B=2, M=30, N=8, d=64, hidden=128)
    for kw in (dict(logit_clamp=None, renorm_eps=1e-8, slot_clamp=None),
               dict(logit_clamp=30.0, renorm_eps=None, slot_clamp=50.0)):
        got = tc.slot_forward_torch(tokens, slots0, w, 3, **kw)
        ref = osa.slot_attention_forward(tokens.numpy(), slots0.numpy(), {n: t.numpy() for n, t in w.items()}, 3, **kw)
        assert normwise_rel_err(got.numpy(), ref) <= 1e-5


def test_event_attention_torch_matches_oracle():
    g = torch.Generator().manual_seed(2)
    q, k, v = (torch.randn(6, 20, 2, 16, generator=g) for _ in range(3))
    m = (torch.rand(6, 20, generator=g) < 0.3).float()
    m[:, 0] = 1
    got = tc.event_attention_torch(q, k, v, m)
    ref = oe.track_causal_attention(q.numpy(), k.numpy(), v.numpy(), oe.event_index(m.numpy()))
    assert normwise_rel_err(got.numpy(), ref) <= 1e-5
