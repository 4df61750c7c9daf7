"""CPU pins of oracle/modules.py against torch's library modules with identical weights.

The SSM block's scan is the (separately pinned) scan oracle; around it the block is checked
against nn.LayerNorm / nn.Linear / softplus / silu.  The event block is checked against
nn.MultiheadAttention (bias=False, batch_first, key_padding_mask) + the SwiGLU FFN built from
nn.Linear.  The mask rule is checked on constructed cases."""

from __future__ import annotations

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import modules as om
from oracle.ssm_scan import ssm_scan_ref


def _sd(module):
    return {k: v.detach().double().numpy() for k, v in module.state_dict().items()}


def test_ssm_block_against_torch_pieces():
    torch.manual_seed(0)
    d, S = 16, 4
    norm, in_p, gate_p = nn.LayerNorm(d).double(), nn.Linear(d, 2 * d, bias=False).double(), nn.Linear(d, 2 * d, bias=False).double()
    dt_p, B_p, C_p = nn.Linear(2 * d, 2 * d).double(), nn.Linear(2 * d, S, bias=False).double(), nn.Linear(2 * d, S, bias=False).double()
    out_p = nn.Linear(2 * d, d, bias=False).double()
    A_log = torch.randn(2 * d, S, dtype=torch.float64)
    x = torch.randn(3, 7, d, dtype=torch.float64)
    with torch.no_grad():
        h = norm(x)
        z = in_p(h)
        gate = F.silu(gate_p(h))
        dt = F.softplus(dt_p(z)).clamp(1e-3, 1.0)
        y = ssm_scan_ref(z.numpy(), dt.numpy(), A_log.numpy(), B_p(z).numpy(), C_p(z).numpy(), clamp_mode="model")
        ref = (x + out_p(torch.from_numpy(y) * gate)).numpy()
    p = {"norm.weight": norm.weight, "norm.bias": norm.bias, "in_proj.weight": in_p.weight,
         "gate_proj.weight": gate_p.weight, "dt_proj.weight": dt_p.weight, "dt_proj.bias": dt_p.bias,
         "B_proj.weight": B_p.weight, "C_proj.weight": C_p.weight, "A_log": A_log, "out_proj.weight": out_p.weight}
    got = om.simplified_ssm_block_ref(x.numpy(), {k: v.detach().numpy() for k, v in p.items()})
    np.testing.assert_allclose(got, ref, rtol=1e-11, atol=1e-12)


def test_event_block_against_multihead_attention():
    torch.manual_seed(1)
    d, H, P, N = 32, 4, 5, 7
    norm1, norm2 = nn.LayerNorm(d).double(), nn.LayerNorm(d).double()
    mha = nn.MultiheadAttention(d, H, batch_first=True, bias=False).double()
    w1, w3, w2 = nn.Linear(d, 4 * d, bias=False).double(), nn.Linear(d, 4 * d, bias=False).double(), nn.Linear(4 * d, d, bias=False).double()
    x = torch.randn(P, N, d, dtype=torch.float64)
    kp = torch.rand(P, N) < 0.3
    kp[:, 0] = False
    with torch.no_grad():
        h = norm1(x)
        a, _ = mha(h, h, h, key_padding_mask=kp)
        x1 = x + a
        h2 = norm2(x1)
        ref = (x1 + w2(F.silu(w1(h2)) * w3(h2))).numpy()
    p = {"norm1.weight": norm1.weight, "norm1.bias": norm1.bias, "attn.in_proj_weight": mha.in_proj_weight,
         "attn.out_proj.weight": mha.out_proj.weight, "norm2.weight": norm2.weight, "norm2.bias": norm2.bias,
         "ffn.w1.weight": w1.weight, "ffn.w2.weight": w2.weight, "ffn.w3.weight": w3.weight}
    got = om.event_block_ref(x.numpy(), kp.numpy(), {k: v.detach().numpy() for k, v in p.items()}, H)
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-12)


def test_event_mask_rule_cases():
    tl = np.log(0.7 / 0.3)                             # threshold 0.7
    probs = np.array([[0.1, 0.8, 0.2], [0.9, 0.1, 0.75]])
    m = om.event_mask_rule_ref(probs, tl)
    np.testing.assert_array_equal(m, [[0, 1, 0], [1, 0, 1]])
    probs2 = np.array([[0.1, 0.2, 0.3], [0.1, 0.9, 0.1]])   # row 0 empty -> column 0 set in every row
    np.testing.assert_array_equal(om.event_mask_rule_ref(probs2, tl), [[1, 0, 0], [1, 1, 0]])


def _hier_case(B=3, T=9, N=5, D=8, DL2=12, S2=3, p=0.4, seed=0):
    g = np.random.default_rng(seed)
    mask = (g.random((B, T)) < p).astype(np.float32)
    mask[0, :] = 1.0            # a clip whose every frame is an event
    mask[1, :] = 0.0            # a clip with none
    K = max(int(mask.sum(axis=1).max()), 1)
    return (g.standard_normal((B, T, N, D)), g.standard_normal((B, K, N, D)), mask,
            g.standard_normal((B, S2, DL2)), (g.random((B, N)) < 0.7).astype(np.float64))


def test_hierarchy_forward_against_torch_modules():
    """hierarchy_manager.py:120-162 built from nn.Linear / nn.Sigmoid with the same weights, the scatter as a
    loop over each clip's events in ascending t."""
    from oracle.events import event_index
    torch.manual_seed(1)
    level0, level1, mask, ctx, obj = _hier_case()
    B, T, N, D = level0.shape
    l2_to_l1 = nn.Linear(ctx.shape[2], D, bias=False).double()
    gate = nn.Sequential(nn.Linear(2 * D, D), nn.Sigmoid()).double()
    comb = torch.tensor(level0)
    for b in range(B):
        for k, t in enumerate(np.nonzero(mask[b] > 0.5)[0]):
            comb[b, t] = torch.tensor(level1[b, k])
    l2b = l2_to_l1(torch.tensor(ctx).mean(dim=1))[:, None, None, :].expand_as(comb)
    gv = gate(torch.cat([comb, l2b], dim=-1))
    want = ((gv * l2b + (1 - gv) * comb) * torch.tensor(obj)[:, None, :, None]).detach().numpy()
    got = om.hierarchy_forward_ref(level0, level1, event_index(mask), l2_to_l1.weight.detach().numpy(),
                                   gate[0].weight.detach().numpy(), gate[0].bias.detach().numpy(), ctx, obj)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_hierarchy_forward_closed_forms():
    from oracle.events import event_index, scatter
    level0, level1, mask, ctx, obj = _hier_case(seed=2)
    B, T, N, D = level0.shape
    idx = event_index(mask)
    comb = scatter(level0, level1, idx)
    w_l2 = np.eye(D, ctx.shape[2])                  # l2 = the first D entries of the mean context
    l2 = ctx.mean(axis=1)[:, :D][:, None, None, :]
    w0 = np.zeros((D, 2 * D))
    # no context: the scatter times the alive mask
    np.testing.assert_array_equal(om.hierarchy_forward_ref(level0, level1, idx, w_l2, w0, None, None, obj),
                                  comb * obj[:, None, :, None])
    # a gate of exactly 1/2
    half = om.hierarchy_forward_ref(level0, level1, idx, w_l2, w0, np.zeros(D), ctx, None)
    np.testing.assert_allclose(half, 0.5 * (comb + l2), rtol=1e-14, atol=1e-14)
    # saturated gates select the Level-2 context or the scattered states
    hi = om.hierarchy_forward_ref(level0, level1, idx, w_l2, w0, np.full(D, 60.0), ctx, obj)
    np.testing.assert_allclose(hi, np.broadcast_to(l2, comb.shape) * obj[:, None, :, None], atol=1e-20)
    lo = om.hierarchy_forward_ref(level0, level1, idx, w_l2, w0, np.full(D, -60.0), ctx, obj)
    np.testing.assert_allclose(lo, comb * obj[:, None, :, None], rtol=1e-12, atol=1e-20)
    # only the combined half of W_gate sees the states: a gate on channel j from state channel j alone
    w = np.zeros((D, 2 * D))
    w[np.arange(D), np.arange(D)] = 1.0
    diag = om.hierarchy_forward_ref(level0, level1, idx, w_l2, w, None, ctx, None)
    s = 1.0 / (1.0 + np.exp(-comb))
    np.testing.assert_allclose(diag, s * l2 + (1 - s) * comb, rtol=1e-13, atol=1e-13)
