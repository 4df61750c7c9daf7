"""CPU tests of the folded-LayerNorm weight sets (no GPU): SlotWeights' w1_n / w1_n_sum / w1_n_bias and
Level1Weights' fold array implement LN(x) W^T + b = rstd (x Wn^T - mean rowsum(Wn)) + (W beta + b) with
Wn = W diag(gamma) rounded to the compute dtype.  Each stored tensor is checked against its definition and the
stored set against the unfolded layer in float64 on rows with a mean offset, to the rounding of Wn: a gamma
applied on the wrong axis, a missing bias term or swapped w1 / w3 halves fail."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import torch

from oracle import slot_attention as sa


def _f64(t):
    return t.detach().double().cpu().numpy()


def _folded_apply(x, wn, s, b):
    """rstd (x wn^T - mean s) + b in float64 (the kernels' epilogue form)."""
    mu = x.mean(1, keepdims=True)
    rstd = 1.0 / np.sqrt(((x - mu) ** 2).mean(1, keepdims=True) + 1e-5)
    return rstd * (x @ wn.T - mu * s[None, :]) + b[None, :]


def _rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def test_slot_weights_fold_norm_slots_into_w1():
    from hclsm_amd.kernels.slot_iteration import SlotWeights
    from hclsm_amd.workloads import slot_config
    g = torch.Generator().manual_seed(7)
    d, hidden = 64, 128
    _, _, w = slot_config(B=1, M=8, N=4, d=d, hidden=hidden, seed=3)
    w["ln_mlp_w"] = torch.rand(d, generator=g) + 0.5
    w["ln_mlp_b"] = torch.randn(d, generator=g) * 0.3
    w["b1"] = torch.randn(hidden, generator=g) * 0.2
    W = SlotWeights.from_dict(w, torch.bfloat16, device="cpu")
    w1, gam, bet, b1 = (_f64(torch.as_tensor(w[k])) for k in ("w1", "ln_mlp_w", "ln_mlp_b", "b1"))
    wn = W.t["w1_n"]
    assert wn.dtype == torch.bfloat16 and wn.shape == (hidden, d)
    assert torch.equal(wn, (torch.as_tensor(w["w1"]).float() * torch.as_tensor(w["ln_mlp_w"]).float()[None, :]).to(torch.bfloat16))
    assert np.allclose(_f64(W.t["w1_n_sum"]), _f64(wn).sum(1), rtol=1e-6, atol=1e-6)
    assert np.allclose(_f64(W.t["w1_n_bias"]), w1 @ bet + b1, rtol=1e-5, atol=1e-5)
    h = _f64(torch.randn(40, d, generator=g)) * 0.7 + 1.5
    want = sa.layer_norm(h, gam, bet) @ w1.T + b1
    got = _folded_apply(h, _f64(wn), _f64(W.t["w1_n_sum"]), _f64(W.t["w1_n_bias"]))
    assert _rel(got, want) <= 8e-3
    # fp32 weight sets carry no folded copy (the fp32 iteration keeps its LayerNorm launch)
    assert "w1_n" not in SlotWeights.from_dict(w, torch.float32, device="cpu").t


def test_level1_weights_fold_array():
    from hclsm_amd.dynamics import Level1EventDynamics
    from hclsm_amd.kernels.level1_packed import Level1Weights
    torch.manual_seed(11)
    cfg = SimpleNamespace(d_model=128, n_layers=2, n_heads=2)
    l1 = Level1EventDynamics(cfg, 64)
    g = torch.Generator().manual_seed(12)
    with torch.no_grad():
        for ln in [l1.norm] + [m for b in l1.blocks for m in (b.norm1, b.norm2)]:
            ln.weight.copy_(torch.rand(ln.weight.shape, generator=g) + 0.5)
            ln.bias.copy_(torch.randn(ln.bias.shape, generator=g) * 0.3)
    W = Level1Weights.from_module(l1, torch.bfloat16)
    assert W.fold is not None and len(W.fold) == 3 + 7 * cfg.n_layers and W.fold_ptrs is not None
    assert Level1Weights.from_module(l1, torch.float32).fold is None
    x = _f64(torch.randn(50, cfg.d_model, generator=g)) * 0.8 - 1.2

    def check(w_mod, ln, wn, s, b):
        want = sa.layer_norm(x, _f64(ln.weight), _f64(ln.bias)) @ _f64(w_mod).T
        assert wn.dtype == torch.bfloat16 and np.allclose(_f64(s), _f64(wn).sum(1), rtol=1e-6, atol=1e-6)
        assert _rel(_folded_apply(x, _f64(wn), _f64(s), _f64(b)), want) <= 8e-3

    check(l1.proj_out.weight, l1.norm, *W.fold[0:3])
    H = l1.blocks[0].ffn.w1.weight.shape[0]
    for i, blk in enumerate(l1.blocks):
        qkv, qkv_s, qkv_b, w1n, w3n, sums, bias = W.fold[3 + 7 * i: 10 + 7 * i]
        check(blk.attn.in_proj_weight, blk.norm1, qkv, qkv_s, qkv_b)
        check(blk.ffn.w1.weight, blk.norm2, w1n, sums[:H], bias[:H])   # w1 rows first
        check(blk.ffn.w3.weight, blk.norm2, w3n, sums[H:], bias[H:])   # then w3
