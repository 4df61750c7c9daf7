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


# ---------------------------------------------------------------------------
# Pins of the composite oracles' glue (level0_ssm_ref: level0_ssm.py:159-220; level1_ref:
# level1_event.py:85-133).  Each property fails for a plausible glue mistake: a mean over all objects
# instead of the alive ones, a condition broadcast over the wrong axis, a missing clamp / nan_to_num /
# mask, a mixing of events or slots, a pad mask that is not applied.
# ---------------------------------------------------------------------------

def _block_params(g, d, S, expand=2, zero_out=False):
    di = expand * d
    r = lambda *s: g.standard_normal(s) / np.sqrt(s[-1])
    p = {"norm.weight": 1 + 0.1 * g.standard_normal(d), "norm.bias": 0.1 * g.standard_normal(d),
         "in_proj.weight": r(di, d), "gate_proj.weight": r(di, d), "dt_proj.weight": r(di, di),
         "dt_proj.bias": g.standard_normal(di) - 1.0, "B_proj.weight": r(S, di), "C_proj.weight": r(S, di),
         "A_log": -0.5 * g.random((di, S)), "out_proj.weight": r(d, di)}
    if zero_out:
        p["out_proj.weight"] = np.zeros((d, di))
    return p


def _level0_params(g, d, S, n_blocks, zero_out=False, cond=None):
    p = {}
    for pre in ("global_blocks", "object_blocks"):
        for i in range(n_blocks):
            for k, v in _block_params(g, d, S, zero_out=zero_out).items():
                p[f"{pre}.{i}.{k}"] = v
    p["condition_proj.weight"] = g.standard_normal((d, d)) / np.sqrt(d) if cond is None else cond
    return p


def test_level0_dead_objects_do_not_reach_alive_outputs():
    g = np.random.default_rng(10)
    B, N, T, d, S = 2, 5, 6, 8, 4
    p = _level0_params(g, d, S, 2)
    s = g.standard_normal((B, N, T, d))
    mask = np.array([[1, 0, 1, 1, 0], [0, 1, 1, 0, 1]], np.float64)
    out = om.level0_ssm_ref(s, mask, p, 2)
    s2 = s.copy()
    s2[mask == 0] = 50 * g.standard_normal(s2[mask == 0].shape)
    out2 = om.level0_ssm_ref(s2, mask, p, 2)
    np.testing.assert_array_equal(out2[mask == 1], out[mask == 1])
    assert np.all(out[mask == 0] == 0) and np.all(out2[mask == 0] == 0)
    # the global mean is over alive objects: changing an alive object changes the other alive outputs
    s3 = s.copy()
    s3[0, 0] += 1.0
    out3 = om.level0_ssm_ref(s3, mask, p, 2)
    assert np.abs(out3[0, 2] - out[0, 2]).max() > 1e-6


def test_level0_object_permutation_equivariance_and_causality():
    g = np.random.default_rng(11)
    B, N, T, d, S = 2, 6, 7, 8, 4
    p = _level0_params(g, d, S, 1)
    s = g.standard_normal((B, N, T, d))
    mask = (g.random((B, N)) < 0.7).astype(np.float64)
    mask[:, 0] = 1
    out = om.level0_ssm_ref(s, mask, p, 1)
    perm = g.permutation(N)
    outp = om.level0_ssm_ref(s[:, perm], mask[:, perm], p, 1)
    np.testing.assert_allclose(outp, out[:, perm], rtol=1e-12, atol=1e-12)
    s2 = s.copy()
    s2[:, :, 4:] = g.standard_normal(s2[:, :, 4:].shape)
    out2 = om.level0_ssm_ref(s2, mask, p, 1)
    np.testing.assert_array_equal(out2[:, :, :4], out[:, :, :4])
    # no mask: the same as every object alive
    np.testing.assert_allclose(om.level0_ssm_ref(s, None, p, 1), om.level0_ssm_ref(s, np.ones((B, N)), p, 1),
                               rtol=1e-13, atol=1e-13)


def test_level0_reduces_to_the_object_blocks_without_conditioning():
    g = np.random.default_rng(12)
    B, N, T, d, S = 2, 3, 5, 8, 4
    p = _level0_params(g, d, S, 2, cond=np.zeros((8, 8)))
    s = g.standard_normal((B, N, T, d))
    mask = np.array([[1, 1, 0], [1, 0, 1]], np.float64)
    x = s.reshape(B * N, T, d)
    for i in range(2):
        x = om.simplified_ssm_block_ref(x, {k[len(f"object_blocks.{i}."):]: v for k, v in p.items()
                                            if k.startswith(f"object_blocks.{i}.")})
    want = np.clip(x.reshape(B, N, T, d), -100, 100) * mask[:, :, None, None]
    np.testing.assert_allclose(om.level0_ssm_ref(s, mask, p, 2), want, rtol=1e-13, atol=1e-13)
    # the global blocks then do not matter
    p2 = dict(p)
    for k in p:
        if k.startswith("global_blocks."):
            p2[k] = p[k] * 3.0
    np.testing.assert_array_equal(om.level0_ssm_ref(s, mask, p2, 2), om.level0_ssm_ref(s, mask, p, 2))


def test_level0_identity_blocks_give_the_conditioned_clamped_states():
    """With every out_proj zero each block is the identity (x + 0): the output is then
    clip(s + W_c . mean over alive objects of s, +-100) * mask, with NaN mapped to 0."""
    g = np.random.default_rng(13)
    B, N, T, d, S = 2, 4, 5, 8, 4
    W = g.standard_normal((d, d))
    p = _level0_params(g, d, S, 2, zero_out=True, cond=W)
    s = 40 * g.standard_normal((B, N, T, d))            # large enough for the +-100 clamp to bind
    mask = np.array([[1, 1, 0, 1], [0, 1, 1, 1]], np.float64)
    alive_mean = (s * mask[:, :, None, None]).sum(1) / mask.sum(1)[:, None, None]
    want = np.clip(s + (alive_mean @ W.T)[:, None], -100, 100) * mask[:, :, None, None]
    got = om.level0_ssm_ref(s, mask, p, 2)
    assert np.any(np.abs(got) == 100)
    np.testing.assert_allclose(got, want, rtol=1e-13, atol=1e-12)
    s[1, 2, 3, 0] = np.nan                               # an alive object's NaN: its frame's outputs become 0
    got = om.level0_ssm_ref(s, mask, p, 2)
    assert np.all(got[1, :, 3] == 0) and np.isfinite(got).all()


def _level1_params(g, d_slot, d_model, n_layers, hidden, zero_blocks=False):
    r = lambda *s: g.standard_normal(s) / np.sqrt(s[-1])
    p = {"proj_in.weight": r(d_model, d_slot), "norm.weight": 1 + 0.1 * g.standard_normal(d_model),
         "norm.bias": 0.1 * g.standard_normal(d_model), "proj_out.weight": r(d_slot, d_model)}
    for i in range(n_layers):
        b = {"norm1.weight": 1 + 0.1 * g.standard_normal(d_model), "norm1.bias": 0.1 * g.standard_normal(d_model),
             "attn.in_proj_weight": r(3 * d_model, d_model), "attn.out_proj.weight": r(d_model, d_model),
             "norm2.weight": 1 + 0.1 * g.standard_normal(d_model), "norm2.bias": 0.1 * g.standard_normal(d_model),
             "ffn.w1.weight": r(hidden, d_model), "ffn.w3.weight": r(hidden, d_model),
             "ffn.w2.weight": r(d_model, hidden)}
        if zero_blocks:
            b["attn.out_proj.weight"] = np.zeros((d_model, d_model))
            b["ffn.w2.weight"] = np.zeros((d_model, hidden))
        p.update({f"blocks.{i}.{k}": v for k, v in b.items()})
    return p


def _level1_case(seed, zero_blocks=False):
    g = np.random.default_rng(seed)
    B, K, N, d_slot, d_model, H = 2, 3, 5, 8, 16, 4
    p = _level1_params(g, d_slot, d_model, 2, 32, zero_blocks)
    ev = g.standard_normal((B, K, N, d_slot))
    pad = np.array([[1, 1, 0], [1, 1, 1]], np.float64)
    obj = np.array([[1, 0, 1, 1, 1], [1, 1, 1, 0, 0]], np.float64)
    return g, p, ev, pad, obj, H


def test_level1_events_are_independent_and_pads_are_zero():
    g, p, ev, pad, obj, H = _level1_case(20)
    out = om.level1_ref(ev, pad, obj, p, 2, H)
    assert np.all(out[0, 2] == 0)                        # padded event: exactly zero
    ev2 = ev.copy()
    ev2[0, 1] = g.standard_normal(ev2[0, 1].shape)       # another event of the same clip
    ev2[0, 2] = 1e3                                      # the padded event's own rows
    out2 = om.level1_ref(ev2, pad, obj, p, 2, H)
    np.testing.assert_array_equal(out2[0, 0], out[0, 0])
    np.testing.assert_array_equal(out2[1], out[1])
    assert np.abs(out2[0, 1] - out[0, 1]).max() > 1e-6
    # without a pad mask, event k of a padded slot is computed like any other
    raw = om.level1_ref(ev, None, obj, p, 2, H)
    np.testing.assert_array_equal(raw * pad[:, :, None, None], out)


def test_level1_slot_permutation_and_dead_keys():
    g, p, ev, pad, obj, H = _level1_case(21)
    out = om.level1_ref(ev, pad, obj, p, 2, H)
    perm = g.permutation(ev.shape[2])
    outp = om.level1_ref(ev[:, :, perm], pad, obj[:, perm], p, 2, H)
    np.testing.assert_allclose(outp, out[:, :, perm], rtol=1e-12, atol=1e-12)
    # keys of dead slots are excluded: the alive slots' outputs ignore the dead slots' states
    ev2 = ev.copy()
    dead = obj == 0
    ev2[:, :, :][np.broadcast_to(dead[:, None, :], ev.shape[:3])] = 7.0
    out2 = om.level1_ref(ev2, pad, obj, p, 2, H)
    alive = np.broadcast_to(~dead[:, None, :], ev.shape[:3])
    np.testing.assert_allclose(out2[alive], out[alive], rtol=1e-12, atol=1e-12)


def test_level1_identity_blocks_reduce_to_the_projections():
    """With attn.out_proj and ffn.w2 zero every block is the identity: out = proj_out(LN(proj_in ev))."""
    from oracle.slot_attention import layer_norm
    g, p, ev, pad, obj, H = _level1_case(22, zero_blocks=True)
    want = layer_norm(ev @ p["proj_in.weight"].T, p["norm.weight"], p["norm.bias"]) @ p["proj_out.weight"].T
    want = want * pad[:, :, None, None]
    np.testing.assert_allclose(om.level1_ref(ev, pad, obj, p, 2, H), want, rtol=1e-12, atol=1e-12)
