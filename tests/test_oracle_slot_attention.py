"""CPU pins of oracle/slot_attention.py against torch's library modules and closed forms.

  * core: torch.softmax(dim=1) + bmm; columns sum to 1 (tests/test_kernels.py:66-71);
    +eps gives column sums S/(S+eps); token-permutation invariance of out and slot
    equivariance; the reference test fixtures (tests/test_kernels.py:50-56).
  * GRU: torch.nn.GRUCell with identical weights.
  * iteration: a torch composition of nn.LayerNorm / nn.Linear / nn.GRUCell / softmax with
    identical weights, in both the reference mode (clamps) and config-2 mode (renorm).
  * renorm: rows of the renormalised attention sum to 1 over tokens.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import slot_attention as sa


@pytest.mark.parametrize("B,N,M,D", [(2, 16, 64, 128), (1, 8, 32, 64), (4, 32, 196, 256)])
def test_core_against_torch_softmax_and_column_sums(B, N, M, D):
    g = torch.Generator().manual_seed(B * N)
    Q, K, V = (torch.randn(s, generator=g, dtype=torch.float64) for s in ((B, N, D), (B, M, D), (B, M, D)))
    out, attn = sa.slot_attention_core(Q.numpy(), K.numpy(), V.numpy())
    ref_attn = torch.softmax(torch.bmm(Q, K.transpose(1, 2)) * D ** -0.5, dim=1)
    np.testing.assert_allclose(attn, ref_attn.numpy(), rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(out, torch.bmm(ref_attn, V).numpy(), rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(attn.sum(axis=1), 1.0, atol=1e-12)


def test_core_denominator_eps_and_permutations():
    r = np.random.default_rng(1)
    Q, K, V = r.standard_normal((2, 5, 8)), r.standard_normal((2, 7, 8)), r.standard_normal((2, 7, 8))
    out0, a0 = sa.slot_attention_core(Q, K, V)
    out1, a1 = sa.slot_attention_core(Q, K, V, denom_eps=1e-3)
    logits = np.einsum("bnd,bmd->bnm", Q, K) / np.sqrt(8)
    e = np.exp(logits - logits.max(1, keepdims=True))
    S = e.sum(1)
    np.testing.assert_allclose(a1.sum(1), S / (S + 1e-3), rtol=1e-12)
    pm = r.permutation(7)
    o2, a2 = sa.slot_attention_core(Q, K[:, pm], V[:, pm])
    np.testing.assert_allclose(o2, out0, rtol=1e-12)
    np.testing.assert_allclose(a2, a0[:, :, pm], rtol=1e-12)
    pn = r.permutation(5)
    o3, _ = sa.slot_attention_core(Q[:, pn], K, V)
    np.testing.assert_allclose(o3, out0[:, pn], rtol=1e-12)


def test_gru_cell_matches_torch():
    g = torch.Generator().manual_seed(3)
    cell = nn.GRUCell(12, 12).double()
    x = torch.randn(5, 12, generator=g, dtype=torch.float64)
    h = torch.randn(5, 12, generator=g, dtype=torch.float64)
    ref = cell(x, h).detach().numpy()
    got = sa.gru_cell(x.numpy(), h.numpy(), cell.weight_ih.detach().numpy(), cell.weight_hh.detach().numpy(),
                      cell.bias_ih.detach().numpy(), cell.bias_hh.detach().numpy())
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-14)


def _torch_iteration(slots, k, v, mods, logit_clamp, renorm_eps, slot_clamp):
    """dynamic_slots.py:98-131 written with torch modules (library routines)."""
    ln_pre, wq, gru, ln_mlp, mlp = mods
    B, N, d = slots.shape
    q = wq(ln_pre(slots))
    logits = torch.bmm(q, k.transpose(1, 2)) * d ** -0.5
    if logit_clamp:
        logits = logits.clamp(-logit_clamp, logit_clamp)
    attn = F.softmax(logits, dim=1)
    if renorm_eps is not None:
        attn = attn + renorm_eps
        attn = attn / attn.sum(dim=-1, keepdim=True)
    upd = torch.bmm(attn, v)
    s = gru(upd.reshape(-1, d), slots.reshape(-1, d)).reshape(B, N, d)
    s = s + mlp(ln_mlp(s))
    if slot_clamp:
        s = s.clamp(-slot_clamp, slot_clamp)
    return s


@pytest.mark.parametrize("mode", ["reference", "config2"])
def test_iteration_matches_torch_modules(mode):
    torch.manual_seed(4)
    d, hidden, B, N, M = 16, 64 if mode == "reference" else 24, 2, 5, 9
    ln_pre, ln_mlp = nn.LayerNorm(d).double(), nn.LayerNorm(d).double()
    with torch.no_grad():
        for ln in (ln_pre, ln_mlp):
            ln.weight.uniform_(0.5, 1.5)
            ln.bias.uniform_(-0.2, 0.2)
    wq = nn.Linear(d, d, bias=False).double()
    gru = nn.GRUCell(d, d).double()
    mlp = nn.Sequential(nn.Linear(d, hidden), nn.ReLU(), nn.Linear(hidden, d)).double()
    slots = torch.randn(B, N, d, dtype=torch.float64) * 3
    k = torch.randn(B, M, d, dtype=torch.float64) * 3
    v = torch.randn(B, M, d, dtype=torch.float64)
    kw = dict(logit_clamp=30.0, renorm_eps=None, slot_clamp=0.5) if mode == "reference" else \
        dict(logit_clamp=None, renorm_eps=1e-8, slot_clamp=None)
    ref = _torch_iteration(slots, k, v, (ln_pre, wq, gru, ln_mlp, mlp), **kw).detach().numpy()
    W = dict(ln_pre_w=ln_pre.weight, ln_pre_b=ln_pre.bias, w_q=wq.weight, w_ih=gru.weight_ih, w_hh=gru.weight_hh,
             b_ih=gru.bias_ih, b_hh=gru.bias_hh, ln_mlp_w=ln_mlp.weight, ln_mlp_b=ln_mlp.bias,
             w1=mlp[0].weight, b1=mlp[0].bias, w2=mlp[2].weight, b2=mlp[2].bias)
    W = {n: t.detach().numpy() for n, t in W.items()}
    got = sa.slot_iteration(slots.numpy(), k.numpy(), v.numpy(), W, **kw)
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-12)
    if mode == "reference":
        assert np.abs(got).max() <= 0.5 + 1e-15    # slot clamp applied


def test_logit_clamp_binds_and_renorm_rows_sum_to_one():
    r = np.random.default_rng(5)
    Q = r.standard_normal((1, 3, 4)) * 40
    K = r.standard_normal((1, 6, 4)) * 40
    V = r.standard_normal((1, 6, 4))
    _, a_clamped = sa.slot_attention_core(Q, K, V, scale=1.0, logit_clamp=30.0)
    logits = np.clip(np.einsum("bnd,bmd->bnm", Q, K), -30, 30)
    e = np.exp(logits - logits.max(1, keepdims=True))
    np.testing.assert_allclose(a_clamped, e / e.sum(1, keepdims=True), rtol=1e-12)
    attn = a_clamped + 1e-8
    attn = attn / attn.sum(-1, keepdims=True)
    np.testing.assert_allclose(attn.sum(-1), 1.0, rtol=1e-12)


def _birth_case(M, seed=8):
    """Float64 torch modules for dynamic_slots_forward_ref and the oracle's W dict of the same weights."""
    torch.manual_seed(seed)
    d, d_in, B, N = 16, 12, 3, 6
    mods = dict(ln_in=nn.LayerNorm(d_in), ln_pre=nn.LayerNorm(d), wq=nn.Linear(d, d, bias=False),
                wk=nn.Linear(d_in, d, bias=False), wv=nn.Linear(d_in, d, bias=False), gru=nn.GRUCell(d, d),
                ln_mlp=nn.LayerNorm(d), mlp=nn.Sequential(nn.Linear(d, 4 * d), nn.ReLU(), nn.Linear(4 * d, d)),
                head=nn.Sequential(nn.Linear(d, d // 4), nn.ReLU(), nn.Linear(d // 4, 1)), birth=nn.Linear(d_in, d))
    mods = {k: m.double() for k, m in mods.items()}
    W = dict(ln_in_w=mods["ln_in"].weight, ln_in_b=mods["ln_in"].bias, ln_pre_w=mods["ln_pre"].weight,
             ln_pre_b=mods["ln_pre"].bias, w_q=mods["wq"].weight, w_k=mods["wk"].weight, w_v=mods["wv"].weight,
             w_ih=mods["gru"].weight_ih, w_hh=mods["gru"].weight_hh, b_ih=mods["gru"].bias_ih,
             b_hh=mods["gru"].bias_hh, ln_mlp_w=mods["ln_mlp"].weight, ln_mlp_b=mods["ln_mlp"].bias,
             w1=mods["mlp"][0].weight, b1=mods["mlp"][0].bias, w2=mods["mlp"][2].weight, b2=mods["mlp"][2].bias,
             e1_w=mods["head"][0].weight, e1_b=mods["head"][0].bias, e2_w=mods["head"][2].weight,
             e2_b=mods["head"][2].bias, birth_w=mods["birth"].weight, birth_b=mods["birth"].bias)
    W = {k: v.detach().numpy() for k, v in W.items()}
    x = torch.randn(B, M, d_in, dtype=torch.float64)
    s0 = torch.randn(B, N, d, dtype=torch.float64)
    return mods, W, x, s0


def test_dynamic_slots_forward_and_birth_against_torch_modules():
    """dynamic_slots.py:149-199 with torch modules: the iterations, the existence head, and birth at the first
    dormant slot from birth_proj(inputs[b, argmax residual]) -- M = 1 token, so the residual's argmax is 0 and
    the birth decision is exact; thresholds that make every / no clip give birth."""
    mods, W, x, s0 = _birth_case(M=1)
    with torch.no_grad():
        xn = mods["ln_in"](x)
        k, v = mods["wk"](xn), mods["wv"](xn)
        s = s0
        for _ in range(2):
            s = _torch_iteration(s, k, v, (mods["ln_pre"], mods["wq"], mods["gru"], mods["ln_mlp"], mods["mlp"]),
                                 30.0, None, 50.0)
        alive = torch.sigmoid(mods["head"](s).squeeze(-1))
        born = mods["birth"](x[:, 0])
    thr = float(alive.median())                        # some slots dormant in some clips
    got, got_alive = sa.dynamic_slots_forward_ref(x.numpy(), s0.numpy(), W, 2, thr, -1.0)
    np.testing.assert_allclose(got_alive, alive.numpy(), rtol=1e-12, atol=1e-14)
    want = s.clone()
    births = 0
    for b in range(x.shape[0]):
        dormant = torch.nonzero(alive[b] < thr).flatten()
        if len(dormant):
            want[b, dormant[0]] = born[b]
            births += 1
    assert births >= 2
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-10, atol=1e-12)
    none, _ = sa.dynamic_slots_forward_ref(x.numpy(), s0.numpy(), W, 2, thr, 2.0)      # residual <= 1: no birth
    np.testing.assert_allclose(none, s.numpy(), rtol=1e-10, atol=1e-12)
    none, _ = sa.dynamic_slots_forward_ref(x.numpy(), s0.numpy(), W, 2, 0.0, -1.0)     # nothing dormant
    np.testing.assert_allclose(none, s.numpy(), rtol=1e-10, atol=1e-12)


def test_birth_residual_is_rounding_noise():
    """The residual |1 - sum over slots of a softmax over slots| is rounding noise (every token's column sums to
    one), so a birth threshold above ~1e-12 never fires -- the decision the reference takes in practice."""
    mods, W, x, s0 = _birth_case(M=9, seed=9)
    got, alive = sa.dynamic_slots_forward_ref(x.numpy(), s0.numpy(), W, 1, 1.0, 1e-9)
    plain, _ = sa.dynamic_slots_forward_ref(x.numpy(), s0.numpy(), W, 1, 0.0, 1e-9)
    np.testing.assert_array_equal(got, plain)
