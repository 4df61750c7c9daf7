"""GPU parity of the slot tracker (hclsm_slot_track_* and the SlotTracker module) against oracle/objects.py.

* cost: tracker_cost_ref; fp32 normwise 1e-5 over alive pairs, 5e-3 absolute where a dead-slot penalty
  puts the cost near 1e4 / 2e4 (fp32 spacing there is 1e-3 / 2e-3); bf16 operands 2e-2.
* Sinkhorn matching: sinkhorn_ref on the same fp32 cost.  Confidence within 1e-4 (all alive) or 5e-3
  (dead slots: the 1e4 penalties put log_alpha near -2e5, where fp32 spacing is 0.016; an fp32 emulation
  of the reference's ops differs from float64 by 1.2e-3 there); perm and matched bit-exact on every row
  whose top-2 gap in the oracle's assignment exceeds twice the tolerance.  Rows left out: alive slots
  whose favoured partner is dead (every entry underflows, fp32 and the reference's fp32 torch code return
  index 0 where float64 still orders them) and near-ties; the test bounds their share.
* reorder + GRU: reorder_update_ref; reordered bit-exact, hidden fp32 1e-5 / bf16 2e-2.
* whole loop: track_sequence_ref with discriminative match weights (the score falls with |a - b|) on clips
  whose slots move by a random permutation per frame with their alive flags: every alive row's top-2 gap
  is above 0.98 in the oracle and dead rows resolve to exact ties (lowest index), so tracked slots, alive
  and perms are bit-exact; final hidden 1e-5 / 2e-2.
"""

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


def _module(D, N, seed, discriminative=False):
    from hclsm_amd.objects import SlotTracker
    torch.manual_seed(seed)
    m = SlotTracker(SimpleNamespace(d_slot=D, n_max_slots=N)).cuda()
    if discriminative:
        with torch.no_grad():
            for p in m.match_mlp.parameters():
                p.mul_(0.1)
            w1 = m.match_mlp[0].weight
            w1[:, 2 * D:] += torch.eye(D, device="cuda")
            w2 = m.match_mlp[2].weight
            for q in range(D // 4):
                w2[q, 4 * q:4 * q + 4] += 1.0
            m.match_mlp[4].weight.add_(-0.05)
    return m


def _params(m):
    return {k: _np(v) for k, v in m.state_dict().items()}


def _slots(F, N, D, seed, dead=0.25):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(F, N, D, generator=g)
    b = torch.randn(F, N, D, generator=g)
    at = (torch.rand(F, N, generator=g) > dead).float()
    at1 = (torch.rand(F, N, generator=g) > dead).float()
    return a.cuda(), b.cuda(), at.cuda(), at1.cuda()


COST_CASES = [  # F, N, D
    (3, 16, 128),    # tiny preset (config.py:199-203)
    (2, 32, 192),    # small preset
    (2, 24, 64),     # ragged N (pairs spill across workgroup tiles and frames)
    (1, 64, 256),    # base preset
    (1, 128, 384),   # large preset
]


def _check_cost(cost, ref, at, at1, tol):
    alive = (at[:, :, None] > 0.5) & (at1[:, None, :] > 0.5)
    assert normwise_rel_err(cost[alive], ref[alive]) <= tol
    if (~alive).any():
        scale = np.abs(ref[alive]).max() if alive.any() else 1.0
        assert np.abs(cost[~alive] - ref[~alive]).max() <= 5e-3 + 4 * tol * scale


@pytest.mark.parametrize("F,N,D", COST_CASES)
def test_cost_fp32_matches_oracle(F, N, D):
    from hclsm_amd.kernels.slot_tracker import TrackerWeights, track_cost
    m = _module(D, N, seed=F + N + D)
    a, b, at, at1 = _slots(F, N, D, seed=N + D)
    a[0, 0, :5] = 80.0   # beyond the +-50 input clamp
    W = TrackerWeights.from_module(m, torch.float32)
    cost = track_cost(a, b, at, at1, W)
    ref = ob.tracker_cost_ref(_np(a), _np(b), _np(at), _np(at1), _params(m))
    _check_cost(_np(cost), ref, _np(at), _np(at1), 1e-5)
    # no alive masks: no penalties
    cost0 = track_cost(a, b, None, None, W)
    one = np.ones((F, N))
    assert normwise_rel_err(_np(cost0), ob.tracker_cost_ref(_np(a), _np(b), one, one, _params(m))) <= 1e-5


@pytest.mark.parametrize("F,N,D", COST_CASES)
def test_cost_bf16_matches_oracle(F, N, D):
    from hclsm_amd.kernels.slot_tracker import TrackerWeights, track_cost
    m = _module(D, N, seed=F + N + D + 1)
    a, b, at, at1 = _slots(F, N, D, seed=N + D + 1)
    W = TrackerWeights.from_module(m, torch.bfloat16)
    cost = track_cost(a, b, at, at1, W)
    ref = ob.tracker_cost_ref(_np(a), _np(b), _np(at), _np(at1), _params(m))
    _check_cost(_np(cost), ref, _np(at), _np(at1), 2e-2)


def _crafted_cost(F, N, seed, dead):
    """Costs favouring a random permutation by ~1 with noise 0.3, plus the reference's penalties."""
    g = torch.Generator().manual_seed(seed)
    base = 0.3 * torch.randn(F, N, N, generator=g)
    for f in range(F):
        base[f, torch.arange(N), torch.randperm(N, generator=g)] -= 1.0
    at = (torch.rand(F, N, generator=g) > dead).float()
    at1 = (torch.rand(F, N, generator=g) > dead).float()
    base, at, at1 = base.cuda(), at.cuda(), at1.cuda()
    score = -base
    score = score - 1e4 * (at < 0.5).float()[:, :, None]
    score = score - 1e4 * (at1 < 0.5).float()[:, None, :]
    return -score, at, at1


def _oracle_match(cost, at, at1):
    c = np.clip(_np(cost), -1e4, 1e4)
    la = -c / 0.05
    for _ in range(20):
        m = la.max(axis=2, keepdims=True)
        la = la - (m + np.log(np.exp(la - m).sum(axis=2, keepdims=True)))
        m = la.max(axis=1, keepdims=True)
        la = la - (m + np.log(np.exp(la - m).sum(axis=1, keepdims=True)))
    A = np.exp(la)
    perm, conf = ob.sinkhorn_ref(c)
    srt = np.sort(A, axis=-1)
    gap = srt[..., -1] - srt[..., -2]
    matched = (_np(at) > 0.5) * np.take_along_axis(_np(at1) > 0.5, perm, 1) * (conf > 0.3)
    return perm, conf, matched, gap


@pytest.mark.parametrize("N", [16, 32, 48, 64, 100, 128])
@pytest.mark.parametrize("dead", [0.0, 0.25])
def test_match_matches_oracle(N, dead):
    from hclsm_amd.kernels.slot_tracker import track_match
    F = 6
    cost, at, at1 = _crafted_cost(F, N, seed=N + int(100 * dead), dead=dead)
    perm, matched, conf = track_match(cost, at, at1)
    rp, rc, rm, gap = _oracle_match(cost, at, at1)
    tol = 1e-4 if dead == 0.0 else 5e-3
    assert np.abs(_np(conf) - rc).max() <= tol
    sure = gap > 2 * tol
    assert sure.mean() >= (0.95 if dead == 0.0 else 0.7), f"only {sure.mean():.3f} of the rows are decisive"
    assert (perm.cpu().numpy()[sure] == rp[sure]).all()
    clear = sure & (np.abs(rc - 0.3) > 2 * tol)
    assert (_np(matched)[clear] == rm[clear]).all()


def test_match_edge_cases():
    """n_iters = 0 (argmax of exp(-cost / T) itself), one slot, no alive masks, confidence threshold."""
    from hclsm_amd.kernels.slot_tracker import track_match
    cost, at, at1 = _crafted_cost(3, 32, seed=5, dead=0.0)
    perm, matched, conf = track_match(cost, None, None, n_iters=0)
    la = -np.clip(_np(cost), -1e4, 1e4) / 0.05
    assert (perm.cpu().numpy() == la.argmax(-1)).all()
    np.testing.assert_allclose(_np(conf), np.exp(la.max(-1)), rtol=1e-5)
    c1 = torch.full((4, 1, 1), 0.7, device="cuda")
    perm, matched, conf = track_match(c1)
    assert (perm == 0).all() and torch.allclose(conf, torch.ones_like(conf)) and (matched == 1).all()


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_reorder_update_matches_oracle(dtype, tol):
    from hclsm_amd.kernels.slot_tracker import TrackerWeights, track_reorder_update
    F, N, D = 4, 32, 192
    m = _module(D, N, seed=3)
    g = torch.Generator().manual_seed(4)
    s1 = torch.randn(F, N, D, generator=g).cuda()
    h = torch.randn(F, N, D, generator=g).cuda()
    perm = torch.stack([torch.randperm(N, generator=g) for _ in range(F)]).cuda()
    perm[0, :3] = 5    # argmax perms need not be permutations
    matched = (torch.rand(F, N, generator=g) > 0.3).float().cuda()
    W = TrackerWeights.from_module(m, dtype)
    re, h1 = track_reorder_update(s1, perm, h, matched, W)
    rre, rh = ob.reorder_update_ref(_np(s1), perm.cpu().numpy(), _np(h), _np(matched), _params(m))
    assert (_np(re) == rre).all()
    assert normwise_rel_err(_np(h1), rh) <= tol


def _clip(B, T, N, D, seed, dead=0.2):
    """Slots that move between frames: frame t = frame t-1 permuted + noise 0.1, alive flags moving with
    them."""
    g = torch.Generator().manual_seed(seed)
    x = torch.empty(B, T, N, D)
    alive = torch.empty(B, T, N)
    x[:, 0] = torch.randn(B, N, D, generator=g)
    alive[:, 0] = (torch.rand(B, N, generator=g) > dead).float()
    for t in range(1, T):
        for b in range(B):
            pi = torch.randperm(N, generator=g)
            x[b, t] = x[b, t - 1, pi] + 0.1 * torch.randn(N, D, generator=g)
            alive[b, t] = alive[b, t - 1, pi]
    return x.cuda(), alive.cuda()


SEQ_CASES = [  # B, T, N, D, dtype
    (3, 6, 32, 192, torch.float32),
    (3, 6, 32, 192, torch.bfloat16),
    (2, 5, 16, 128, torch.float32),
    (2, 4, 48, 128, torch.float32),
    (1, 4, 128, 384, torch.bfloat16),
]


@pytest.mark.parametrize("B,T,N,D,dtype", SEQ_CASES)
def test_sequence_matches_oracle(B, T, N, D, dtype):
    from hclsm_amd.kernels.slot_tracker import TrackerWeights, track_sequence
    m = _module(D, N, seed=B + T + N, discriminative=True)
    x, alive = _clip(B, T, N, D, seed=N + D)
    W = TrackerWeights.from_module(m, dtype)
    r = track_sequence(x, alive, W, with_hidden=True)
    rt, ra, rh = ob.track_sequence_ref(_np(x), _np(alive), _params(m))
    assert (_np(r["tracked"]) == rt).all()
    assert (_np(r["alive"]) == ra).all()
    assert normwise_rel_err(_np(r["hidden"]), rh) <= (1e-5 if dtype == torch.float32 else 2e-2)
    # frame 0 is the identity; perm of frame t indexes the slots of frame t
    assert (r["perm"][:, 0].cpu() == torch.arange(N)).all()
    gathered = torch.gather(x, 2, r["perm"][..., None].expand(B, T, N, D))
    assert torch.equal(gathered, r["tracked"])


def test_sequence_without_hidden_or_alive():
    from hclsm_amd.kernels.slot_tracker import TrackerWeights, track_sequence
    B, T, N, D = 2, 5, 32, 128
    m = _module(D, N, seed=11, discriminative=True)
    x, _ = _clip(B, T, N, D, seed=12)
    W = TrackerWeights.from_module(m, torch.float32)
    r = track_sequence(x, None, W)
    assert r["hidden"] is None and r["alive"] is None
    rt, _, _ = ob.track_sequence_ref(_np(x), np.ones((B, T, N)), _params(m))
    assert (_np(r["tracked"]) == rt).all()
    r1 = track_sequence(x[:, :1], None, W)   # one frame: nothing to match
    assert torch.equal(r1["tracked"], x[:, :1])


def test_module_paths():
    """SlotTracker: C path under no_grad, torch path with autograd, both against the oracle; track() against
    the oracle's loop; state-dict names of the reference module."""
    D, N = 128, 16
    m = _module(D, N, seed=21, discriminative=True)
    assert set(m.state_dict()) == {"match_mlp.0.weight", "match_mlp.0.bias", "match_mlp.2.weight",
                                   "match_mlp.2.bias", "match_mlp.4.weight", "match_mlp.4.bias",
                                   "hidden_gru.weight_ih", "hidden_gru.weight_hh", "hidden_gru.bias_ih",
                                   "hidden_gru.bias_hh"}
    x, alive = _clip(2, 4, N, D, seed=22)
    rt, ra, rh = ob.track_sequence_ref(_np(x), _np(alive), _params(m))
    with torch.no_grad():
        t, a, h = m.track(x, alive, return_hidden=True)
        assert (_np(t) == rt).all() and (_np(a) == ra).all()
        assert normwise_rel_err(_np(h), rh) <= 1e-5
        cost = m.compute_cost_matrix(x[:, 0], x[:, 1], alive[:, 0], alive[:, 1])
    xg = x.clone().requires_grad_(True)
    t2, a2, h2 = m.track(xg, alive, return_hidden=True)     # torch path
    assert (_np(t2) == rt).all() and (_np(a2) == ra).all()
    assert normwise_rel_err(_np(h2), rh) <= 1e-5
    t2.sum().backward()
    assert xg.grad is not None
    cost2 = m.compute_cost_matrix(xg[:, 0], xg[:, 1], alive[:, 0], alive[:, 1])
    ref = ob.tracker_cost_ref(_np(x[:, 0]), _np(x[:, 1]), _np(alive[:, 0]), _np(alive[:, 1]), _params(m))
    _check_cost(_np(cost), ref, _np(alive[:, 0]), _np(alive[:, 1]), 1e-5)
    _check_cost(_np(cost2), ref, _np(alive[:, 0]), _np(alive[:, 1]), 1e-5)


def test_shape_limits():
    from hclsm_amd.kernels.slot_tracker import track_supported
    assert track_supported(32, 192, torch.bfloat16, sequence=True)
    assert track_supported(128, 384, torch.float32, sequence=True)
    assert not track_supported(129, 192, torch.float32, sequence=True)
    assert not track_supported(32, 96, torch.float32)
    assert not track_supported(32, 448, torch.bfloat16)


@pytest.mark.parametrize("F,N,D", [COST_CASES[1], COST_CASES[3], COST_CASES[4]])
def test_cost_fp16_matches_oracle(F, N, D):
    """fp16 operands: the weight-resident kernel (D <= 192) and the chunked one."""
    from hclsm_amd.kernels.slot_tracker import TrackerWeights, track_cost
    m = _module(D, N, seed=F + N + D + 3)
    a, b, at, at1 = _slots(F, N, D, seed=N + D + 3)
    W = TrackerWeights.from_module(m, torch.float16)
    cost = track_cost(a, b, at, at1, W)
    ref = ob.tracker_cost_ref(_np(a), _np(b), _np(at), _np(at1), _params(m))
    _check_cost(_np(cost), ref, _np(at), _np(at1), 1e-2)


def test_sequence_fp16_matches_oracle():
    from hclsm_amd.kernels.slot_tracker import TrackerWeights, track_sequence
    B, T, N, D = 2, 5, 32, 192
    m = _module(D, N, seed=31, discriminative=True)
    x, alive = _clip(B, T, N, D, seed=32)
    W = TrackerWeights.from_module(m, torch.float16)
    r = track_sequence(x, alive, W, with_hidden=True)
    rt, ra, rh = ob.track_sequence_ref(_np(x), _np(alive), _params(m))
    assert (_np(r["tracked"]) == rt).all() and (_np(r["alive"]) == ra).all()
    assert normwise_rel_err(_np(r["hidden"]), rh) <= 1e-2
