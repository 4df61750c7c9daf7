"""Pins of oracle/objects.py (RelationGraph, SlotTracker) against what the mathematics fixes: an
element-by-element loop restatement on tiny inputs, slot-permutation equivariance, dead-slot masking,
the agreement of the reference's two GNN paths for >= 2 rounds, Sinkhorn's marginals and its agreement
with the optimal assignment (scipy's Hungarian solver) on separated costs, torch's GRUCell."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import objects as ob
from oracle.slot_attention import layer_norm, sigmoid


def _gnn_params(D, E, seed):
    g = np.random.default_rng(seed)
    r = lambda *s: g.standard_normal(s) / np.sqrt(s[-1])
    return {"pair_norm.weight": 1 + 0.1 * g.standard_normal(4 * D), "pair_norm.bias": 0.1 * g.standard_normal(4 * D),
            "edge_mlp.0.weight": r(2 * E, 4 * D), "edge_mlp.0.bias": 0.1 * g.standard_normal(2 * E),
            "edge_mlp.2.weight": r(E, 2 * E), "edge_mlp.2.bias": 0.1 * g.standard_normal(E),
            "edge_weight.weight": r(1, E), "edge_weight.bias": 0.1 * g.standard_normal(1),
            "msg_mlp.0.weight": r(D, E), "msg_mlp.0.bias": 0.1 * g.standard_normal(D),
            "update_mlp.0.weight": r(D, 2 * D), "update_mlp.0.bias": 0.1 * g.standard_normal(D),
            "update_mlp.2.weight": r(D, D), "update_mlp.2.bias": 0.1 * g.standard_normal(D),
            "causal_mlp.0.weight": r(E // 2, E), "causal_mlp.0.bias": 0.1 * g.standard_normal(E // 2),
            "causal_mlp.2.weight": r(1, E // 2), "causal_mlp.2.bias": 0.1 * g.standard_normal(1)}


def _loop_gnn_round(x, p, mask):
    """One message-passing round written element by element (no broadcasting)."""
    F, N, D = x.shape
    relu = lambda v: np.maximum(v, 0)
    out = np.empty_like(x)
    e_all = np.empty((F, N, N, p["edge_mlp.2.weight"].shape[0]))
    for f in range(F):
        for i in range(N):
            agg = np.zeros(D)
            for j in range(N):
                pf = np.concatenate([x[f, i], x[f, j], x[f, i] - x[f, j], x[f, i] * x[f, j]])
                mu, var = pf.mean(), pf.var()
                pf = (pf - mu) / np.sqrt(var + 1e-5) * p["pair_norm.weight"] + p["pair_norm.bias"]
                h = relu(p["edge_mlp.0.weight"] @ pf + p["edge_mlp.0.bias"])
                e = relu(p["edge_mlp.2.weight"] @ h + p["edge_mlp.2.bias"])
                e_all[f, i, j] = e
                w = 1 / (1 + np.exp(-(p["edge_weight.weight"][0] @ e + p["edge_weight.bias"][0]))) * mask[f, i, j]
                agg += relu(p["msg_mlp.0.weight"] @ e + p["msg_mlp.0.bias"]) * w
            u = relu(p["update_mlp.0.weight"] @ np.concatenate([x[f, i], agg]) + p["update_mlp.0.bias"])
            out[f, i] = x[f, i] + p["update_mlp.2.weight"] @ u + p["update_mlp.2.bias"]
    return out, e_all


def test_gnn_matches_loop_restatement():
    D, E, F, N = 6, 4, 2, 3
    p = _gnn_params(D, E, 0)
    x = np.random.default_rng(1).standard_normal((F, N, D))
    alive = np.array([[1, 1, 0], [1, 1, 1]], np.float64)
    mask = alive[:, :, None] * alive[:, None, :]
    x1, e0 = _loop_gnn_round(x, p, mask)
    got, causal = ob.relation_graph_ref(x, alive, p, n_rounds=1)
    np.testing.assert_allclose(got, x1 * alive[..., None], rtol=1e-12, atol=1e-12)
    relu = lambda v: np.maximum(v, 0)
    for f in range(F):
        for i in range(N):
            for j in range(N):
                c = p["causal_mlp.2.weight"][0] @ relu(p["causal_mlp.0.weight"] @ e0[f, i, j] + p["causal_mlp.0.bias"])
                want = 1 / (1 + np.exp(-(c + p["causal_mlp.2.bias"][0]))) * mask[f, i, j]
                assert abs(causal[f, i, j] - want) < 1e-12


def test_gnn_permutation_equivariance_and_dead_slots():
    D, E, F, N = 8, 6, 3, 5
    p = _gnn_params(D, E, 2)
    g = np.random.default_rng(3)
    x = g.standard_normal((F, N, D))
    alive = np.ones((F, N))
    alive[1, 3] = 0.0
    for rounds in (1, 2):
        y, c = ob.relation_graph_ref(x, alive, p, rounds)
        pi = g.permutation(N)
        yp, cp = ob.relation_graph_ref(x[:, pi], alive[:, pi], p, rounds)
        np.testing.assert_allclose(yp, y[:, pi], rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(cp, c[:, pi][:, :, pi], rtol=1e-10, atol=1e-12)
        # a dead slot: zero output, zero causal row / column, and its features do not reach live slots
        assert np.all(y[1, 3] == 0) and np.all(c[1, 3] == 0) and np.all(c[1, :, 3] == 0)
        x2 = x.copy()
        x2[1, 3] += 5.0
        y2, c2 = ob.relation_graph_ref(x2, alive, p, rounds)
        np.testing.assert_allclose(y2, y, rtol=1e-12, atol=1e-12)


def test_gnn_paths_agree_for_two_rounds_and_differ_only_in_causal_for_one():
    D, E, F, N = 8, 6, 2, 6
    p = _gnn_params(D, E, 4)
    x = np.random.default_rng(5).standard_normal((F, N, D))
    a, ca = ob.relation_graph_ref(x, None, p, 2, chunked=False)
    b, cb = ob.relation_graph_ref(x, None, p, 2, chunked=True)
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(ca, cb, rtol=1e-12, atol=1e-12)
    a1, ca1 = ob.relation_graph_ref(x, None, p, 1, chunked=False)
    b1, cb1 = ob.relation_graph_ref(x, None, p, 1, chunked=True)
    np.testing.assert_allclose(a1, b1, rtol=1e-12, atol=1e-12)
    e0, _ = ob.edges_ref(x, p)
    np.testing.assert_allclose(ca1, ob._causal(e0, p), rtol=1e-12)        # all-pairs: from the input nodes
    e1, _ = ob.edges_ref(a1, p)
    np.testing.assert_allclose(cb1, ob._causal(e1, p), rtol=1e-12)        # chunked: from the updated nodes


def test_sinkhorn_marginals_and_optimal_assignment():
    from scipy.optimize import linear_sum_assignment
    g = np.random.default_rng(6)
    F, N = 4, 7
    cost = g.standard_normal((F, N, N))
    la = -cost / 0.05
    for _ in range(20):
        la = la - np.log(np.exp(la - la.max(2, keepdims=True)).sum(2, keepdims=True)) - la.max(2, keepdims=True)
        la = la - np.log(np.exp(la - la.max(1, keepdims=True)).sum(1, keepdims=True)) - la.max(1, keepdims=True)
    np.testing.assert_allclose(np.exp(la).sum(1), 1.0, rtol=1e-10)             # columns exactly normalised
    perm, conf = ob.sinkhorn_ref(cost)
    np.testing.assert_allclose(conf, np.exp(la).max(2), rtol=1e-10)
    # separated costs: the assignment is the optimal one
    for f in range(F):
        pi = g.permutation(N)
        c = 0.05 * g.standard_normal((N, N))
        c[np.arange(N), pi] -= 3.0
        perm, conf = ob.sinkhorn_ref(c[None])
        r, col = linear_sum_assignment(c)
        assert np.array_equal(perm[0], col) and np.array_equal(perm[0], pi)
        assert conf.min() > 0.9


def test_gru_cell_matches_torch():
    g = torch.Generator().manual_seed(7)
    cell = torch.nn.GRUCell(6, 6).double()
    x, h = torch.randn(4, 6, generator=g, dtype=torch.float64), torch.randn(4, 6, generator=g, dtype=torch.float64)
    p = {f"hidden_gru.{k}": v.detach().numpy() for k, v in cell.state_dict().items()}
    np.testing.assert_allclose(ob.gru_cell(x.numpy(), h.numpy(), p), cell(x, h).detach().numpy(), rtol=1e-12)


def test_tracker_identity_frames_and_dead_penalty():
    D = 8
    g = np.random.default_rng(8)
    p = {"match_mlp.0.weight": g.standard_normal((D, 3 * D)) / 5, "match_mlp.0.bias": np.zeros(D),
         "match_mlp.2.weight": g.standard_normal((D // 4, D)) / 3, "match_mlp.2.bias": np.zeros(D // 4),
         "match_mlp.4.weight": g.standard_normal((1, D // 4)), "match_mlp.4.bias": np.zeros(1)}
    s = g.standard_normal((2, 5, D))
    alive = np.ones((2, 5))
    alive[0, 4] = 0.0
    cost = ob.tracker_cost_ref(s, s, alive, alive, p)
    base = ob.tracker_cost_ref(s, s, np.ones_like(alive), np.ones_like(alive), p)
    assert np.allclose(cost[0, 4, :4] - base[0, 4, :4], 1e4) and np.allclose(cost[0, :4, 4] - base[0, :4, 4], 1e4)
    assert np.allclose(cost[0, 4, 4] - base[0, 4, 4], 2e4)


def _loop_mp_round(x, p, mask):
    """One gnn_message_pass round (no pair norm) element by element: (new nodes, edge features)."""
    F, N, D = x.shape
    relu = lambda v: np.maximum(v, 0)
    out = np.empty_like(x)
    e_all = np.empty((F, N, N, p["edge_mlp.2.weight"].shape[0]))
    for f in range(F):
        for i in range(N):
            agg = np.zeros(D)
            for j in range(N):
                pf = np.concatenate([x[f, i], x[f, j], x[f, i] - x[f, j], x[f, i] * x[f, j]])
                e = relu(p["edge_mlp.2.weight"] @ relu(p["edge_mlp.0.weight"] @ pf + p["edge_mlp.0.bias"])
                         + p["edge_mlp.2.bias"])
                e_all[f, i, j] = e
                w = 1 / (1 + np.exp(-(p["edge_weight.weight"][0] @ e + p["edge_weight.bias"][0]))) * mask[f, i, j]
                agg += relu(p["msg_mlp.0.weight"] @ e + p["msg_mlp.0.bias"]) * w
            u = relu(p["update_mlp.0.weight"] @ np.concatenate([x[f, i], agg]) + p["update_mlp.0.bias"])
            out[f, i] = x[f, i] + p["update_mlp.2.weight"] @ u + p["update_mlp.2.bias"]
    return out, e_all


def test_gnn_message_pass_matches_loop_restatement_and_chunk_window():
    """gnn_message_pass_ref against the element-wise loop (2 rounds: edges of the second round come from the
    once-updated nodes), the chunked form's last-chunk window, and zero rounds."""
    D, E, F, N = 6, 4, 2, 5
    p = _gnn_params(D, E, 6)
    x = np.random.default_rng(7).standard_normal((F, N, D))
    alive = np.array([[1, 1, 0, 1, 1], [1, 0.5, 1, 1, 1]], np.float64)   # a fractional alive value too
    mask = alive[:, :, None] * alive[:, None, :]
    x1, _ = _loop_mp_round(x, p, mask)
    x2, e1 = _loop_mp_round(x1, p, mask)
    got, e = ob.gnn_message_pass_ref(x, alive, p, 2)
    np.testing.assert_allclose(got, x2 * alive[..., None], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(e, e1, rtol=1e-12, atol=1e-12)
    gc, ec = ob.gnn_message_pass_ref(x, alive, p, 2, chunk_size=2)
    np.testing.assert_array_equal(gc, got)
    np.testing.assert_allclose(ec, e1[:, :, 4:], rtol=1e-12, atol=1e-12)   # last chunk of targets: [4, 5)
    g0, e0 = ob.gnn_message_pass_ref(x, alive, p, 0)
    assert e0 is None
    np.testing.assert_array_equal(g0, x * alive[..., None])
    # the pair norm is the only difference from RelationGraph: with an identity-like norm removed, the
    # relation graph's edges differ, so a stray LayerNorm in the message pass would be caught above
    rg, _ = ob.relation_graph_ref(x, alive, p, 1, chunked=True)
    mp, _ = ob.gnn_message_pass_ref(x, alive, p, 1)
    assert np.abs(rg - mp).max() > 1e-3


# ---- the tracker's composite functions (slot_tracker.py:74-158, model.py:229-252) -------------------------

def _match_params(D, seed):
    g = np.random.default_rng(seed)
    r = lambda *s: g.standard_normal(s) / np.sqrt(s[-1])
    return {"match_mlp.0.weight": r(D, 3 * D), "match_mlp.0.bias": 0.1 * g.standard_normal(D),
            "match_mlp.2.weight": r(D // 4, D), "match_mlp.2.bias": 0.1 * g.standard_normal(D // 4),
            "match_mlp.4.weight": r(1, D // 4), "match_mlp.4.bias": 0.1 * g.standard_normal(1),
            "hidden_gru.weight_ih": r(3 * D, D), "hidden_gru.weight_hh": r(3 * D, D),
            "hidden_gru.bias_ih": 0.1 * g.standard_normal(3 * D), "hidden_gru.bias_hh": 0.1 * g.standard_normal(3 * D)}


class _TorchTracker(torch.nn.Module):
    """The reference's SlotTracker module tree (match_mlp Sequential, hidden_gru GRUCell) in float64, with its
    forward / reorder_and_update written as the torch ops of slot_tracker.py:74-158 (logsumexp Sinkhorn,
    gather along dim 1): a second implementation, in another library, for the numpy oracle to agree with."""

    def __init__(self, D, p):
        super().__init__()
        self.match_mlp = torch.nn.Sequential(torch.nn.Linear(3 * D, D), torch.nn.ReLU(), torch.nn.Linear(D, D // 4),
                                             torch.nn.ReLU(), torch.nn.Linear(D // 4, 1)).double()
        self.hidden_gru = torch.nn.GRUCell(D, D).double()
        self.load_state_dict({k: torch.from_numpy(np.asarray(v, np.float64)) for k, v in p.items()})

    def cost(self, s_t, s_t1, a_t, a_t1):
        B, N, D = s_t.shape
        a = torch.clamp(s_t, -50, 50)[:, :, None, :].expand(B, N, N, D)
        b = torch.clamp(s_t1, -50, 50)[:, None, :, :].expand(B, N, N, D)
        score = self.match_mlp(torch.cat([a, b, (a - b).abs()], dim=-1)).squeeze(-1)
        score = score - 1e4 * (a_t < 0.5).double()[:, :, None] - 1e4 * (a_t1 < 0.5).double()[:, None, :]
        return -score

    def forward(self, s_t, s_t1, a_t, a_t1):
        la = -torch.clamp(self.cost(s_t, s_t1, a_t, a_t1), -1e4, 1e4) / 0.05
        for _ in range(20):
            la = la - torch.logsumexp(la, dim=2, keepdim=True)
            la = la - torch.logsumexp(la, dim=1, keepdim=True)
        asg = la.exp()
        perm, conf = asg.argmax(dim=2), asg.max(dim=2).values
        matched = (a_t > 0.5).double() * (a_t1 > 0.5).double().gather(1, perm) * (conf > 0.3).double()
        return perm, matched

    def reorder_and_update(self, s_t1, perm, hidden, matched):
        B, N, D = s_t1.shape
        re = s_t1.gather(1, perm.unsqueeze(-1).expand(B, N, D))
        h1 = self.hidden_gru(re.reshape(-1, D), hidden.reshape(-1, D)).reshape(B, N, D)
        return re, matched.unsqueeze(-1) * h1 + (1 - matched).unsqueeze(-1) * re

    def track(self, slots, alive):
        B, T, N, D = slots.shape
        hidden = torch.zeros(B, N, D, dtype=torch.float64)
        tr, al = [slots[:, 0]], [alive[:, 0]]
        for t in range(1, T):
            perm, matched = self(tr[-1], slots[:, t], al[-1], alive[:, t])
            re, hidden = self.reorder_and_update(slots[:, t], perm, hidden, matched)
            tr.append(re)
            al.append(alive[:, t].gather(1, perm))
        return torch.stack(tr, 1), torch.stack(al, 1), hidden


def _loop_cost(s_t, s_t1, a_t, a_t1, p):
    """tracker cost written element by element: one match-MLP evaluation per (i, j)."""
    F, N, D = s_t.shape
    relu = lambda v: np.maximum(v, 0)
    out = np.empty((F, N, N))
    for f in range(F):
        for i in range(N):
            for j in range(N):
                a, b = np.clip(s_t[f, i], -50, 50), np.clip(s_t1[f, j], -50, 50)
                feat = np.concatenate([a, b, np.abs(a - b)])
                h = relu(p["match_mlp.0.weight"] @ feat + p["match_mlp.0.bias"])
                h = relu(p["match_mlp.2.weight"] @ h + p["match_mlp.2.bias"])
                sc = p["match_mlp.4.weight"][0] @ h + p["match_mlp.4.bias"][0]
                sc -= 1e4 * (a_t[f, i] < 0.5) + 1e4 * (a_t1[f, j] < 0.5)
                out[f, i, j] = -sc
    return out


def test_tracker_cost_matches_loop_and_torch_match_mlp():
    """The cost against an element-by-element loop and against nn.Sequential with the same float64 weights: the
    [s_t; s_t1; |s_t - s_t1|] order, the +-50 clamp (inputs beyond it) and both dead-slot penalties."""
    D, F, N = 8, 2, 5
    p = _match_params(D, 11)
    g = np.random.default_rng(12)
    s_t, s_t1 = 3 * g.standard_normal((F, N, D)), 3 * g.standard_normal((F, N, D))
    s_t[0, 1, 2], s_t1[1, 3, 0] = 80.0, -75.0              # clamped to +-50
    a_t, a_t1 = np.ones((F, N)), np.ones((F, N))
    a_t[0, 2], a_t1[0, 4], a_t1[1, 1] = 0.0, 0.3, 0.0       # dead on either side (0.3 < 0.5 is dead)
    got = ob.tracker_cost_ref(s_t, s_t1, a_t, a_t1, p)
    np.testing.assert_allclose(got, _loop_cost(s_t, s_t1, a_t, a_t1, p), rtol=1e-12, atol=1e-9)
    tt = _TorchTracker(D, p)
    want = tt.cost(*(torch.from_numpy(v) for v in (s_t, s_t1, a_t, a_t1))).detach().numpy()
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-9)
    # the order of the three feature blocks matters: the same weights on [s_t1; s_t; |.|] give another cost
    swapped = ob.tracker_cost_ref(s_t1, s_t, a_t1, a_t, p).transpose(0, 2, 1)
    assert np.abs(swapped - got).max() > 1e-3


def test_tracker_forward_and_reorder_match_torch_ops():
    """tracker_forward_ref (perm, matched) and reorder_update_ref (gather by perm, GRUCell carry, unmatched rows
    take the new slot) against the torch ops of slot_tracker.py:122-158, with some slots dead and some rows of
    low confidence (near-tied costs)."""
    D, F, N = 8, 3, 6
    p = _match_params(D, 13)
    g = np.random.default_rng(14)
    s_t = g.standard_normal((F, N, D))
    s_t1 = s_t[:, g.permutation(N)] + 0.3 * g.standard_normal((F, N, D))
    s_t1[2] = s_t1[2, :1] + 1e-3 * g.standard_normal((N, D))   # frame 2: near-identical slots, low confidence
    a_t, a_t1 = np.ones((F, N)), np.ones((F, N))
    a_t[1, 0], a_t1[0, 3] = 0.0, 0.0
    tt = _TorchTracker(D, p)
    T = lambda v: torch.from_numpy(np.asarray(v, np.float64))
    perm_t, matched_t = tt(T(s_t), T(s_t1), T(a_t), T(a_t1))
    perm, matched = ob.tracker_forward_ref(s_t, s_t1, a_t, a_t1, p)
    np.testing.assert_array_equal(perm, perm_t.numpy())
    np.testing.assert_array_equal(matched, matched_t.numpy())
    assert 0 < matched.sum() < matched.size                  # both matched and unmatched rows occur
    hidden = g.standard_normal((F, N, D))
    re_t, h_t = tt.reorder_and_update(T(s_t1), perm_t, T(hidden), matched_t)
    re, h1 = ob.reorder_update_ref(s_t1, perm, hidden, matched, p)
    np.testing.assert_array_equal(re, re_t.numpy())
    np.testing.assert_allclose(h1, h_t.detach().numpy(), rtol=1e-12, atol=1e-12)
    # the gather is along the slot axis: row i of the reordered frame is slot perm[i] of the new frame
    for f in range(F):
        for i in range(N):
            np.testing.assert_array_equal(re[f, i], s_t1[f, perm[f, i]])
            if matched[f, i] == 0:
                np.testing.assert_array_equal(h1[f, i], re[f, i])


def test_track_sequence_matches_torch_loop():
    """The frame loop of model.py:229-252 against the same loop over the torch tracker (float64)."""
    D, B, T, N = 8, 2, 4, 5
    p = _match_params(D, 15)
    g = np.random.default_rng(16)
    slots = g.standard_normal((B, T, N, D))
    for t in range(1, T):
        slots[:, t] = slots[:, t - 1][:, g.permutation(N)] + 0.2 * g.standard_normal((B, N, D))
    alive = (g.random((B, T, N)) > 0.2).astype(np.float64)
    tt = _TorchTracker(D, p)
    tr_t, al_t, h_t = tt.track(torch.from_numpy(slots), torch.from_numpy(alive))
    tr, al, h = ob.track_sequence_ref(slots, alive, p)
    np.testing.assert_allclose(tr, tr_t.detach().numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(al, al_t.numpy())
    np.testing.assert_allclose(h, h_t.detach().numpy(), rtol=1e-12, atol=1e-12)


def _distance_params(D, c=20.0):
    """A match MLP whose score is -c * sum |s_t - s_t1|: layer 0 passes the |diff| block through, layer 2 sums
    groups of four, layer 4 scales by -c.  With it the cost is c * L1 distance, so the assignment is known."""
    W0 = np.zeros((D, 3 * D))
    W0[:, 2 * D:] = np.eye(D)
    W2 = np.zeros((D // 4, D))
    for k in range(D // 4):
        W2[k, 4 * k:4 * k + 4] = 1.0
    g = np.random.default_rng(17)
    r = lambda *s: g.standard_normal(s) / np.sqrt(s[-1])
    return {"match_mlp.0.weight": W0, "match_mlp.0.bias": np.zeros(D), "match_mlp.2.weight": W2,
            "match_mlp.2.bias": np.zeros(D // 4), "match_mlp.4.weight": -c * np.ones((1, D // 4)),
            "match_mlp.4.bias": np.zeros(1), "hidden_gru.weight_ih": r(3 * D, D), "hidden_gru.weight_hh": r(3 * D, D),
            "hidden_gru.bias_ih": np.zeros(3 * D), "hidden_gru.bias_hh": np.zeros(3 * D)}


def test_track_sequence_closed_forms():
    """With the L1-distance match MLP: identical frames give identity permutations and tracked = slots; frames
    that are a known permutation of the previous one recover it (tracked = the first frame every step); a dead
    slot keeps its row and its alive flag, and is never matched.  A swapped feature order or a gather along the
    wrong axis fails these."""
    D, B, T, N = 8, 2, 5, 6
    p = _distance_params(D)
    g = np.random.default_rng(18)
    base = g.standard_normal((B, N, D))
    alive = np.ones((B, T, N))
    # identical frames
    same = np.repeat(base[:, None], T, axis=1)
    tr, al, _ = ob.track_sequence_ref(same, alive, p)
    np.testing.assert_array_equal(tr, same)
    np.testing.assert_array_equal(al, alive)
    for t in range(T - 1):
        perm, matched = ob.tracker_forward_ref(same[:, t], same[:, t + 1], alive[:, t], alive[:, t + 1], p)
        np.testing.assert_array_equal(perm, np.tile(np.arange(N), (B, 1)))
        np.testing.assert_array_equal(matched, np.ones((B, N)))
    # each frame a known permutation of the previous one: tracking undoes it
    frames, pis = [base], []
    for t in range(1, T):
        pi = np.stack([g.permutation(N) for _ in range(B)])
        pis.append(pi)
        frames.append(np.take_along_axis(frames[-1], pi[..., None], axis=1))
    seq = np.stack(frames, 1)
    tr, al, _ = ob.track_sequence_ref(seq, alive, p)
    for t in range(T):
        np.testing.assert_array_equal(tr[:, t], base)
    inv = np.argsort(pis[0], axis=1)
    perm, _ = ob.tracker_forward_ref(seq[:, 0], seq[:, 1], alive[:, 0], alive[:, 1], p)
    np.testing.assert_array_equal(perm, inv)
    # a dead slot (row 2 of batch 0, in every frame) keeps its place and its flag, and is never matched
    dead = alive.copy()
    dead[0, :, 2] = 0.0
    tr, al, h = ob.track_sequence_ref(same, dead, p)
    np.testing.assert_array_equal(al, dead)
    np.testing.assert_array_equal(tr, same)
    perm, matched = ob.tracker_forward_ref(same[:, 0], same[:, 1], dead[:, 0], dead[:, 1], p)
    assert perm[0, 2] == 2 and matched[0, 2] == 0 and matched[0].sum() == N - 1
    np.testing.assert_array_equal(h[0, 2], same[0, -1, 2])   # unmatched rows carry the new slot as hidden state
