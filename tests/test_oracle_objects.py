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
