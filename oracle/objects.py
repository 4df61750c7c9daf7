"""Oracle: the object-layer step between slot attention and Level-0.  TEST INFRASTRUCTURE ONLY.

Numpy float64 restatements taking parameters as plain arrays (names as in the reference's state dicts):

  relation_graph_ref   hclsm/objects/relation_graph.py:68-193 (RelationGraph.forward: both the all-pairs
                       path for N <= 32, :171-188, and the chunked path for N > 32, :150-170, whose
                       order of edge recomputation differs)
  edges_ref            :68-92 (pair features [o_i; o_j; o_i - o_j; o_i * o_j], LayerNorm, edge MLP, weight)
  sinkhorn_ref         hclsm/objects/slot_tracker.py:15-43 (log-domain row / column normalisation)
  tracker_cost_ref     :77-110 (match MLP over [s_t; s_t1; |s_t - s_t1|], dead-slot penalties)
  tracker_forward_ref  :112-138 (perm, matched)
  reorder_update_ref   :140-158 (gather by perm, GRUCell carry, unmatched rows take the new slot)
  track_sequence_ref   the frame loop of hclsm/model.py:229-252 (tracked slots and alive masks)
  gnn_message_pass_ref hclsm/kernels/gnn_message_pass.py:38-100 and :168-243 (no pair norm, no causal head;
                       edge features of the last round, or of its last target chunk)
"""

from __future__ import annotations

import numpy as np

from oracle.slot_attention import layer_norm, sigmoid


def _f(x):
    return np.asarray(x, np.float64)


def _lin(x, p, name):
    y = x @ _f(p[name + ".weight"]).T
    b = p.get(name + ".bias")
    return y if b is None else y + _f(b)


def _relu(x):
    return np.maximum(x, 0.0)


def pair_features(a, b):
    """[a_i; b_j; a_i - b_j; a_i * b_j] for all (i, j): (..., N, N, 4D)."""
    ai = a[..., :, None, :]
    bj = b[..., None, :, :]
    ai, bj = np.broadcast_arrays(ai, bj)
    return np.concatenate([ai, bj, ai - bj, ai * bj], axis=-1)


def edges_ref(nodes, p):
    """edge features (F, N, N, E) and sigmoid edge weights (F, N, N) before masking (:68-92)."""
    x = _f(nodes)
    pf = layer_norm(pair_features(x, x), _f(p["pair_norm.weight"]), _f(p["pair_norm.bias"]))
    h = _relu(_lin(pf, p, "edge_mlp.0"))
    e = _relu(_lin(h, p, "edge_mlp.2"))
    w = sigmoid(_lin(e, p, "edge_weight")[..., 0])
    return e, w


def _messages(e, w, p):
    return (_relu(_lin(e, p, "msg_mlp.0")) * w[..., None]).sum(axis=-2)      # sum over j


def _update(x, agg, p):
    u = _relu(_lin(np.concatenate([x, agg], axis=-1), p, "update_mlp.0"))
    return x + _lin(u, p, "update_mlp.2")


def _causal(e, p):
    return sigmoid(_lin(_relu(_lin(e, p, "causal_mlp.0")), p, "causal_mlp.2")[..., 0])


def relation_graph_ref(nodes, alive, p, n_rounds, chunked=None):
    """RelationGraph.forward -> (nodes (F, N, D), causal (F, N, N)).  chunked=None picks the reference's
    rule (N > 32, :149).  Chunked path: every round recomputes the edges from the current nodes, causal
    edges come from the final nodes.  All-pairs path: edges from the input nodes, recomputed after each
    round only when n_rounds > 1, causal edges from the last computed edges."""
    x = _f(nodes)
    F, N, D = x.shape
    if chunked is None:
        chunked = N > 32
    mask = np.ones((F, N, N)) if alive is None else _f(alive)[:, :, None] * _f(alive)[:, None, :]
    if chunked:
        for _ in range(n_rounds):
            e, w = edges_ref(x, p)
            x = _update(x, _messages(e, w * mask, p), p)
        e, _ = edges_ref(x, p)
        causal = _causal(e, p) * mask
    else:
        e, w = edges_ref(x, p)
        w = w * mask
        for _ in range(n_rounds):
            x = _update(x, _messages(e, w, p), p)
            if n_rounds > 1:
                e, w = edges_ref(x, p)
                w = w * mask
        causal = _causal(e, p) * mask
    if alive is not None:
        x = x * _f(alive)[..., None]
    return x, causal


def sinkhorn_ref(cost, n_iters=20, temperature=0.05):
    """(perm (F, N) int, confidence (F, N)) of the Sinkhorn-normalised exp(-cost / temperature)."""
    la = -_f(cost) / max(temperature, 1e-6)
    for _ in range(n_iters):
        m = la.max(axis=2, keepdims=True)
        la = la - (m + np.log(np.exp(la - m).sum(axis=2, keepdims=True)))
        m = la.max(axis=1, keepdims=True)
        la = la - (m + np.log(np.exp(la - m).sum(axis=1, keepdims=True)))
    a = np.exp(la)
    return a.argmax(axis=2), a.max(axis=2)


def tracker_cost_ref(s_t, s_t1, alive_t, alive_t1, p):
    """(F, N, N) matching cost, lower = better (:77-110)."""
    a = np.clip(_f(s_t), -50, 50)
    b = np.clip(_f(s_t1), -50, 50)
    ai, bj = np.broadcast_arrays(a[:, :, None, :], b[:, None, :, :])
    feat = np.concatenate([ai, bj, np.abs(ai - bj)], axis=-1)
    h = _relu(_lin(feat, p, "match_mlp.0"))
    h = _relu(_lin(h, p, "match_mlp.2"))
    score = _lin(h, p, "match_mlp.4")[..., 0]
    score = score - 1e4 * (_f(alive_t) < 0.5)[:, :, None] - 1e4 * (_f(alive_t1) < 0.5)[:, None, :]
    return -score


def tracker_forward_ref(s_t, s_t1, alive_t, alive_t1, p):
    cost = np.clip(tracker_cost_ref(s_t, s_t1, alive_t, alive_t1, p), -1e4, 1e4)
    perm, conf = sinkhorn_ref(cost, 20, 0.05)
    at = (_f(alive_t) > 0.5).astype(np.float64)
    at1 = (_f(alive_t1) > 0.5).astype(np.float64)
    matched = at * np.take_along_axis(at1, perm, axis=1) * (conf > 0.3)
    return perm, matched


def gru_cell(x, h, p, name="hidden_gru"):
    gi = x @ _f(p[name + ".weight_ih"]).T + _f(p[name + ".bias_ih"])
    gh = h @ _f(p[name + ".weight_hh"]).T + _f(p[name + ".bias_hh"])
    H = h.shape[-1]
    r = sigmoid(gi[..., :H] + gh[..., :H])
    z = sigmoid(gi[..., H:2 * H] + gh[..., H:2 * H])
    n = np.tanh(gi[..., 2 * H:] + r * gh[..., 2 * H:])
    return (1 - z) * n + z * h


def reorder_update_ref(s_t1, perm, hidden_t, matched, p):
    re = np.take_along_axis(_f(s_t1), perm[..., None], axis=1)
    h1 = gru_cell(re, _f(hidden_t), p)
    m = _f(matched)[..., None]
    return re, m * h1 + (1 - m) * re


def track_sequence_ref(slots, alive, p):
    """The tracking loop of model.py:229-252 for slots (B, T, N, D), alive (B, T, N): returns tracked
    slots (B, T, N, D), reordered alive (B, T, N) and the final hidden state."""
    slots, alive = _f(slots), _f(alive)
    B, T, N, D = slots.shape
    hidden = np.zeros((B, N, D))
    tracked, al = [slots[:, 0]], [alive[:, 0]]
    for t in range(1, T):
        perm, matched = tracker_forward_ref(tracked[-1], slots[:, t], al[-1], alive[:, t], p)
        re, hidden = reorder_update_ref(slots[:, t], perm, hidden, matched, p)
        tracked.append(re)
        al.append(np.take_along_axis(alive[:, t], perm, axis=1))
    return np.stack(tracked, 1), np.stack(al, 1), hidden


def gnn_message_pass_ref(nodes, alive, p, n_rounds, chunk_size=None):
    """naive_gnn_message_pass (gnn_message_pass.py:38-100) -> (nodes (F, N, D), edge features of the last round
    (F, N, N, E), or None for no rounds).  With chunk_size, the edge features of the last chunk of targets
    (F, N, C, E), as chunked_gnn_message_pass keeps them (:225-227); the nodes are the same.  p: the
    parameters edge_mlp.0 / .2, edge_weight, msg_mlp.0, update_mlp.0 / .2 (.weight / .bias)."""
    x = _f(nodes)
    F, N, D = x.shape
    mask = np.ones((F, N, N)) if alive is None else _f(alive)[:, :, None] * _f(alive)[:, None, :]
    e = None
    for _ in range(n_rounds):
        pf = pair_features(x, x)
        e = _relu(_lin(_relu(_lin(pf, p, "edge_mlp.0")), p, "edge_mlp.2"))
        w = sigmoid(_lin(e, p, "edge_weight")[..., 0]) * mask
        x = _update(x, _messages(e, w, p), p)
    if alive is not None:
        x = x * _f(alive)[:, :, None]
    if e is not None and chunk_size is not None:
        e = e[:, :, ((N - 1) // chunk_size) * chunk_size:]
    return x, e
