"""Oracle: slot attention core and the slot-attention iteration.  TEST INFRASTRUCTURE ONLY.

Core (reference hclsm/kernels/slot_attention_kernel.py):
  logits = Q K^T * scale            (B, N, M)           naive :286, Triton pass 1 :69-86
  attn   = softmax over slots (N)   per token column    naive :287, Triton pass 2 :114-128
           (Triton adds 1e-8 to the denominator, :126 -> ``denom_eps``)
  out    = attn V                   (B, N, D)           naive :288, Triton :131-149

Iteration (reference hclsm/objects/dynamic_slots.py:98-131, DynamicSlotAttention._iteration_step):
  sn      = LayerNorm_pre(slots)                                   :111
  q       = sn W_q^T                                               :112
  logits  = q k^T * scale, optionally clamped to +-logit_clamp     :116-118
  attn    = softmax over slots                                     :119
  attn    = (attn + eps) / sum_tokens(attn + eps)   if renorm_eps  (benchmark config 2's weighted mean)
  updates = attn v                                                 :121
  slots   = GRUCell(updates, slots)                                :123-126 (torch GRUCell equations)
  slots   = slots + MLP(LayerNorm(slots))                          :128 (Linear, ReLU, Linear)
  slots   = clamp(slots, +-slot_clamp)              if slot_clamp  :130
Reference mode: logit_clamp=30, slot_clamp=50, renorm_eps=None, MLP hidden 4*d.
Config-2 mode:  no clamps, renorm_eps=1e-8, MLP hidden 768.

Forward up to the iterations (dynamic_slots.py:149-164): k, v = LN_in(inputs) W_k^T, W_v^T,
then n_iter iterations from the given initial slots (the Gaussian draw of _init_slots :86-96
is the caller's).  dynamic_slots_forward_ref adds the existence head and slot birth (:166-199).
All float64.
"""

from __future__ import annotations

import numpy as np


def layer_norm(x, w=None, b=None, eps=1e-5):
    x = np.asarray(x, np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    y = (x - mu) / np.sqrt(var + eps)
    if w is not None:
        y = y * w
    if b is not None:
        y = y + b
    return y


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def slot_attention_core(Q, K, V, scale=None, denom_eps=0.0, logit_clamp=None):
    """Returns (out (B,N,D), attn (B,N,M)); softmax over the slot axis."""
    Q = np.asarray(Q, np.float64)
    K = np.asarray(K, np.float64)
    V = np.asarray(V, np.float64)
    if scale is None:
        scale = Q.shape[-1] ** -0.5
    logits = np.einsum("bnd,bmd->bnm", Q, K) * scale
    if logit_clamp is not None:
        logits = np.clip(logits, -logit_clamp, logit_clamp)
    mx = logits.max(axis=1, keepdims=True)
    e = np.exp(logits - mx)
    attn = e / (e.sum(axis=1, keepdims=True) + denom_eps)
    return np.einsum("bnm,bmd->bnd", attn, V), attn


def gru_cell(x, h, w_ih, w_hh, b_ih, b_hh):
    """torch.nn.GRUCell: rows of w_* are [r; z; n]."""
    gi = x @ w_ih.T + b_ih
    gh = h @ w_hh.T + b_hh
    H = h.shape[-1]
    r = sigmoid(gi[..., :H] + gh[..., :H])
    z = sigmoid(gi[..., H:2 * H] + gh[..., H:2 * H])
    n = np.tanh(gi[..., 2 * H:] + r * gh[..., 2 * H:])
    return (1 - z) * n + z * h


def slot_iteration(slots, k, v, W, scale=None, logit_clamp=None, renorm_eps=None, slot_clamp=None):
    """One iteration.  W: dict of float arrays with keys
    ln_pre_w, ln_pre_b, w_q, w_ih, w_hh, b_ih, b_hh, ln_mlp_w, ln_mlp_b, w1, b1, w2, b2."""
    slots = np.asarray(slots, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    W = {n: np.asarray(a, np.float64) for n, a in W.items()}
    d = slots.shape[-1]
    if scale is None:
        scale = d ** -0.5
    sn = layer_norm(slots, W["ln_pre_w"], W["ln_pre_b"])
    q = sn @ W["w_q"].T
    logits = np.einsum("bnd,bmd->bnm", q, k) * scale
    if logit_clamp is not None:
        logits = np.clip(logits, -logit_clamp, logit_clamp)
    mx = logits.max(axis=1, keepdims=True)
    e = np.exp(logits - mx)
    attn = e / e.sum(axis=1, keepdims=True)
    if renorm_eps is not None:
        attn = attn + renorm_eps
        attn = attn / attn.sum(axis=-1, keepdims=True)
    updates = np.einsum("bnm,bmd->bnd", attn, v)
    B, N, _ = slots.shape
    h = gru_cell(updates.reshape(-1, d), slots.reshape(-1, d), W["w_ih"], W["w_hh"], W["b_ih"], W["b_hh"]).reshape(B, N, d)
    m = layer_norm(h, W["ln_mlp_w"], W["ln_mlp_b"])
    m = np.maximum(m @ W["w1"].T + W["b1"], 0.0) @ W["w2"].T + W["b2"]
    out = h + m
    if slot_clamp is not None:
        out = np.clip(out, -slot_clamp, slot_clamp)
    return out


def slot_attention_forward(inputs, slots0, W, n_iter, **mode):
    """k/v projections of LN_in(inputs) (dynamic_slots.py:152-154) followed by n_iter iterations.
    Extra W keys: ln_in_w, ln_in_b, w_k, w_v."""
    W64 = {n: np.asarray(a, np.float64) for n, a in W.items()}
    x = layer_norm(inputs, W64["ln_in_w"], W64["ln_in_b"])
    k = x @ W64["w_k"].T
    v = x @ W64["w_v"].T
    s = np.asarray(slots0, np.float64)
    for _ in range(n_iter):
        s = slot_iteration(s, k, v, W64, **mode)
    return s


def dynamic_slots_forward_ref(inputs, slots0, W, n_iter, existence_threshold, birth_threshold, scale=None):
    """DynamicSlotAttention.forward (dynamic_slots.py:149-199) from given initial slots (the _init_slots draw
    is the caller's), reference mode (logits +-30, slots +-50): the iterations, the existence head
    (:167-168) and slot birth (:180-199: the residual |1 - sum over slots of the unclamped softmax| per
    token; for each clip whose largest residual exceeds birth_threshold and that has a dormant slot, alive <
    existence_threshold, the first dormant slot becomes birth_proj(inputs[b, token of the largest residual],
    the first such token on ties).  Extra W keys: e1_w, e1_b, e2_w, e2_b (existence_head.0 / .2), birth_w,
    birth_b.  Returns (slots (B, N, d), alive (B, N))."""
    W64 = {n: np.asarray(a, np.float64) for n, a in W.items()}
    x_in = np.asarray(inputs, np.float64)
    d = W64["w_q"].shape[0]
    scale = d ** -0.5 if scale is None else scale
    s = slot_attention_forward(x_in, slots0, W64, n_iter, scale=scale, logit_clamp=30.0, slot_clamp=50.0)
    h = np.maximum(s @ W64["e1_w"].T + W64["e1_b"], 0.0)
    alive = sigmoid((h @ W64["e2_w"].T + W64["e2_b"])[..., 0])
    k = layer_norm(x_in, W64["ln_in_w"], W64["ln_in_b"]) @ W64["w_k"].T
    q = layer_norm(s, W64["ln_pre_w"], W64["ln_pre_b"]) @ W64["w_q"].T
    _, attn = slot_attention_core(q, k, k, scale=scale)
    residual = np.abs(1.0 - attn.sum(axis=1))                                  # (B, M)
    out = s.copy()
    for b in range(s.shape[0]):
        dormant = np.nonzero(alive[b] < existence_threshold)[0]
        if residual[b].max() > birth_threshold and dormant.size:
            tok = int(np.argmax(residual[b]))
            out[b, dormant[0]] = x_in[b, tok] @ W64["birth_w"].T + W64["birth_b"]
    return out, alive
