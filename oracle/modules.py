"""Oracle: the in-model modules around the hot-path kernels.  TEST INFRASTRUCTURE ONLY.

Numpy float64 restatements, taking parameters as plain arrays (names as in the reference's
state dicts):
  block_scan_ref            hclsm/dynamics/level0_ssm.py:73-103 (softplus/clamp of dt, scan, silu gate)
  simplified_ssm_block_ref  hclsm/dynamics/level0_ssm.py:58-107 (scan in model mode)
  level0_ssm_ref            hclsm/dynamics/level0_ssm.py:159-220
  event_block_ref           hclsm/dynamics/level1_event.py:44-54 (MHA over slots + SwiGLU)
  level1_ref                hclsm/dynamics/level1_event.py:85-133
  event_mask_rule_ref       hclsm/dynamics/event_detector.py:160-170
  hierarchy_forward_ref     hclsm/dynamics/hierarchy_manager.py:120-162 (scatter, Level-2 gate, alive mask)
"""

from __future__ import annotations

import numpy as np

from oracle.events import scatter, slots_attention
from oracle.slot_attention import layer_norm, sigmoid
from oracle.ssm_scan import ssm_scan_ref


def _lin(x, w, b=None):
    y = x @ np.asarray(w, np.float64).T
    return y if b is None else y + b


def softplus(x):
    return np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20))))


def silu(x):
    return x * sigmoid(x)


def block_scan_ref(z, dt_in, A_log, B, C, gate):
    """silu(gate) * clamped scan of z with dt = clip(softplus(dt_in), 1e-3, 1) (level0_ssm.py:73-103)."""
    dt = np.clip(softplus(np.asarray(dt_in, np.float64)), 1e-3, 1.0)
    return ssm_scan_ref(z, dt, A_log, B, C, clamp_mode="model") * silu(np.asarray(gate, np.float64))


def simplified_ssm_block_ref(x, p):
    """p keys: norm.weight, norm.bias, in_proj.weight, gate_proj.weight, dt_proj.weight, dt_proj.bias,
    B_proj.weight, C_proj.weight, A_log, out_proj.weight."""
    x = np.asarray(x, np.float64)
    h = layer_norm(x, p["norm.weight"], p["norm.bias"])
    z = _lin(h, p["in_proj.weight"])
    y = block_scan_ref(z, _lin(z, p["dt_proj.weight"], p["dt_proj.bias"]), p["A_log"], _lin(z, p["B_proj.weight"]),
                       _lin(z, p["C_proj.weight"]), _lin(h, p["gate_proj.weight"]))
    return x + _lin(y, p["out_proj.weight"])


def level0_ssm_ref(obj_states, obj_mask, p, n_blocks):
    """p: state-dict-like mapping with keys global_blocks.{i}.*, object_blocks.{i}.*, condition_proj.weight."""
    s = np.asarray(obj_states, np.float64)
    B, N, T, D = s.shape
    blk = lambda pre, i: {k[len(f"{pre}.{i}."):]: v for k, v in p.items() if k.startswith(f"{pre}.{i}.")}
    if obj_mask is not None:
        m = np.asarray(obj_mask, np.float64)
        n_alive = np.maximum(m.sum(1, keepdims=True), 1.0)
        g = (s * m[:, :, None, None]).sum(1) / n_alive[:, :, None]
    else:
        g = s.mean(1)
    for i in range(n_blocks):
        g = simplified_ssm_block_ref(g, blk("global_blocks", i))
    cond = _lin(g, p["condition_proj.weight"])
    x = (s + cond[:, None]).reshape(B * N, T, D)
    for i in range(n_blocks):
        x = simplified_ssm_block_ref(x, blk("object_blocks", i))
    x = np.clip(np.nan_to_num(x.reshape(B, N, T, D), nan=0.0, posinf=100.0, neginf=-100.0), -100, 100)
    if obj_mask is not None:
        x = x * np.asarray(obj_mask, np.float64)[:, :, None, None]
    return x


def event_block_ref(x, key_pad, p, n_heads):
    """p keys: norm1.*, attn.in_proj_weight, attn.out_proj.weight, norm2.*, ffn.w1/w2/w3.weight."""
    x = np.asarray(x, np.float64)
    P, N, d = x.shape
    dh = d // n_heads
    h = layer_norm(x, p["norm1.weight"], p["norm1.bias"])
    q, k, v = np.split(_lin(h, p["attn.in_proj_weight"]), 3, axis=-1)
    o = slots_attention(*(t.reshape(P, N, n_heads, dh) for t in (q, k, v)), key_pad=key_pad)
    x = x + _lin(o.reshape(P, N, d), p["attn.out_proj.weight"])
    h2 = layer_norm(x, p["norm2.weight"], p["norm2.bias"])
    f = _lin(silu(_lin(h2, p["ffn.w1.weight"])) * _lin(h2, p["ffn.w3.weight"]), p["ffn.w2.weight"])
    return x + f


def level1_ref(event_states, event_pad_mask, obj_mask, p, n_layers, n_heads):
    e = np.asarray(event_states, np.float64)
    B, K, N, D = e.shape
    x = _lin(e.reshape(B * K, N, D), p["proj_in.weight"])
    kp = None
    if obj_mask is not None:
        kp = np.broadcast_to(~(np.asarray(obj_mask) > 0.5)[:, None, :], (B, K, N)).reshape(B * K, N)
    for i in range(n_layers):
        blk = {k[len(f"blocks.{i}."):]: v for k, v in p.items() if k.startswith(f"blocks.{i}.")}
        x = event_block_ref(x, kp, blk, n_heads)
    x = _lin(layer_norm(x, p["norm.weight"], p["norm.bias"]), p["proj_out.weight"]).reshape(B, K, N, D)
    if event_pad_mask is not None:
        x = x * np.asarray(event_pad_mask, np.float64)[:, :, None, None]
    return x


def event_mask_rule_ref(probs, threshold_logit):
    probs = np.asarray(probs, np.float64)
    thr = sigmoid(np.asarray(threshold_logit, np.float64))
    hard = (probs > thr).astype(np.float64)
    mask = hard - probs + probs
    if mask.shape[1] and hard.sum(1).min() == 0:
        mask[:, 0] = 1.0
    return mask


def hierarchy_forward_ref(level0, level1, index, w_l2, w_gate, b_gate=None, level2_context=None, obj_mask=None):
    """HierarchyManager.forward (hierarchy_manager.py:120-162).  level0 (B, T, N, D); level1 (B, K, N, D) padded
    Level-1 rows; index an oracle.events.event_index of the mask; w_l2 = l2_to_l1.weight (D, d_l2);
    w_gate / b_gate = gate_l2_l0.0 (D, 2D) / (D,).
      combined = scatter of the Level-1 rows into level0                         (:143)
      l2 = l2_to_l1(mean over summaries of level2_context), broadcast           (:147-152)
      gate = sigmoid(W_gate [combined; l2] + b_gate)                             (:153-154)
      combined = gate * l2 + (1 - gate) * combined                               (:155)
      out = combined * obj_mask[b, None, n, None]                                (:159-160)"""
    combined = scatter(np.asarray(level0, np.float64), np.asarray(level1, np.float64), index)
    if level2_context is not None:
        ctx = np.asarray(level2_context, np.float64)
        l2 = _lin(ctx.mean(axis=1), w_l2)                                        # (B, D)
        l2b = np.broadcast_to(l2[:, None, None, :], combined.shape)
        gate = sigmoid(_lin(np.concatenate([combined, l2b], axis=-1), w_gate, b_gate))
        combined = gate * l2b + (1.0 - gate) * combined
    if obj_mask is not None:
        combined = combined * np.asarray(obj_mask, np.float64)[:, None, :, None]
    return combined
