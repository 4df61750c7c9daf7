"""CPU restatements of the reference's PyTorch paths with torch ops, for the CPU baseline of bench.py.
TEST INFRASTRUCTURE ONLY: imported by bench.py's cpu_baseline leg and by tests/ (which check these
against the numpy oracle); never by the product.

    scan_torch            hclsm/kernels/ssm_scan_kernel.py:42-86 (sequential loop; raw or clamped model form)
    slot_forward_torch    hclsm/objects/dynamic_slots.py:98-131, 152-164 (LN, Linear, GRUCell, MLP ops)
    event_attention_torch gather of hierarchy_manager.py:42-77 + per-track causal SDPA over the events
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def scan_torch(x, dt, A_log, B, C, D=None, clamp_mode="raw"):
    """The reference's T loop (ssm_scan_kernel.py:60-86) in fp32; raw mode drops the clamps."""
    x, dt, B, C = (t.float() for t in (x, dt, B, C))
    A = -torch.exp(A_log.float())
    if clamp_mode == "model":
        A = -torch.exp(A_log.float()).clamp(1e-6, 1.0)
        dt = dt.clamp(1e-3, 1.0)
    n, T, d = x.shape
    h = torch.zeros(n, d, A.shape[1])
    ys = []
    for t in range(T):
        arg = dt[:, t, :, None] * A[None]
        if clamp_mode == "model":
            arg = arg.clamp(-20.0, 0.0)
        h = torch.exp(arg) * h + (dt[:, t, :, None] * B[:, t, None, :]) * x[:, t, :, None]
        ys.append((h * C[:, t, None, :]).sum(-1))
    y = torch.stack(ys, 1)
    if D is not None:
        y = y + D.float() * x
    return y


def slot_forward_torch(inputs, slots0, W, n_iter, logit_clamp=None, renorm_eps=None, slot_clamp=None):
    """k, v = LN_in(inputs) W_k^T, W_v^T; n_iter iterations of LN_pre, q, logits (scale d^-0.5, optional
    clamp), softmax over slots, [renorm], attn v, GRUCell, LN-MLP residual, [clamp]; fp32 torch ops."""
    d = slots0.shape[-1]
    x = F.layer_norm(inputs.float(), (inputs.shape[-1],), W["ln_in_w"], W["ln_in_b"])
    k, v = x @ W["w_k"].T, x @ W["w_v"].T
    slots = slots0.float()
    for _ in range(n_iter):
        q = F.layer_norm(slots, (d,), W["ln_pre_w"], W["ln_pre_b"]) @ W["w_q"].T
        logits = torch.bmm(q, k.transpose(1, 2)) * d ** -0.5
        if logit_clamp:
            logits = logits.clamp(-logit_clamp, logit_clamp)
        attn = torch.softmax(logits, dim=1)
        if renorm_eps is not None:
            attn = (attn + renorm_eps) / (attn + renorm_eps).sum(dim=-1, keepdim=True)
        upd = torch.bmm(attn, v)
        B, N, _ = slots.shape
        h = torch._VF.gru_cell(upd.reshape(-1, d), slots.reshape(-1, d), W["w_ih"], W["w_hh"], W["b_ih"], W["b_hh"])
        h = h.reshape(B, N, d)
        m = F.layer_norm(h, (d,), W["ln_mlp_w"], W["ln_mlp_b"])
        slots = h + torch.relu(m @ W["w1"].T + W["b1"]) @ W["w2"].T + W["b2"]
        if slot_clamp:
            slots = slots.clamp(-slot_clamp, slot_clamp)
    return slots


def event_attention_torch(q, k, v, event_mask):
    """Per track: the event timesteps (mask > 0.5, ascending), causal SDPA among them; packed output
    (total events, H, dh) in track order."""
    outs = []
    ev = event_mask > 0.5
    for p in range(q.shape[0]):
        idx = torch.nonzero(ev[p]).flatten()
        if idx.numel() == 0:
            continue
        qs, ks, vs = (t[p, idx].float().transpose(0, 1) for t in (q, k, v))    # (H, L, dh)
        outs.append(F.scaled_dot_product_attention(qs, ks, vs, is_causal=True).transpose(0, 1))
    return torch.cat(outs, 0)
