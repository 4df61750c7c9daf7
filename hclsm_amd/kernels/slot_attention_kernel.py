"""Slot attention on MI355X -- drop-in for ``hclsm/kernels/slot_attention_kernel.py``.

Reference names kept (same positional signatures, defaults and return types):

    slot_attention_fn(Q, K, V, scale=None, backend="auto") -> (out, attn)     (:324-355)
    naive_slot_attention(Q, K, V, scale=None) -> (out, attn)                 (:265-291)
    compiled_slot_attention(Q, K, V, scale=None) -> (out, attn)              (:308-317)
    fused_slot_attention_triton(Q, K, V, scale=None) -> (out, attn)          (:239-258)

All run ``hclsm_slot_attn_core`` (two MFMA launches: logits + softmax over the slot axis per
(frame, 64-token block), then attn @ V per (frame, 64-column block)).  Semantics per name:
    "auto" / "triton" / "hip" and fused_slot_attention_triton: denominator + 1e-8 (:126)
    "naive" / "compiled" and their functions:                  plain softmax (:287, :303)
Softmax over SLOTS (dim=1): every token's column of attn sums to 1.  Q: (B, N, D),
K, V: (B, M, D); out (B, N, D) in Q.dtype; attn (B, N, M) in Q.dtype.  D must be a multiple of
16 (32 for 16-bit inputs).  Autograd: the backward is the reference's own bmm formulation
(:215-236) in torch on the GPU.
"""

from __future__ import annotations

import torch

from hclsm_amd import _lib
from hclsm_amd.kernels._common import common_float_dtype, require_gpu

_EPS_BACKENDS = ("auto", "triton", "hip")

# The reference exports this flag from this module (:14-20); there is no Triton path here.
TRITON_AVAILABLE = False


_WS_BYTES: dict = {}   # (B, N, M, dtype code) -> hclsm_slot_attn_core_workspace


def _core_raw(Q, K, V, scale, denom_eps, logit_clamp=None, renorm_eps=None, want_attn=True,
              attn_dtype=None):
    B, N, D = Q.shape
    M = K.shape[1]
    io = common_float_dtype(Q, K, V)
    q, k, v = (t.to(io).contiguous() for t in (Q, K, V))
    out = torch.empty((B, N, D), dtype=io, device=Q.device)
    at = attn_dtype or io
    attn = torch.empty((B, N, M), dtype=at, device=Q.device) if want_attn else None
    L = _lib.lib()
    key = (B, N, M, _lib.dtype_code(io))
    wsb = _WS_BYTES.get(key)
    if wsb is None:
        wsb = int(L.hclsm_slot_attn_core_workspace(*key))
        _lib.check(wsb if wsb < 0 else 0, "hclsm_slot_attn_core_workspace")
        if len(_WS_BYTES) > 256:
            _WS_BYTES.clear()
        _WS_BYTES[key] = wsb
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=Q.device)
    rc = L.hclsm_slot_attn_core(
        _lib.ptr(q), D, N * D, _lib.ptr(k), D, M * D, _lib.ptr(v), D, M * D, _lib.ptr(out), D, N * D,
        _lib.ptr(attn), _lib.dtype_code(at), B, N, M, D, float(scale), float(denom_eps),
        float(logit_clamp) if logit_clamp else 0.0, float(renorm_eps) if renorm_eps is not None else -1.0,
        _lib.dtype_code(io), _lib.ptr(ws), ws.numel(), _lib.stream_of(q))
    _lib.check(rc, "hclsm_slot_attn_core")
    return out, attn


class _SlotAttnCore(torch.autograd.Function):
    @staticmethod
    def forward(ctx, Q, K, V, scale, denom_eps, logit_clamp=None):
        out, attn = _core_raw(Q, K, V, scale, denom_eps, logit_clamp=logit_clamp)
        ctx.save_for_backward(Q, K, V, attn)
        ctx.scale = scale
        ctx.logit_clamp = logit_clamp
        return out.to(Q.dtype), attn.to(Q.dtype)

    @staticmethod
    def backward(ctx, grad_out, grad_attn):
        Q, K, V, attn = ctx.saved_tensors
        attn = attn.to(grad_out.dtype if grad_out is not None else Q.dtype)
        d_attn = torch.zeros_like(attn) if grad_out is None else torch.bmm(grad_out, V.transpose(1, 2).contiguous())
        if grad_attn is not None:
            d_attn = d_attn + grad_attn
        sum_da = (attn * d_attn).sum(dim=1, keepdim=True)      # softmax over slots (dim 1)
        d_logits = attn * (d_attn - sum_da) * ctx.scale
        if ctx.logit_clamp:   # clamp passes gradient only inside [-c, c] (dynamic_slots.py:118)
            logits = torch.bmm(Q, K.transpose(1, 2).contiguous()) * ctx.scale
            d_logits = d_logits * (logits.abs() <= ctx.logit_clamp).to(d_logits.dtype)
        d_Q = torch.bmm(d_logits, K)
        d_K = torch.bmm(d_logits.transpose(1, 2).contiguous(), Q)
        d_V = torch.bmm(attn.transpose(1, 2).contiguous(), grad_out) if grad_out is not None else torch.zeros_like(V)
        return d_Q, d_K, d_V, None, None, None


def slot_attention_core(Q, K, V, scale=None, denom_eps=0.0, logit_clamp=None):
    """The core with the in-model options: logits clamped to +-logit_clamp before the softmax over
    slots (dynamic_slots.py:116-119).  Differentiable."""
    _check(Q, K, V)
    if scale is None:
        scale = Q.shape[-1] ** -0.5
    return _SlotAttnCore.apply(Q, K, V, float(scale), float(denom_eps), logit_clamp)


def _check(Q, K, V):
    require_gpu("slot_attention", Q, K, V)
    if Q.dim() != 3 or K.dim() != 3 or V.shape != K.shape or Q.shape[0] != K.shape[0] or Q.shape[2] != K.shape[2]:
        raise ValueError(f"expected Q (B,N,D), K/V (B,M,D); got {tuple(Q.shape)}, {tuple(K.shape)}, {tuple(V.shape)}")


def _run(Q, K, V, scale, denom_eps):
    _check(Q, K, V)
    if scale is None:
        scale = Q.shape[-1] ** -0.5
    if torch.is_grad_enabled() and (Q.requires_grad or K.requires_grad or V.requires_grad):
        return _SlotAttnCore.apply(Q, K, V, float(scale), float(denom_eps))
    out, attn = _core_raw(Q, K, V, float(scale), float(denom_eps))   # nothing to differentiate: no graph node
    return out.to(Q.dtype), attn.to(Q.dtype)


def naive_slot_attention(Q, K, V, scale=None):
    """Softmax over slots, no epsilon (reference :265-291), on the HIP core."""
    return _run(Q, K, V, scale, 0.0)


def compiled_slot_attention(Q, K, V, scale=None):
    """Name kept from :308-317 (torch.compile of the naive math); same semantics as naive."""
    return _run(Q, K, V, scale, 0.0)


def fused_slot_attention_triton(Q, K, V, scale=None):
    """Name kept from :239-258: softmax denominator + 1e-8 as the Triton kernel (:126)."""
    return _run(Q, K, V, scale, 1e-8)


def slot_attention_fn(Q, K, V, scale=None, backend="auto"):
    """Dispatcher with the reference's signature (:324-355)."""
    return _run(Q, K, V, scale, 1e-8 if backend in _EPS_BACKENDS else 0.0)
