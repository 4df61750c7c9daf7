"""The slot-attention iteration on MI355X (reference objects/dynamic_slots.py:98-164).

``slot_attention_iteration`` runs one ``DynamicSlotAttention._iteration_step`` as a short
sequence of libhclsm_amd launches on the current stream:

    LayerNorm_pre(slots) -> q = . W_q^T                  hclsm_layer_norm, hclsm_linear (MFMA)
    logits, softmax over slots, [renorm], attn @ v       hclsm_slot_attn_core (MFMA, 1 WG / frame)
    GRUCell(updates, slots)                              hclsm_gru_cell (6 gate products + blend)
    slots + MLP(LayerNorm(slots)) [clamp]                hclsm_layer_norm, hclsm_linear x2

``slot_attention_forward`` adds the k/v projections of LayerNorm_in(inputs) (one MFMA
linear over the concatenated [W_k; W_v]) and runs n_iter iterations (dynamic_slots.py:149-164).

Slots are carried in fp32 between steps; every MFMA operand is in the compute dtype
(bf16 for the benchmark configuration, fp32 for reference-precision runs).  Semantics
are selected by ``SlotMode``: the reference module's clamps (logits +-30 :118, slots
+-50 :130, MLP hidden 4*d), or BASELINE config 2 (no clamps, +1e-8 renormalised weighted
mean, MLP hidden 768).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from hclsm_amd import _lib
from hclsm_amd.kernels._common import require_gpu


@dataclass(frozen=True)
class SlotMode:
    logit_clamp: float | None = None
    renorm_eps: float | None = None
    slot_clamp: float | None = None


REFERENCE_MODE = SlotMode(logit_clamp=30.0, renorm_eps=None, slot_clamp=50.0)   # dynamic_slots.py:118,130
CONFIG2_MODE = SlotMode(logit_clamp=None, renorm_eps=1e-8, slot_clamp=None)

_WEIGHT_KEYS = ("w_q", "w_ih", "w_hh", "w1", "w2", "w_k", "w_v")
_F32_KEYS = ("ln_pre_w", "ln_pre_b", "b_ih", "b_hh", "ln_mlp_w", "ln_mlp_b", "b1", "b2", "ln_in_w", "ln_in_b")


@dataclass
class SlotWeights:
    """Device copies of the iteration's parameters: matrices in the compute dtype, vectors fp32."""
    dtype: torch.dtype
    d: int
    hidden: int
    t: dict

    @classmethod
    def from_dict(cls, w: dict, dtype=torch.bfloat16, device="cuda") -> "SlotWeights":
        t = {}
        for k, val in w.items():
            if val is None:
                continue
            val = torch.as_tensor(val)
            t[k] = val.to(device=device, dtype=dtype if k in _WEIGHT_KEYS else torch.float32).contiguous()
        if "w_k" in t and "w_v" in t:
            t["w_kv"] = torch.cat([t["w_k"], t["w_v"]], 0).contiguous()
        d = t["w_q"].shape[0]
        return cls(dtype, d, t["w1"].shape[0], t)

    @classmethod
    def from_module(cls, m, dtype=torch.bfloat16) -> "SlotWeights":
        """From a DynamicSlotAttention-shaped module (attribute names of dynamic_slots.py:47-82)."""
        w = dict(ln_pre_w=m.norm_pre_attn.weight, ln_pre_b=m.norm_pre_attn.bias, w_q=m.project_q.weight,
                 w_ih=m.gru.weight_ih, w_hh=m.gru.weight_hh, b_ih=m.gru.bias_ih, b_hh=m.gru.bias_hh,
                 ln_mlp_w=m.norm_slots.weight, ln_mlp_b=m.norm_slots.bias, w1=m.mlp[0].weight, b1=m.mlp[0].bias,
                 w2=m.mlp[2].weight, b2=m.mlp[2].bias, ln_in_w=m.norm_input.weight, ln_in_b=m.norm_input.bias,
                 w_k=m.project_k.weight, w_v=m.project_v.weight)
        return cls.from_dict({k: v.detach() for k, v in w.items()}, dtype, m.project_q.weight.device)


def _ln(x, ldx, M, D, w, b, out_dtype, stream, eps=1e-5):
    y = torch.empty((M, D), dtype=out_dtype, device=x.device)
    rc = _lib.lib().hclsm_layer_norm(_lib.ptr(x), ldx, _lib.ptr(w), _lib.ptr(b), _lib.ptr(y), D, M, D, eps,
                                     _lib.dtype_code(x.dtype), _lib.dtype_code(out_dtype), stream)
    _lib.check(rc, "hclsm_layer_norm")
    return y


def _linear(x, w, bias=None, resid=None, relu=False, clamp=None, out_dtype=None, shadow=False, stream=None):
    M, K = x.shape
    N = w.shape[0]
    out_dtype = out_dtype or x.dtype
    y = torch.empty((M, N), dtype=out_dtype, device=x.device)
    y2 = torch.empty((M, N), dtype=x.dtype, device=x.device) if shadow else None
    rc = _lib.lib().hclsm_linear(_lib.ptr(x), K, _lib.ptr(w), K, _lib.ptr(bias), _lib.ptr(resid),
                                 0 if resid is None else resid.shape[1], _lib.ptr(y), N, _lib.dtype_code(out_dtype),
                                 _lib.ptr(y2), N, M, N, K, int(relu), float(clamp) if clamp else 0.0,
                                 _lib.dtype_code(x.dtype), stream)
    _lib.check(rc, "hclsm_linear")
    return (y, y2) if shadow else y


def _core(q, k, v, B, N, M, d, ldk, kbs, scale, mode, stream):
    out = torch.empty((B * N, d), dtype=q.dtype, device=q.device)
    rc = _lib.lib().hclsm_slot_attn_core(
        _lib.ptr(q), d, N * d, _lib.ptr(k), ldk, kbs, _lib.ptr(v), ldk, kbs, _lib.ptr(out), d, N * d,
        None, _lib.F32, B, N, M, d, float(scale), 0.0,
        float(mode.logit_clamp) if mode.logit_clamp else 0.0,
        float(mode.renorm_eps) if mode.renorm_eps is not None else -1.0, _lib.dtype_code(q.dtype), stream)
    _lib.check(rc, "hclsm_slot_attn_core")
    return out


def _gru(upd, hb, hf, W, stream):
    M, d = hf.shape
    out = torch.empty((M, d), dtype=torch.float32, device=hf.device)
    t = W.t
    rc = _lib.lib().hclsm_gru_cell(_lib.ptr(upd), upd.shape[1], _lib.ptr(hb), d, _lib.ptr(hf), d, _lib.ptr(t["w_ih"]),
                                   _lib.ptr(t["w_hh"]), _lib.ptr(t.get("b_ih")), _lib.ptr(t.get("b_hh")),
                                   _lib.ptr(out), d, None, d, M, d, upd.shape[1], _lib.dtype_code(upd.dtype), stream)
    _lib.check(rc, "hclsm_gru_cell")
    return out


def _iteration(slots_f, slots_b, k, v, B, N, M, W, mode, scale, ldk, kbs, stream):
    d = W.d
    t = W.t
    sn = _ln(slots_f, d, B * N, d, t.get("ln_pre_w"), t.get("ln_pre_b"), W.dtype, stream)
    q = _linear(sn, t["w_q"], stream=stream)
    upd = _core(q, k, v, B, N, M, d, ldk, kbs, scale, mode, stream)
    h = _gru(upd, slots_b, slots_f, W, stream)
    hn = _ln(h, d, B * N, d, t.get("ln_mlp_w"), t.get("ln_mlp_b"), W.dtype, stream)
    m1 = _linear(hn, t["w1"], bias=t.get("b1"), relu=True, stream=stream)
    return _linear(m1, t["w2"], bias=t.get("b2"), resid=h, clamp=mode.slot_clamp, out_dtype=torch.float32,
                   shadow=True, stream=stream)


def slot_attention_iteration(slots: torch.Tensor, k: torch.Tensor, v: torch.Tensor, W: SlotWeights,
                             mode: SlotMode = REFERENCE_MODE, scale: float | None = None) -> torch.Tensor:
    """One iteration.  slots (B, N, d) (any float dtype; carried as fp32), k, v (B, M, d) in
    W.dtype.  Returns the new slots (B, N, d) fp32."""
    require_gpu("slot_attention_iteration", slots, k, v)
    B, N, d = slots.shape
    M = k.shape[1]
    if scale is None:
        scale = d ** -0.5
    sf = slots.reshape(B * N, d).to(torch.float32).contiguous()
    sb = sf.to(W.dtype)
    kc = k.to(W.dtype).contiguous()
    vc = v.to(W.dtype).contiguous()
    out, _ = _iteration(sf, sb, kc, vc, B, N, M, W, mode, scale, d, M * d, _lib.stream_of(sf))
    return out.reshape(B, N, d)


def slot_attention_forward(inputs: torch.Tensor, slots0: torch.Tensor, W: SlotWeights, n_iter: int,
                           mode: SlotMode = REFERENCE_MODE, scale: float | None = None) -> torch.Tensor:
    """k, v = LN_in(inputs) W_k^T, W_v^T (one MFMA linear over [W_k; W_v]), then n_iter iterations
    from slots0.  inputs (B, M, d_in), slots0 (B, N, d).  Returns slots (B, N, d) fp32."""
    require_gpu("slot_attention_forward", inputs, slots0)
    B, M, d_in = inputs.shape
    N, d = slots0.shape[1], W.d
    if scale is None:
        scale = d ** -0.5
    st = _lib.stream_of(inputs)
    t = W.t
    x = inputs.reshape(B * M, d_in).contiguous()
    xn = _ln(x, d_in, B * M, d_in, t.get("ln_in_w"), t.get("ln_in_b"), W.dtype, st)
    kv = _linear(xn, t["w_kv"], stream=st)                      # (B*M, 2d): k | v
    k = kv
    v = kv[:, d:]
    sf = slots0.reshape(B * N, d).to(torch.float32).contiguous()
    sb = sf.to(W.dtype)
    for _ in range(n_iter):
        sf, sb = _iteration(sf, sb, k, v, B, N, M, W, mode, scale, 2 * d, M * 2 * d, st)
    return sf.reshape(B, N, d)
