"""DynamicSlotAttention on MI355X: counterpart of hclsm/objects/dynamic_slots.py.

Same parameters and names as the reference module (:47-82), so its state dict loads unchanged.

* Without autograd (inference, torch.no_grad): the k/v projections and all n_iterations run as
  one call of the fused C entry ``hclsm_slot_attention_forward`` (MFMA GEMMs, fused attention
  core, fused GRU) with the reference's in-model semantics: logits clamped to +-30, MLP hidden
  4*d, slots clamped to +-50.  Compute dtype fp32, or bf16 under a bf16 autocast.  The keys it
  computed are reused for the birth attention.
* With autograd (training): the iteration is torch LayerNorm / Linear / GRUCell around the HIP
  slot-attention core (differentiable, logit clamp included), with a HipFallbackWarning.
Slot initialisation draws from the global RNG as the reference does (:86-96); slot birth
(:180-199) is vectorised without the reference's host synchronisation and Python loop.
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from hclsm_amd.kernels._common import warn_fallback
from hclsm_amd.kernels.slot_attention_kernel import slot_attention_core
from hclsm_amd.kernels.slot_iteration import SlotMode, SlotWeights, forms_kq, slot_attention_forward

_LOGIT_CLAMP = 30.0   # dynamic_slots.py:118
_SLOT_CLAMP = 50.0    # dynamic_slots.py:130


class DynamicSlotAttention(nn.Module):
    def __init__(self, config, d_input: int, use_gradient_checkpointing: bool = False) -> None:
        super().__init__()
        self.d_slot = config.d_slot
        self.n_max_slots = config.n_max_slots
        self.n_iterations = config.n_iterations
        self.existence_threshold = config.existence_threshold
        self.birth_threshold = config.birth_threshold
        self.use_gradient_checkpointing = use_gradient_checkpointing
        d = config.d_slot
        self.slot_mu = nn.Parameter(torch.randn(d) * 0.02)
        self.slot_log_sigma = nn.Parameter(torch.full((d,), -2.0))
        self.project_k = nn.Linear(d_input, d, bias=False)
        self.project_v = nn.Linear(d_input, d, bias=False)
        self.project_q = nn.Linear(d, d, bias=False)
        self.gru = nn.GRUCell(d, d)
        nn.init.orthogonal_(self.gru.weight_ih)
        nn.init.orthogonal_(self.gru.weight_hh)
        nn.init.zeros_(self.gru.bias_ih)
        nn.init.zeros_(self.gru.bias_hh)
        self.norm_slots = nn.LayerNorm(d)
        self.mlp = nn.Sequential(nn.Linear(d, d * 4), nn.ReLU(), nn.Linear(d * 4, d))
        self.norm_input = nn.LayerNorm(d_input)
        self.norm_pre_attn = nn.LayerNorm(d)
        self.existence_head = nn.Sequential(nn.Linear(d, d // 4), nn.ReLU(), nn.Linear(d // 4, 1))
        self.birth_proj = nn.Linear(d_input, d)
        self.scale = d ** -0.5

    def _init_slots(self, batch_size: int, device) -> torch.Tensor:
        sigma = self.slot_log_sigma.exp()
        eps = torch.randn(batch_size, self.n_max_slots, self.d_slot, device=device)
        return self.slot_mu + sigma * eps

    def _iteration_step(self, slots, k, v):
        """Differentiable iteration (dynamic_slots.py:98-131) with the HIP attention core."""
        B = slots.shape[0]
        q = self.project_q(self.norm_pre_attn(slots))
        updates, _ = slot_attention_core(q, k, v, scale=self.scale, logit_clamp=_LOGIT_CLAMP)
        slots = self.gru(updates.reshape(-1, self.d_slot), slots.reshape(-1, self.d_slot))
        slots = slots.reshape(B, self.n_max_slots, self.d_slot)
        slots = slots + self.mlp(self.norm_slots(slots))
        return torch.clamp(slots, min=-_SLOT_CLAMP, max=_SLOT_CLAMP)

    def _needs_grad(self, inputs) -> bool:
        if not torch.is_grad_enabled():
            return False
        return inputs.requires_grad or any(p.requires_grad for p in self.parameters())

    def forward(self, inputs: torch.Tensor, return_attention: bool = False):
        B, M, _ = inputs.shape
        slots = self._init_slots(B, inputs.device)
        use_kq = False
        if self._needs_grad(inputs):
            warn_fallback("DynamicSlotAttention", "autograd (LayerNorm / Linear / GRUCell as torch ops around the "
                                                  "HIP attention core; the fused forward has no backward)")
            x = self.norm_input(inputs)
            k, v = self.project_k(x), self.project_v(x)
            for _ in range(self.n_iterations):
                if self.use_gradient_checkpointing and self.training:
                    slots = torch.utils.checkpoint.checkpoint(self._iteration_step, slots, k, v, use_reentrant=False)
                else:
                    slots = self._iteration_step(slots, k, v)
        else:
            dtype = torch.bfloat16 if (torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16) \
                else torch.float32
            W = SlotWeights.from_module(self, dtype)
            mode = SlotMode(logit_clamp=_LOGIT_CLAMP, renorm_eps=None, slot_clamp=_SLOT_CLAMP)
            # 16-bit fused-core shapes form kq = k W_q instead of k: birth's logits are then LN_pre(slots) kq^T
            use_kq = forms_kq(B, slots.shape[1], inputs.shape[1], inputs.shape[2], W)
            slots, k = slot_attention_forward(inputs.float(), slots.float(), W, self.n_iterations, mode,
                                              scale=self.scale, return_k=not use_kq, return_kq=use_kq)
            slots = slots.to(inputs.dtype)
        alive = torch.sigmoid(self.existence_head(slots).squeeze(-1))              # :167-168
        final_attn = None
        with torch.no_grad():
            q = self.norm_pre_attn(slots)
            if not use_kq:
                q = self.project_q(q)
            k = k.to(q.dtype)
            _, attn = slot_attention_core(q.detach(), k.detach(), k.detach(), scale=self.scale)   # :172-177
            if return_attention:
                final_attn = attn
            residual = (1.0 - attn.sum(dim=1)).abs()                              # :186-188
            max_residual, max_token_idx = residual.max(dim=-1)
            dormant = alive < self.existence_threshold                            # :190
            do_birth = (max_residual > self.birth_threshold) & dormant.any(dim=1)  # :191-196
            first_dormant = dormant.to(torch.int8).argmax(dim=1)
            token = inputs[torch.arange(B, device=inputs.device), max_token_idx]
            born = self.birth_proj(token).to(slots.dtype)
            sel = F.one_hot(first_dormant, self.n_max_slots).bool() & do_birth[:, None]
        slots = torch.where(sel[..., None], born[:, None, :], slots)
        if return_attention:
            return slots, alive, final_attn
        return slots, alive
