"""Level-1 event dynamics on MI355X: counterpart of hclsm/dynamics/level1_event.py.

Same module tree and parameter names (``attn`` stays an nn.MultiheadAttention so state dicts
load unchanged).  Without autograd, ``forward`` (padded events, the reference's call) and
``forward_packed`` run the whole stack -- projections, LayerNorms, MHA over the slots with key padding
from the alive mask (:37-52), SwiGLU -- in one hclsm_level1_forward call.  Under autograd the
blocks run as torch ops around the MFMA attention core (``hclsm_amd.kernels.slots_attention``) and
say so with a HipFallbackWarning.
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from hclsm_amd.kernels._common import warn_fallback
from hclsm_amd.kernels.event_attention import slots_attention
from hclsm_amd.kernels.level1_packed import Level1Weights, level1_forward_dense, level1_forward_packed
from hclsm_amd.kernels.sparse_event_attn import EventIndex


class SwiGLUFFN(nn.Module):
    """w2(silu(w1 x) * w3 x) with hidden = expansion * d_model (reference :17-28)."""

    def __init__(self, d_model: int, expansion: int = 4) -> None:
        super().__init__()
        hidden = d_model * expansion
        self.w1 = nn.Linear(d_model, hidden, bias=False)
        self.w3 = nn.Linear(d_model, hidden, bias=False)
        self.w2 = nn.Linear(hidden, d_model, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.w2(F.silu(self.w1(x)) * self.w3(x))


class EventTransformerBlock(nn.Module):
    """Pre-LN block: x + MHA(LN x) over the slot axis, then x + SwiGLU(LN x) (reference :31-54)."""

    def __init__(self, d_model: int, n_heads: int) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(d_model)
        self.attn = nn.MultiheadAttention(d_model, n_heads, batch_first=True, bias=False)
        self.norm2 = nn.LayerNorm(d_model)
        self.ffn = SwiGLUFFN(d_model)

    def forward(self, x: torch.Tensor, key_padding_mask: torch.Tensor | None = None) -> torch.Tensor:
        normed = self.norm1(x)
        P, N, d = normed.shape
        H = self.attn.num_heads
        dh = d // H
        qkv = F.linear(normed, self.attn.in_proj_weight, self.attn.in_proj_bias)
        q, k, v = (t.reshape(P, N, H, dh) for t in qkv.split(d, dim=-1))
        o = slots_attention(q, k, v, key_padding_mask)
        attn_out = F.linear(o.reshape(P, N, d), self.attn.out_proj.weight, self.attn.out_proj.bias)
        x = x + attn_out
        return x + self.ffn(self.norm2(x))


class Level1EventDynamics(nn.Module):
    """Sparse transformer over object states at event timesteps (reference :57-133)."""

    def __init__(self, config, d_slot: int, use_gradient_checkpointing: bool = False) -> None:
        super().__init__()
        self.d_model = config.d_model
        self.d_slot = d_slot
        self.use_gradient_checkpointing = use_gradient_checkpointing
        self.proj_in = nn.Linear(d_slot, config.d_model, bias=False)
        self.proj_out = nn.Linear(config.d_model, d_slot, bias=False)
        self.blocks = nn.ModuleList([EventTransformerBlock(config.d_model, config.n_heads)
                                     for _ in range(config.n_layers)])
        self.norm = nn.LayerNorm(config.d_model)

    def forward(self, event_states: torch.Tensor, event_pad_mask: torch.Tensor | None = None,
                obj_mask: torch.Tensor | None = None) -> torch.Tensor:
        B, K, N, D = event_states.shape
        if not self._needs_grad(event_states):
            # every (b, k) of the padded batch is an event of one hclsm_level1_forward call; the padding
            # mask then zeroes the padded ones (:130-131; a padded event whose keys are all dead stays NaN)
            dtype = self._compute_dtype()
            try:
                W = Level1Weights.from_module(self, dtype)
            except ValueError as e:
                warn_fallback("Level1EventDynamics.forward", f"a module the fused stack does not take ({e})")
            else:
                x = level1_forward_dense(event_states, obj_mask, W, out_dtype=self._out_dtype(event_states, dtype))
                if event_pad_mask is not None:
                    x = x * event_pad_mask[:, :, None, None]
                return x
        else:
            warn_fallback("Level1EventDynamics.forward", "autograd (projections, LayerNorms and SwiGLU as torch "
                                                         "ops around the HIP attention core)")
        x = self.proj_in(event_states.reshape(B * K, N, D))                     # :102-107
        kpm = None
        if obj_mask is not None:                                                 # :110-114
            kpm = (~(obj_mask > 0.5)).unsqueeze(1).expand(B, K, N).reshape(B * K, N)
        for block in self.blocks:                                                # :116-122
            if self.use_gradient_checkpointing and self.training:
                x = torch.utils.checkpoint.checkpoint(block, x, kpm, use_reentrant=False)
            else:
                x = block(x, key_padding_mask=kpm)
        x = self.proj_out(self.norm(x)).reshape(B, K, N, D)                      # :124-128
        if event_pad_mask is not None:                                           # :130-131
            x = x * event_pad_mask[:, :, None, None]
        return x

    @staticmethod
    def _compute_dtype() -> torch.dtype:
        """bf16 GEMM operands under a bf16 autocast, fp32 otherwise."""
        if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16:
            return torch.bfloat16
        return torch.float32

    @staticmethod
    def _out_dtype(x: torch.Tensor, dtype: torch.dtype) -> torch.dtype:
        return x.dtype if x.dtype in (torch.float32, dtype) else torch.float32

    def _needs_grad(self, x: torch.Tensor) -> bool:
        if not torch.is_grad_enabled():
            return False
        return x.requires_grad or any(p.requires_grad for p in self.parameters())

    def forward_packed(self, event_states: torch.Tensor, index: EventIndex,
                       obj_mask: torch.Tensor | None = None) -> torch.Tensor:
        """The same computation on packed events: event_states (capacity, N, d_slot) as gathered by
        gather_packed / gather_events_packed with ``index`` (event e < index.total() in row e);
        returns (capacity, N, d_slot), rows past the live count unspecified.  No host sync.

        Without autograd this is one C call (hclsm_level1_forward, compute in fp32, or bf16 under a
        bf16 autocast).  With autograd it is this module's ops over all capacity rows, so the rows past
        the live count must be finite (gather_events_packed zero-fills them in grad mode)."""
        cap, N, D = event_states.shape
        if not self._needs_grad(event_states):
            dtype = self._compute_dtype()
            W = Level1Weights.from_module(self, dtype)
            return level1_forward_packed(event_states, index, obj_mask, W,
                                         out_dtype=self._out_dtype(event_states, dtype))
        warn_fallback("Level1EventDynamics.forward_packed", "autograd (projections, LayerNorms and SwiGLU as torch "
                                                            "ops around the HIP attention core)")
        x = self.proj_in(event_states)
        kpm = None
        if obj_mask is not None:
            # batch row of each packed event; entries past the live count are clamped to a valid row
            rows = index.rows[:cap].long().clamp(0, index.B - 1)
            kpm = ~(obj_mask[rows] > 0.5)
        for block in self.blocks:
            if self.use_gradient_checkpointing and self.training:
                x = torch.utils.checkpoint.checkpoint(block, x, kpm, use_reentrant=False)
            else:
                x = block(x, key_padding_mask=kpm)
        return self.proj_out(self.norm(x))
