"""Level-0 SSM on MI355X: counterpart of hclsm/dynamics/level0_ssm.py.

Same module tree and parameter names as the reference (state dicts load unchanged).  The
selective scan -- a Python loop over T in the reference (:95-100) -- runs on the gfx950 kernel with
the reference's clamped ("model") semantics, with softplus / clamp of dt and the silu gate fused into
it (``hclsm_amd.kernels.ssm_block_scan``); the projections are torch GEMMs.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from hclsm_amd.kernels.ssm_scan_kernel import ssm_block_scan


class SimplifiedSSMBlock(nn.Module):
    """Selective SSM block (reference level0_ssm.py:30-107)."""

    def __init__(self, d_model: int, d_state: int, expand: int = 2) -> None:
        super().__init__()
        self.d_model = d_model
        self.d_state = d_state
        d_inner = d_model * expand
        self.in_proj = nn.Linear(d_model, d_inner, bias=False)
        self.gate_proj = nn.Linear(d_model, d_inner, bias=False)
        self.dt_proj = nn.Linear(d_inner, d_inner, bias=True)
        self.B_proj = nn.Linear(d_inner, d_state, bias=False)
        self.C_proj = nn.Linear(d_inner, d_state, bias=False)
        self.A_log = nn.Parameter(-torch.rand(d_inner, d_state) * 0.5)     # :52
        self.out_proj = nn.Linear(d_inner, d_model, bias=False)
        self.norm = nn.LayerNorm(d_model)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        residual = x
        x = self.norm(x)
        z = self.in_proj(x)                                                 # :72
        gate_in = self.gate_proj(x)                                         # :73 (silu in the kernel)
        dt_in = self.dt_proj(z)                                             # :76 (softplus, clamp in the kernel)
        B_param = self.B_proj(z)
        C_param = self.C_proj(z)
        # clamped scan (:82-101, A = -clamp(exp(A_log), 1e-6, 1), fp32 state) times silu(gate) (:103)
        y = ssm_block_scan(z, dt_in, self.A_log, B_param, C_param, gate_in)
        return residual + self.out_proj(y.to(x.dtype))


class Level0SSM(nn.Module):
    """Per-object SSM tracks with a global conditioning track (reference level0_ssm.py:126-220)."""

    def __init__(self, config, d_slot: int, use_gradient_checkpointing: bool = False) -> None:
        super().__init__()
        self.d_slot = d_slot
        self.use_gradient_checkpointing = use_gradient_checkpointing
        self.object_blocks = nn.ModuleList([SimplifiedSSMBlock(d_slot, config.d_state, config.expand_ratio)
                                            for _ in range(config.n_blocks)])
        self.global_blocks = nn.ModuleList([SimplifiedSSMBlock(d_slot, config.d_state, config.expand_ratio)
                                            for _ in range(config.n_blocks)])
        self.condition_proj = nn.Linear(d_slot, d_slot, bias=False)

    def _run(self, block, x):
        if self.use_gradient_checkpointing and self.training:
            return torch.utils.checkpoint.checkpoint(block, x, use_reentrant=False)
        return block(x)

    def forward(self, obj_states: torch.Tensor, obj_mask: torch.Tensor | None = None) -> torch.Tensor:
        B, N, T, D = obj_states.shape
        if obj_mask is not None:                                            # :176-181
            n_alive = obj_mask.sum(dim=1, keepdim=True).clamp(min=1.0)
            global_in = (obj_states * obj_mask[:, :, None, None]).sum(dim=1) / n_alive[:, :, None]
        else:
            global_in = obj_states.mean(dim=1)
        g = global_in
        for block in self.global_blocks:                                    # :184-191
            g = self._run(block, g)
        cond = self.condition_proj(g)                                       # :194
        x = obj_states.reshape(B * N, T, D) + cond.unsqueeze(1).expand(B, N, T, D).reshape(B * N, T, D)
        for block in self.object_blocks:                                    # :202-208
            x = self._run(block, x)
        x = x.reshape(B, N, T, D)
        x = torch.nan_to_num(x, nan=0.0, posinf=100.0, neginf=-100.0)       # :213-214
        x = torch.clamp(x, min=-100.0, max=100.0)
        if obj_mask is not None:                                            # :217-218
            x = x * obj_mask[:, :, None, None]
        return x
