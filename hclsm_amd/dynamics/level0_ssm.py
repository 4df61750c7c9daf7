"""Level-0 SSM on MI355X: counterpart of hclsm/dynamics/level0_ssm.py.

Same module tree and parameter names as the reference (state dicts load unchanged).  The
selective scan -- a Python loop over T in the reference (:95-100) -- runs on the gfx950 kernel with
the reference's clamped ("model") semantics, with softplus / clamp of dt and the silu gate fused into
it (``hclsm_amd.kernels.ssm_block_scan``); the output projection runs as one hclsm_linear launch with the
residual add in its epilogue (:104-107); the input-side projections are torch GEMMs.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from hclsm_amd import _lib
from hclsm_amd.kernels._common import warn_fallback
from hclsm_amd.kernels.ssm_scan_kernel import ssm_block_scan


def _compute_dtype(y: torch.Tensor, weight: torch.Tensor):
    """The dtype the output projection runs in: bf16 / fp16 under a CUDA autocast of that type, else the dtype
    y and the weight share; None where that is not a pair hclsm_linear takes."""
    if torch.is_autocast_enabled("cuda"):
        dt = torch.get_autocast_dtype("cuda")
        return dt if dt in (torch.bfloat16, torch.float16) else None
    return y.dtype if (y.dtype == weight.dtype and y.dtype in (torch.float32, torch.bfloat16, torch.float16)) else None


class _OutProjResidual(torch.autograd.Function):
    """residual + y W^T (level0_ssm.py:104-107) as one hclsm_linear launch: the GEMM adds the fp32 residual in its
    epilogue and writes fp32.  Backward: the two matmuls in torch, in the same compute dtype."""

    @staticmethod
    def forward(ctx, y, weight, residual, cdt):
        K, N = y.shape[-1], weight.shape[0]
        x2 = y.reshape(-1, K).to(cdt).contiguous()
        w = weight.to(cdt).contiguous()
        r2 = residual.reshape(-1, N).contiguous()
        out = torch.empty_like(r2)
        rc = _lib.lib().hclsm_linear(_lib.ptr(x2), K, _lib.dtype_code(cdt), _lib.ptr(w), K, None, _lib.ptr(r2), N,
                                     _lib.ptr(out), N, _lib.F32, None, 0, x2.shape[0], N, K, 0, 0.0, 0, None, None,
                                     1e-5, _lib.dtype_code(cdt), _lib.stream_of(x2))
        _lib.check(rc, "hclsm_linear")
        ctx.save_for_backward(x2, w)
        ctx.shapes = (y.shape, y.dtype, weight.dtype)
        return out.reshape(residual.shape)

    @staticmethod
    def backward(ctx, g):
        x2, w = ctx.saved_tensors
        y_shape, y_dtype, w_dtype = ctx.shapes
        g2 = g.reshape(-1, w.shape[0]).to(w.dtype)
        gy = (g2 @ w).reshape(y_shape).to(y_dtype) if ctx.needs_input_grad[0] else None
        gw = (g2.t() @ x2).to(w_dtype) if ctx.needs_input_grad[1] else None
        return gy, gw, (g if ctx.needs_input_grad[2] else None), None


def out_proj_residual(y: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
    """residual + y weight^T on one hclsm_linear launch where it applies (fp32 residual and weight; K a multiple of 4,
    of 32 for 16-bit operands); otherwise the torch ops, with a HipFallbackWarning."""
    cdt = _compute_dtype(y, weight)
    K = y.shape[-1]
    ok = (cdt is not None and residual.dtype == torch.float32 and weight.dtype == torch.float32 and y.is_cuda
          and residual.is_cuda and residual.shape[-1] == weight.shape[0] and weight.shape[1] == K
          and K % (4 if cdt == torch.float32 else 32) == 0)
    if ok:
        return _OutProjResidual.apply(y, weight, residual, cdt)
    warn_fallback("SimplifiedSSMBlock.out_proj", f"dtypes / shape outside hclsm_linear (y {y.dtype}, weight "
                                                 f"{weight.dtype}, residual {residual.dtype}, K {K})")
    return residual + torch.nn.functional.linear(y, weight)


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
        return out_proj_residual(y, self.out_proj.weight, residual)   # :104-107, one launch


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
