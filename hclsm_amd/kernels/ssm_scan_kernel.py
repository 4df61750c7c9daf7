"""Selective SSM scan on MI355X -- drop-in for ``hclsm/kernels/ssm_scan_kernel.py``.

Same public names, positional signatures, defaults and return types as the
reference module:

    ssm_scan_fn(x, dt, A_log, B, C, backend="auto") -> y          (ssm_scan_kernel.py:394-421)
    sequential_ssm_scan(x, dt, A_log, B, C) -> y                  (:42-86)
    parallel_ssm_scan_pytorch(x, dt, A_log, B, C) -> y            (:168-218)
    fused_ssm_scan_triton(x, dt, A_log, B, C) -> y                (:379-387)

Every name runs the hand-written gfx950 kernel of libhclsm_amd.so; the reference's
backends differ only in semantics, which map to the kernel's clamp mode:

    backend / function                      mode    reference path it reproduces
    "auto", "triton", "hip", "parallel"     raw     Triton kernel / Blelloch scan (no clamps)
    "sequential", any unknown string        model   sequential_ssm_scan (clamps at :63,68,77)

(The reference's "auto" on a GPU tensor picks Triton, i.e. raw semantics; unknown
backend strings fall through to the sequential path, i.e. model semantics.)

Keyword-only extensions, all defaulting to reference behaviour: ``D`` (skip term
y += D*x), ``clamp_mode`` ("raw"/"model", overrides the backend's mode) and
``return_h_final`` (also return the final state (batch, d_inner, d_state) fp32, as the
Triton kernel stores at :289-290).

Inputs must be on a ROCm GPU; there is no CPU implementation.  Output dtype is
x.dtype (:86, :319).  Autograd: gradients for x, dt, A_log, B, C (and D) come from
the HIP reverse-scan kernel (replacing ``_TritonSSMScan.backward``, :321-377).
"""

from __future__ import annotations

import torch

from hclsm_amd import _lib
from hclsm_amd.kernels._common import common_float_dtype, require_gpu

_RAW_BACKENDS = ("auto", "triton", "hip", "parallel")


def _mode_code(clamp_mode: str) -> int:
    if clamp_mode == "raw":
        return _lib.SCAN_RAW
    if clamp_mode == "model":
        return _lib.SCAN_MODEL
    raise ValueError(f"clamp_mode must be 'raw' or 'model', got {clamp_mode!r}")


def _check_shapes(x, dt, A_log, B, C, D):
    if x.dim() != 3:
        raise ValueError(f"x must be (batch, T, d_inner), got shape {tuple(x.shape)}")
    batch, T, d_inner = x.shape
    if dt.shape != x.shape:
        raise ValueError(f"dt shape {tuple(dt.shape)} != x shape {tuple(x.shape)}")
    if B.dim() != 3 or B.shape[:2] != (batch, T):
        raise ValueError(f"B must be (batch, T, d_state), got {tuple(B.shape)}")
    d_state = B.shape[2]
    if C.shape != B.shape:
        raise ValueError(f"C shape {tuple(C.shape)} != B shape {tuple(B.shape)}")
    if A_log.shape != (d_inner, d_state):
        raise ValueError(f"A_log must be (d_inner, d_state)=({d_inner}, {d_state}), got {tuple(A_log.shape)}")
    if D is not None and D.shape != (d_inner,):
        raise ValueError(f"D must be (d_inner,)=({d_inner},), got {tuple(D.shape)}")
    return batch, T, d_inner, d_state


def _ckpt_workspace(batch, T, d_inner, d_state, io, device):
    """The backward's workspace for the checkpointing forward (bf16 I/O, d_state 16), else None."""
    if io != torch.bfloat16 or d_state != 16:
        return None
    from hclsm_amd.kernels.ssm_scan_bwd import bwd_workspace
    return bwd_workspace(batch, T, d_inner, d_state, device)


def _scan_forward(x, dt, A_log, B, C, D, mode: int, want_h: bool, for_grad: bool = False):
    """Launch hclsm_ssm_scan_fwd; returns (y in x.dtype, h_final or None, checkpointed backward workspace or
    None).  With for_grad, bf16 inputs with d_state 16 go through hclsm_ssm_scan_fwd_ckpt, which also leaves
    the backward's chunk checkpoints in the returned workspace."""
    batch, T, d_inner, d_state = _check_shapes(x, dt, A_log, B, C, D)
    io = common_float_dtype(x, dt, B, C)
    xc = x.to(io).contiguous()
    dtc = dt.to(io).contiguous()
    Bc = B.to(io).contiguous()
    Cc = C.to(io).contiguous()
    Ac = A_log.to(torch.float32).contiguous()
    Dc = None if D is None else D.to(torch.float32).contiguous()
    y = torch.empty((batch, T, d_inner), dtype=io, device=x.device)
    h = torch.empty((batch, d_inner, d_state), dtype=torch.float32, device=x.device) if want_h else None
    ws = _ckpt_workspace(batch, T, d_inner, d_state, io, x.device) if (for_grad and batch * T * d_inner > 0) else None
    if ws is not None:
        code = _lib.lib().hclsm_ssm_scan_fwd_ckpt(
            _lib.ptr(xc), _lib.ptr(dtc), _lib.ptr(Ac), _lib.ptr(Bc), _lib.ptr(Cc), _lib.ptr(Dc),
            _lib.ptr(y), _lib.ptr(h), batch, T, d_inner, d_state,
            _lib.dtype_code(io), mode, _lib.ptr(ws), ws.numel(), _lib.stream_of(x))
        if code == _lib.ERR_UNSUPPORTED:   # layouts the checkpointing kernel does not take: the plain pair
            ws = None
        else:
            _lib.check(code, "hclsm_ssm_scan_fwd_ckpt")
    if ws is None:
        code = _lib.lib().hclsm_ssm_scan_fwd(
            _lib.ptr(xc), _lib.ptr(dtc), _lib.ptr(Ac), _lib.ptr(Bc), _lib.ptr(Cc), _lib.ptr(Dc),
            _lib.ptr(y), _lib.ptr(h), batch, T, d_inner, d_state,
            _lib.dtype_code(io), mode, _lib.stream_of(x))
        _lib.check(code, "hclsm_ssm_scan_fwd")
    if y.dtype != x.dtype:
        y = y.to(x.dtype)
    return y, h, ws


class _HipSSMScan(torch.autograd.Function):
    """Autograd wrapper: HIP forward scan, HIP reverse-scan backward."""

    @staticmethod
    def forward(ctx, x, dt, A_log, B, C, D, mode, want_h):
        y, h, ws = _scan_forward(x, dt, A_log, B, C, D, mode, want_h, for_grad=any(ctx.needs_input_grad[:6]))
        ctx.save_for_backward(x, dt, A_log, B, C, D)
        ctx.mode = mode
        ctx.ws = ws   # the backward workspace holding the forward's checkpoints (or None)
        if h is not None:
            ctx.mark_non_differentiable(h)
            return y, h
        return y

    @staticmethod
    def backward(ctx, gy, *unused):
        from hclsm_amd.kernels.ssm_scan_bwd import scan_backward
        x, dt, A_log, B, C, D = ctx.saved_tensors
        grads = scan_backward(x, dt, A_log, B, C, D, gy, ctx.mode, ws=ctx.ws)
        return (grads["x"], grads["dt"], grads["A_log"], grads["B"], grads["C"],
                grads.get("D"), None, None)


def fused_ssm_scan_hip(x, dt, A_log, B, C, *, D=None, clamp_mode="raw", return_h_final=False):
    """The HIP scan with explicit semantics (see module docstring)."""
    require_gpu("ssm_scan", x, dt, A_log, B, C, D)
    mode = _mode_code(clamp_mode)
    out = _HipSSMScan.apply(x, dt, A_log, B, C, D, mode, bool(return_h_final))
    return out


def fused_ssm_scan_triton(x, dt, A_log, B, C, *, D=None, return_h_final=False):
    """Name kept from ssm_scan_kernel.py:379-387; raw semantics on the HIP kernel."""
    return fused_ssm_scan_hip(x, dt, A_log, B, C, D=D, clamp_mode="raw", return_h_final=return_h_final)


def sequential_ssm_scan(x, dt, A_log, B, C, *, D=None, return_h_final=False):
    """Clamped (model) semantics of ssm_scan_kernel.py:42-86, on the HIP kernel."""
    return fused_ssm_scan_hip(x, dt, A_log, B, C, D=D, clamp_mode="model", return_h_final=return_h_final)


def parallel_ssm_scan_pytorch(x, dt, A_log, B, C, *, D=None, return_h_final=False):
    """Unclamped (raw) semantics of ssm_scan_kernel.py:168-218, on the HIP kernel."""
    return fused_ssm_scan_hip(x, dt, A_log, B, C, D=D, clamp_mode="raw", return_h_final=return_h_final)


def ssm_scan_fn(x, dt, A_log, B, C, backend: str = "auto", *, D=None, clamp_mode=None,
                return_h_final=False):
    """Dispatcher with the reference's signature (ssm_scan_kernel.py:394-421).

    Args:
        x:  (batch, T, d_inner); dt: (batch, T, d_inner); A_log: (d_inner, d_state);
        B, C: (batch, T, d_state).
        backend: "auto" | "triton" | "hip" | "parallel" (raw) or "sequential" (model);
            any other string behaves like "sequential", as in the reference.
    Returns:
        y (batch, T, d_inner) in x.dtype [, h_final (batch, d_inner, d_state) fp32].
    """
    if clamp_mode is None:
        clamp_mode = "raw" if backend in _RAW_BACKENDS else "model"
    return fused_ssm_scan_hip(x, dt, A_log, B, C, D=D, clamp_mode=clamp_mode,
                              return_h_final=return_h_final)


def _block_forward(z, dt_in, A_log, B, C, gate, want_pre: bool, for_grad: bool = False):
    """Launch hclsm_ssm_block_scan_fwd (with for_grad, the checkpointing form where it applies); returns
    (y, y_pre or None, checkpointed backward workspace or None)."""
    batch, T, d_inner, d_state = _check_shapes(z, dt_in, A_log, B, C, None)
    if gate.shape != z.shape:
        raise ValueError(f"gate shape {tuple(gate.shape)} != z shape {tuple(z.shape)}")
    io = common_float_dtype(z, dt_in, B, C, gate)
    zc, dc, Bc, Cc, gc = (t.to(io).contiguous() for t in (z, dt_in, B, C, gate))
    Ac = A_log.to(torch.float32).contiguous()
    y = torch.empty((batch, T, d_inner), dtype=io, device=z.device)
    y_pre = torch.empty_like(y) if want_pre else None
    ws = _ckpt_workspace(batch, T, d_inner, d_state, io, z.device) if (for_grad and batch * T * d_inner > 0) else None
    if ws is not None:
        code = _lib.lib().hclsm_ssm_block_scan_fwd_ckpt(
            _lib.ptr(zc), _lib.ptr(dc), _lib.ptr(Ac), _lib.ptr(Bc), _lib.ptr(Cc), _lib.ptr(gc), _lib.ptr(y),
            _lib.ptr(y_pre), None, batch, T, d_inner, d_state, _lib.dtype_code(io), _lib.ptr(ws), ws.numel(),
            _lib.stream_of(zc))
        if code == _lib.ERR_UNSUPPORTED:
            ws = None
        else:
            _lib.check(code, "hclsm_ssm_block_scan_fwd_ckpt")
    if ws is None:
        code = _lib.lib().hclsm_ssm_block_scan_fwd(
            _lib.ptr(zc), _lib.ptr(dc), _lib.ptr(Ac), _lib.ptr(Bc), _lib.ptr(Cc), _lib.ptr(gc), _lib.ptr(y),
            _lib.ptr(y_pre), None, batch, T, d_inner, d_state, _lib.dtype_code(io), _lib.stream_of(zc))
        _lib.check(code, "hclsm_ssm_block_scan_fwd")
    return y, y_pre, ws


class _HipSSMBlockScan(torch.autograd.Function):
    """Fused block scan forward on HIP; backward = HIP reverse scan in block mode (dt recomputed as
    clamp(softplus(dt_in)) in fp32 exactly as the forward kernel does, gradient returned with respect to
    dt_in through the clamp -- closed interval, as torch's clamp -- and softplus) plus the silu chain rule."""

    @staticmethod
    def forward(ctx, z, dt_in, A_log, B, C, gate):
        need = any(ctx.needs_input_grad)
        y, y_pre, ws = _block_forward(z, dt_in, A_log, B, C, gate, need, for_grad=need)
        if need:
            ctx.save_for_backward(z, dt_in, A_log, B, C, gate, y_pre)
            ctx.ws = ws
        return y

    @staticmethod
    def backward(ctx, g):
        from hclsm_amd.kernels.ssm_scan_bwd import scan_backward
        z, dt_in, A_log, B, C, gate, y_pre = ctx.saved_tensors
        gf, gatef = g.float(), gate.float()
        sg = torch.sigmoid(gatef)
        g_y = gf * gatef * sg
        g_gate = gf * y_pre.float() * sg * (1.0 + gatef * (1.0 - sg))
        grads = scan_backward(z, dt_in.to(y_pre.dtype), A_log, B, C, None, g_y.to(y_pre.dtype), _lib.SCAN_BLOCK,
                              ws=ctx.ws)
        return (grads["x"].to(z.dtype), grads["dt"].to(dt_in.dtype), grads["A_log"], grads["B"].to(B.dtype),
                grads["C"].to(C.dtype), g_gate.to(gate.dtype))


def ssm_block_scan(z, dt_in, A_log, B, C, gate):
    """silu(gate) * clamped-scan(z, clamp(softplus(dt_in), 1e-3, 1), A_log, B, C): the scan of
    SimplifiedSSMBlock (level0_ssm.py:72-103) with its elementwise epilogues in the kernel.
    Output dtype: the common I/O dtype of the inputs.  Differentiable."""
    require_gpu("ssm_block_scan", z, dt_in, A_log, B, C, gate)
    return _HipSSMBlockScan.apply(z, dt_in, A_log, B, C, gate)
