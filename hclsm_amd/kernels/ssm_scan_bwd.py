"""Backward of the selective scan on MI355X (libhclsm_amd.so: hclsm_ssm_scan_bwd).

Replaces the reference's PyTorch reverse scan ``_TritonSSMScan.backward``
(hclsm/kernels/ssm_scan_kernel.py:321-377) in raw mode, and the autograd of the clamped
``sequential_ssm_scan`` (:42-86) in model mode.  Gradients come back in the input dtypes
(x, dt, B, C: their I/O dtype; A_log and D: float32), as the reference returns them (:377).
"""

from __future__ import annotations

import torch

from hclsm_amd import _lib
from hclsm_amd.kernels._common import common_float_dtype


def bwd_workspace(batch, T, d_inner, d_state, device) -> torch.Tensor:
    """Workspace of hclsm_ssm_scan_bwd (checkpoints first, then partial sums)."""
    wsb = int(_lib.lib().hclsm_ssm_scan_bwd_workspace(batch, T, d_inner, d_state))
    if wsb < 0:
        _lib.check(wsb, "hclsm_ssm_scan_bwd_workspace")
    return torch.empty(max(wsb, 256), dtype=torch.uint8, device=device)


def scan_backward(x, dt, A_log, B, C, D, gy, mode: int, ws: torch.Tensor | None = None) -> dict:
    """Gradients of sum(gy * y).  ws: a workspace into which hclsm_ssm_scan_fwd_ckpt (or the block form) wrote
    the checkpoints for these same inputs; the backward then starts from them (hclsm_ssm_scan_bwd_ckpt).
    Without it the backward recomputes them (hclsm_ssm_scan_bwd)."""
    batch, T, d_inner = x.shape
    d_state = B.shape[2]
    io = common_float_dtype(x, dt, B, C)
    xc, dtc, Bc, Cc = (t.to(io).contiguous() for t in (x, dt, B, C))
    gyc = gy.to(io).contiguous()
    Ac = A_log.to(torch.float32).contiguous()
    Dc = None if D is None else D.to(torch.float32).contiguous()
    dev = x.device
    gx = torch.empty_like(xc)
    gdt = torch.empty_like(dtc)
    gB = torch.empty_like(Bc)
    gC = torch.empty_like(Cc)
    gA = torch.empty((d_inner, d_state), dtype=torch.float32, device=dev)
    gD = None if D is None else torch.empty((d_inner,), dtype=torch.float32, device=dev)
    L = _lib.lib()
    fn, name = (L.hclsm_ssm_scan_bwd_ckpt, "hclsm_ssm_scan_bwd_ckpt") if ws is not None else \
        (L.hclsm_ssm_scan_bwd, "hclsm_ssm_scan_bwd")
    if ws is None:
        ws = bwd_workspace(batch, T, d_inner, d_state, dev)
    rc = fn(_lib.ptr(xc), _lib.ptr(dtc), _lib.ptr(Ac), _lib.ptr(Bc), _lib.ptr(Cc), _lib.ptr(Dc),
            _lib.ptr(gyc), _lib.ptr(gx), _lib.ptr(gdt), _lib.ptr(gA), _lib.ptr(gB), _lib.ptr(gC),
            _lib.ptr(gD), batch, T, d_inner, d_state, _lib.dtype_code(io), mode, _lib.ptr(ws),
            ws.numel(), _lib.stream_of(xc))
    _lib.check(rc, name)
    out = {"x": gx.to(x.dtype), "dt": gdt.to(dt.dtype), "A_log": gA.to(A_log.dtype),
           "B": gB.to(B.dtype), "C": gC.to(C.dtype)}
    if D is not None:
        out["D"] = gD.to(D.dtype)
    return out
