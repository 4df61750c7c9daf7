"""Argument checks shared by the hclsm_amd kernel wrappers."""

from __future__ import annotations

import torch


def require_gpu(fn_name: str, *tensors: "torch.Tensor | None") -> torch.device:
    """All tensors must live on one ROCm GPU; there is no CPU path."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                f"hclsm_amd.{fn_name}: tensors must be on a ROCm GPU (got a {t.device} tensor). "
                "hclsm_amd has no CPU implementation; move the inputs to 'cuda'.")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"hclsm_amd.{fn_name}: tensors are on different devices ({dev} and {t.device})")
    if dev is None:
        raise RuntimeError(f"hclsm_amd.{fn_name}: no tensor arguments")
    return dev


def common_float_dtype(*tensors: torch.Tensor) -> torch.dtype:
    """The kernels' I/O element type: shared dtype if all agree, else float32."""
    dts = {t.dtype for t in tensors if t is not None}
    if len(dts) == 1:
        (dt,) = dts
        if dt in (torch.float32, torch.bfloat16, torch.float16):
            return dt
    return torch.float32


class HipFallbackWarning(UserWarning):
    """A call ran the reference's math as torch ops on the GPU instead of an hclsm_amd kernel (autograd through a
    forward-only kernel, or a module structure / shape the kernel does not take)."""


_WARNED: set = set()


def warn_fallback(fn_name: str, reason: str) -> None:
    """Warn (once per function and reason) that fn_name is running torch ops instead of its HIP kernel.  The
    pair is recorded only after the warning was issued, so under ``warnings.simplefilter("error",
    HipFallbackWarning)`` every such call raises."""
    import warnings
    key = (fn_name, reason)
    if key in _WARNED:
        return
    warnings.warn(f"hclsm_amd.{fn_name}: running the reference math as torch ops on the GPU: {reason}",
                  HipFallbackWarning, stacklevel=3)
    _WARNED.add(key)
