"""Hierarchical state management on MI355X -- drop-in for ``hclsm/kernels/hierarchical_state.py``.

Reference names kept (same positional signatures, defaults and return structures):

    hierarchical_state_naive(level0_states, event_scores, event_threshold, gather_fn, level1_fn, level2_fn,
                             scatter_fn)                                                      (:25-67)
    hierarchical_state_fused(... same ...)                                                    (:74-128)
    hierarchical_state_streamed(... same ...)                                                 (:135-186)
    hierarchical_state_fn(... , backend="auto")                                               (:193-221)

Each returns (final_states (B, T, N, D), event_mask (B, T), level1_out (B, K, N, D), level2_out).  The four
callables are the caller's, as in the reference:
    gather_fn(states, mask) -> (event_states, pad_mask, K_max)     (naive form only)
    level1_fn(event_states, pad_mask), level2_fn(event_states, pad_mask)
    scatter_fn(level0_states, level1_out, level2_out, event_mask) -> final_states

event_mask = (event_scores > event_threshold) as float (:55, :96).  The fused and streamed forms gather the
events themselves (:98-114): K_max = max(largest row count, 1) (one host read, as the reference's .item()),
the events of each row in descending score order (the reference's topk(sorted=True); ties, which topk leaves
unordered, by ascending t), rows past a row's count exact zeros.  The gather is ``hclsm_event_gather`` driven by
int32 tables built on the device.  The streamed form runs level1_fn and level2_fn on two side streams of
default priority, each made to wait for the gather first, and the current stream waits for both (:160-172).
"""

from __future__ import annotations

from typing import Callable

import torch

from hclsm_amd import _lib
from hclsm_amd.kernels._common import require_gpu


def _event_mask(event_scores: torch.Tensor, event_threshold: float) -> torch.Tensor:
    return (event_scores > event_threshold).float()


def _gather_by_score(level0_states: torch.Tensor, event_scores: torch.Tensor, event_mask: torch.Tensor):
    """(event_states (B, K, N, D), pad_mask (B, K) bool): each row's events in descending score order."""
    require_gpu("hierarchical_state_fused", level0_states, event_scores)
    B, T = event_scores.shape
    if tuple(level0_states.shape[:2]) != (B, T):
        raise ValueError(f"level0_states must be ({B}, {T}, ...) to match event_scores, "
                         f"got {tuple(level0_states.shape)}")
    dev = level0_states.device
    counts = event_mask.sum(dim=1).to(torch.int32)
    K = max(int(counts.max().item()) if B else 0, 1)                       # :98-99
    ev = event_mask > 0
    key = torch.where(ev, event_scores.float(), torch.full_like(event_scores, float("-inf"), dtype=torch.float32))
    order = torch.sort(key, dim=1, descending=True, stable=True).indices[:, :K]
    indices = order.to(torch.int32).contiguous().reshape(-1)
    offsets = torch.arange(B, dtype=torch.int32, device=dev) * K
    src = level0_states.contiguous()
    out = torch.empty((B, K) + tuple(src.shape[2:]), dtype=src.dtype, device=dev)
    row_bytes = src.element_size()
    for s in src.shape[2:]:
        row_bytes *= s
    rc = _lib.lib().hclsm_event_gather(_lib.ptr(src), _lib.ptr(out), row_bytes, B, T, K, counts.data_ptr(),
                                       offsets.data_ptr(), indices.data_ptr(), _lib.stream_of(src))
    _lib.check(rc, "hclsm_event_gather")
    pad = torch.arange(K, device=dev)[None, :] < counts[:, None]          # :117-118
    return out, pad


def hierarchical_state_naive(level0_states: torch.Tensor, event_scores: torch.Tensor, event_threshold: float,
                             gather_fn: Callable, level1_fn: Callable, level2_fn: Callable, scatter_fn: Callable):
    """Step by step, with the caller's gather (:25-67)."""
    require_gpu("hierarchical_state_naive", level0_states, event_scores)
    event_mask = _event_mask(event_scores, event_threshold)
    event_states, event_pad_mask, _ = gather_fn(level0_states, event_mask)
    level1_out = level1_fn(event_states, event_pad_mask)
    level2_out = level2_fn(event_states, event_pad_mask)
    final_states = scatter_fn(level0_states, level1_out, level2_out, event_mask)
    return final_states, event_mask, level1_out, level2_out


def hierarchical_state_fused(level0_states: torch.Tensor, event_scores: torch.Tensor, event_threshold: float,
                             gather_fn: Callable, level1_fn: Callable, level2_fn: Callable, scatter_fn: Callable):
    """Detection and the score-ordered gather in the call (:74-128); gather_fn is not used, as in the reference."""
    event_mask = _event_mask(event_scores, event_threshold)
    event_states, event_pad_mask = _gather_by_score(level0_states, event_scores, event_mask)
    level1_out = level1_fn(event_states, event_pad_mask)
    level2_out = level2_fn(event_states, event_pad_mask)
    final_states = scatter_fn(level0_states, level1_out, level2_out, event_mask)
    return final_states, event_mask, level1_out, level2_out


def hierarchical_state_streamed(level0_states: torch.Tensor, event_scores: torch.Tensor, event_threshold: float,
                                gather_fn: Callable, level1_fn: Callable, level2_fn: Callable,
                                scatter_fn: Callable):
    """The fused form with level1_fn and level2_fn on two side streams (:135-186)."""
    event_mask = _event_mask(event_scores, event_threshold)
    event_states, event_pad_mask = _gather_by_score(level0_states, event_scores, event_mask)
    main = torch.cuda.current_stream(level0_states.device)
    s1 = torch.cuda.Stream(device=level0_states.device)
    s2 = torch.cuda.Stream(device=level0_states.device)
    s1.wait_stream(main)
    s2.wait_stream(main)
    with torch.cuda.stream(s1):
        level1_out = level1_fn(event_states, event_pad_mask)
    with torch.cuda.stream(s2):
        level2_out = level2_fn(event_states, event_pad_mask)
    main.wait_stream(s1)
    main.wait_stream(s2)
    for t in (event_states, event_pad_mask):
        t.record_stream(s1)
        t.record_stream(s2)
    final_states = scatter_fn(level0_states, level1_out, level2_out, event_mask)
    return final_states, event_mask, level1_out, level2_out


def hierarchical_state_fn(level0_states: torch.Tensor, event_scores: torch.Tensor, event_threshold: float,
                          gather_fn: Callable, level1_fn: Callable, level2_fn: Callable, scatter_fn: Callable,
                          backend: str = "auto"):
    """Dispatch as the reference (:211-221): "naive"; "streamed" (or "auto" on a GPU tensor); else fused."""
    args = (level0_states, event_scores, event_threshold, gather_fn, level1_fn, level2_fn, scatter_fn)
    if backend == "naive":
        return hierarchical_state_naive(*args)
    if backend == "streamed" or (backend == "auto" and level0_states.is_cuda):
        return hierarchical_state_streamed(*args)
    return hierarchical_state_fused(*args)
