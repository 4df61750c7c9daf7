"""Sparse event attention plumbing on MI355X -- drop-in for ``hclsm/kernels/sparse_event_attn.py``.

Reference names kept (same positional signatures, defaults and return types):

    naive_sparse_event_attention(states, event_mask, attn_fn, max_events=None)   (:35-86)
    sparse_event_attention(states, event_mask, attn_fn, max_events=None)         (:153-188)
    sparse_event_attn_fn(states, event_mask, attn_fn, max_events=None, backend="auto")  (:242-263)
    _vectorized_gather(states, event_mask, max_events)                            (:93-131)
    _vectorized_scatter(output, updated_events, event_indices, event_pad_mask)    (:134-150)

Event index construction, gathers and scatters run on libhclsm_amd.so (bit-exact byte
moves driven by int32 counts / offsets / ascending indices).  ``attn_fn`` is the caller's
callable on the padded (B*K, N, D) batch, exactly as in the reference.

Semantics:
  * "naive" uses the reference's ``nonzero`` rule (mask != 0, :65); the vectorised path
    and HierarchyManager use mask > 0.5 (:124, hierarchy_manager.py:61).
  * ``max_events`` defaults to int(max row sum of the mask) as at :56 / :173; K = max(it, 1).
  * Events past K in a row are dropped, earliest-first order kept (the reference's naive
    path keeps idx[:K] in ascending order; its topk path breaks ties arbitrarily).
  * Padded rows are exact zeros (the reference multiplies by the pad mask, which turns
    inf/NaN source rows into NaN; here padding never reads the source).

Packed, sync-free API (new): ``build_event_index`` / ``gather_packed`` / ``scatter_packed``
work on device-side int32 tables and never read a size back to the host.
"""

from __future__ import annotations

from typing import Callable

import torch

from hclsm_amd import _lib
from hclsm_amd.kernels._common import require_gpu


class EventIndex:
    """Device-side event tables of a (B, T) mask (all int32, built without host sync):

        counts  (B,)     events per row
        offsets (B+1,)   exclusive prefix sum; offsets[B] = total
        indices (B*T,)   capacity; the first `total` entries are event timesteps, ascending per row
        rows    (B*T,)   capacity; row of each packed event
        slot_of (B, T)   rank of t among row b's events, -1 otherwise
        stats   (2,)     {total, max count}

    Built by build_event_index, the six tables live in one allocation; launches take raw
    pointers into it (``ptr``) and tensor views are made only when a caller asks for one."""

    _NAMES = ("stats", "counts", "offsets", "indices", "rows", "slot_of")

    def __init__(self, B: int, T: int, counts=None, offsets=None, indices=None, rows=None, slot_of=None,
                 stats=None):
        self.B, self.T = B, T
        self._t = dict(counts=counts, offsets=offsets, indices=indices, rows=rows, slot_of=slot_of, stats=stats)
        self._buf = None
        self._off: dict = {}

    _LAYOUTS: dict = {}

    @classmethod
    def allocate(cls, B: int, T: int, device) -> "EventIndex":
        lay = cls._LAYOUTS.get((B, T))
        if lay is None:
            cap = max(B * T, 1)
            sizes = dict(stats=2, counts=B, offsets=B + 1, indices=cap, rows=cap, slot_of=B * T)
            off, o = {}, 0
            for n in cls._NAMES:
                off[n] = (o, sizes[n])
                o += sizes[n]
            if len(cls._LAYOUTS) > 256:
                cls._LAYOUTS.clear()
            lay = cls._LAYOUTS[(B, T)] = (off, o)
        idx = cls(B, T)
        idx._off = lay[0]            # shared, read-only
        idx._buf = torch.empty(lay[1], dtype=torch.int32, device=device)
        idx._base = idx._buf.data_ptr()
        return idx

    def ptr(self, name: str):
        """Device address of a table (None if absent)."""
        if self._buf is not None:
            return self._base + 4 * self._off[name][0]
        t = self._t[name]
        return None if t is None else t.data_ptr()

    def _get(self, name: str):
        t = self._t[name]
        if t is None and self._buf is not None:
            o, n = self._off[name]
            t = self._buf[o:o + n]
            if name == "slot_of":
                t = t.view(self.B, self.T)
            self._t[name] = t
        return t

    counts = property(lambda self: self._get("counts"))
    offsets = property(lambda self: self._get("offsets"))
    indices = property(lambda self: self._get("indices"))
    rows = property(lambda self: self._get("rows"))
    slot_of = property(lambda self: self._get("slot_of"))
    stats = property(lambda self: self._get("stats"))

    def total(self) -> int:
        """Number of events (reads one int32 back to the host)."""
        return int(self.stats[0].item())

    def kmax(self) -> int:
        return int(self.stats[1].item())


def _mask_code(m: torch.Tensor):
    if m.dtype == torch.float32:
        return m, _lib.F32
    if m.dtype == torch.bfloat16:
        return m, _lib.BF16
    if m.dtype == torch.float16:
        return m, _lib.F16
    if m.dtype in (torch.bool, torch.uint8):
        return m.view(torch.uint8) if m.dtype == torch.bool else m, _lib.U8
    return m.to(torch.float32), _lib.F32


def build_event_index(event_mask: torch.Tensor, rule: str = "gt_half") -> EventIndex:
    """Counts, int32 offsets and ascending indices of a (B, T) event mask, on the GPU."""
    require_gpu("build_event_index", event_mask)
    if event_mask.dim() != 2:
        raise ValueError(f"event_mask must be (B, T), got {tuple(event_mask.shape)}")
    rule_code = {"gt_half": _lib.EVENT_GT_HALF, "nonzero": _lib.EVENT_NONZERO}[rule]
    m, code = _mask_code(event_mask.detach().contiguous())
    B, T = m.shape
    idx = EventIndex.allocate(B, T, m.device)
    p = idx.ptr
    rc = _lib.lib().hclsm_event_index(m.data_ptr(), code, B, T, rule_code, p("counts"), p("offsets"), p("indices"),
                                      p("rows"), p("slot_of"), p("stats"), _lib.stream_of(m))
    _lib.check(rc, "hclsm_event_index")
    return idx


def _check_grid(fn: str, name: str, t: torch.Tensor, idx: EventIndex) -> None:
    """A (B, T, ...) tensor must match the (B, T) of the event index it is used with."""
    if t.dim() < 2 or tuple(t.shape[:2]) != (idx.B, idx.T):
        raise ValueError(f"{fn}: {name} must be ({idx.B}, {idx.T}, ...) to match the event index, "
                         f"got {tuple(t.shape)}")


def _check_rows(fn: str, a_name: str, a_row, b_name: str, b_row) -> None:
    if tuple(a_row) != tuple(b_row):
        raise ValueError(f"{fn}: the rows of {a_name} {tuple(a_row)} and {b_name} {tuple(b_row)} differ")


def _check_packed_rows(fn: str, packed: torch.Tensor, idx: EventIndex) -> None:
    """Packed rows are read at offsets[b] + slot_of[b, t] < total: a tensor with fewer than B*T rows
    must hold at least total rows (one host read of the device-side total, only in that case)."""
    if packed.dim() < 1:
        raise ValueError(f"{fn}: packed must be (rows, ...), got a 0-d tensor")
    if packed.shape[0] < idx.B * idx.T and packed.shape[0] < idx.total():
        raise ValueError(f"{fn}: packed has {packed.shape[0]} rows but the event index holds {idx.total()} events")


def _row_bytes(t: torch.Tensor) -> int:
    n = 1
    for s in t.shape[2:]:
        n *= s
    return n * t.element_size()


def _gather_padded_raw(states: torch.Tensor, idx: EventIndex, K: int) -> torch.Tensor:
    src = states.contiguous()
    out = torch.empty((src.shape[0], K) + tuple(src.shape[2:]), dtype=src.dtype, device=src.device)
    rc = _lib.lib().hclsm_event_gather(_lib.ptr(src), _lib.ptr(out), _row_bytes(src), idx.B, idx.T, K,
                                       idx.ptr("counts"), idx.ptr("offsets"), idx.ptr("indices"), _lib.stream_of(src))
    _lib.check(rc, "hclsm_event_gather")
    return out


def _scatter_padded_raw(base, updates, idx: EventIndex, K: int, like: torch.Tensor) -> torch.Tensor:
    b = None if base is None else base.contiguous()
    u = None if updates is None else updates.contiguous()
    out = torch.empty((idx.B, idx.T) + tuple(like.shape[2:]), dtype=like.dtype, device=like.device)
    rc = _lib.lib().hclsm_event_scatter(_lib.ptr(b), _lib.ptr(u), _lib.ptr(out), _row_bytes(out), idx.B, idx.T, K,
                                        idx.ptr("slot_of"), _lib.stream_of(out))
    _lib.check(rc, "hclsm_event_scatter")
    return out


class _GatherPadded(torch.autograd.Function):
    @staticmethod
    def forward(ctx, states, idx, K):
        ctx.idx, ctx.K = idx, K
        ctx.like = torch.empty((0, 0) + tuple(states.shape[2:]), dtype=states.dtype, device=states.device)
        return _gather_padded_raw(states, idx, K)

    @staticmethod
    def backward(ctx, g):
        # d states[b, t] = g[b, slot_of[b, t]] for event rows with slot < K, else 0
        return _scatter_padded_raw(None, g, ctx.idx, ctx.K, ctx.like), None, None


class _ScatterPadded(torch.autograd.Function):
    @staticmethod
    def forward(ctx, base, updates, idx, K):
        ctx.idx, ctx.K = idx, K
        if updates.dtype != base.dtype:
            updates = updates.to(base.dtype)
        return _scatter_padded_raw(base, updates, idx, K, base)

    @staticmethod
    def backward(ctx, g):
        g = g.contiguous()
        g_base = _scatter_padded_raw(g, None, ctx.idx, ctx.K, g)       # zero at replaced rows
        g_upd = _gather_padded_raw(g, ctx.idx, ctx.K)                  # zero at padded slots
        return g_base, g_upd, None, None


def gather_events_padded(states: torch.Tensor, idx: EventIndex, K: int) -> torch.Tensor:
    """(B, T, ...) -> (B, K, ...) event rows, ascending, zero rows past each row's count."""
    require_gpu("gather_events_padded", states)
    _check_grid("gather_events_padded", "states", states, idx)
    if int(K) < 0:
        raise ValueError(f"gather_events_padded: K must be >= 0, got {K}")
    return _GatherPadded.apply(states, idx, int(K))


def scatter_events_padded(base: torch.Tensor, updates: torch.Tensor, idx: EventIndex) -> torch.Tensor:
    """out = base with out[b, t] = updates[b, slot_of[b,t]] for event rows whose slot < K."""
    require_gpu("scatter_events_padded", base, updates)
    _check_grid("scatter_events_padded", "base", base, idx)
    if updates.dim() != base.dim() or updates.shape[0] != idx.B:
        raise ValueError(f"scatter_events_padded: updates must be ({idx.B}, K) + {tuple(base.shape[2:])}, "
                         f"got {tuple(updates.shape)}")
    _check_rows("scatter_events_padded", "updates", updates.shape[2:], "base", base.shape[2:])
    return _ScatterPadded.apply(base, updates, idx, int(updates.shape[1]))


def pad_mask_from_index(idx: EventIndex, K: int, dtype=torch.float32) -> torch.Tensor:
    ar = torch.arange(K, device=idx.counts.device, dtype=torch.int32)
    return (ar[None, :] < idx.counts[:, None]).to(dtype)


def gather_packed(src: torch.Tensor, idx: EventIndex, capacity: int | None = None,
                  zero_fill: bool = False) -> torch.Tensor:
    """(B, T, ...) -> (capacity, ...) packed event rows (first idx.total() valid); no host sync.
    Rows past the live count are left uninitialised, or zero with ``zero_fill``."""
    require_gpu("gather_packed", src)
    _check_grid("gather_packed", "src", src, idx)
    s = src.contiguous()
    cap = idx.B * idx.T if capacity is None else int(capacity)
    if cap < 0:
        raise ValueError(f"gather_packed: capacity must be >= 0, got {cap}")
    alloc = torch.zeros if zero_fill else torch.empty
    out = alloc((cap,) + tuple(s.shape[2:]), dtype=s.dtype, device=s.device)
    rc = _lib.lib().hclsm_event_gather_packed(_lib.ptr(s), _lib.ptr(out), _row_bytes(s), idx.B, idx.T, cap,
                                              idx.ptr("rows"), idx.ptr("indices"), idx.ptr("stats"),
                                              _lib.stream_of(s))
    _lib.check(rc, "hclsm_event_gather_packed")
    return out


def scatter_packed(base: torch.Tensor | None, packed: torch.Tensor | None, idx: EventIndex,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """out[b, t] = packed[offsets[b] + slot_of[b, t]] at events, base[b, t] elsewhere
    (either one None reads as zeros)."""
    require_gpu("scatter_packed", base, packed)
    if base is None and packed is None:
        raise ValueError("scatter_packed: base and packed are both None")
    p = None if packed is None else packed.contiguous()
    b = None if base is None else base.contiguous()
    like = p if p is not None else b
    if b is not None:
        _check_grid("scatter_packed", "base", b, idx)
    if p is not None:
        _check_packed_rows("scatter_packed", p, idx)
        if b is not None:
            _check_rows("scatter_packed", "packed", p.shape[1:], "base", b.shape[2:])
    if b is not None and p is not None and b.dtype != p.dtype:
        raise TypeError(f"scatter_packed: base and packed must share a dtype, got {b.dtype} and {p.dtype}")
    if out is None:
        rest = tuple(p.shape[1:]) if p is not None else tuple(b.shape[2:])
        out = torch.empty((idx.B, idx.T) + rest, dtype=like.dtype, device=like.device)
    else:
        require_gpu("scatter_packed", out, like)
        _check_grid("scatter_packed", "out", out, idx)
        _check_rows("scatter_packed", "out", out.shape[2:], "packed" if p is not None else "base",
                    p.shape[1:] if p is not None else b.shape[2:])
        if out.dtype != like.dtype or not out.is_contiguous():
            raise ValueError("scatter_packed: out must be contiguous and typed like its inputs")
    rb = out.element_size()
    for s in out.shape[2:]:
        rb *= s
    rc = _lib.lib().hclsm_event_scatter_packed(_lib.ptr(b), _lib.ptr(p), _lib.ptr(out), rb, idx.B, idx.T,
                                               idx.ptr("offsets"), idx.ptr("slot_of"), _lib.stream_of(like))
    _lib.check(rc, "hclsm_event_scatter_packed")
    return out


class _GatherPacked(torch.autograd.Function):
    @staticmethod
    def forward(ctx, states, idx, zero_fill):
        ctx.idx = idx
        ctx.like = torch.empty((0, 0) + tuple(states.shape[2:]), dtype=states.dtype, device=states.device)
        return gather_packed(states, idx, zero_fill=zero_fill)

    @staticmethod
    def backward(ctx, g):
        # d states[b, t] = g[offsets[b] + slot_of[b, t]] at events, 0 elsewhere
        return scatter_packed(None, g.contiguous(), ctx.idx), None, None


class _ScatterPacked(torch.autograd.Function):
    @staticmethod
    def forward(ctx, base, packed, idx):
        ctx.idx = idx
        if packed.dtype != base.dtype:
            packed = packed.to(base.dtype)
        return scatter_packed(base, packed, idx)

    @staticmethod
    def backward(ctx, g):
        g = g.contiguous()
        g_base = scatter_packed(g, None, ctx.idx)           # zero at replaced rows
        g_packed = gather_packed(g, ctx.idx, zero_fill=True)
        return g_base, g_packed, None


def gather_events_packed(states: torch.Tensor, idx: EventIndex) -> torch.Tensor:
    """Differentiable packed gather: (B, T, ...) -> (B*T, ...) with event e < idx.total() in row e
    (rows ascending per batch row, batch rows in order); no host sync.  In grad mode the rows after the live
    count are zero (torch ops over all capacity rows then stay finite, and so do their weight gradients);
    otherwise they are unspecified: the C entry points read the live rows only, and every row op and
    per-event attention keeps a later row to itself."""
    require_gpu("gather_events_packed", states)
    _check_grid("gather_events_packed", "states", states, idx)
    return _GatherPacked.apply(states, idx, torch.is_grad_enabled())


def scatter_events_packed(base: torch.Tensor, packed: torch.Tensor, idx: EventIndex) -> torch.Tensor:
    """Differentiable packed scatter: base with out[b, t] = packed[offsets[b] + slot_of[b, t]] at
    events; no host sync."""
    require_gpu("scatter_events_packed", base, packed)
    _check_grid("scatter_events_packed", "base", base, idx)
    _check_packed_rows("scatter_events_packed", packed, idx)
    _check_rows("scatter_events_packed", "packed", packed.shape[1:], "base", base.shape[2:])
    return _ScatterPacked.apply(base, packed, idx)


# ---------------------------------------------------------------------------
# reference-named API
# ---------------------------------------------------------------------------

def _max_events_default(event_mask: torch.Tensor) -> int:
    # sparse_event_attn.py:56 / :173 -- int() of the largest row sum (one host read)
    return int(event_mask.float().sum(dim=1).max().item()) if event_mask.numel() else 0


def _run(states, event_mask, attn_fn, max_events, rule):
    require_gpu("sparse_event_attention", states, event_mask)
    B, T, N, D = states.shape
    if max_events is None:
        max_events = _max_events_default(event_mask)
    K = max(int(max_events), 1)
    idx = build_event_index(event_mask, rule)
    ev = gather_events_padded(states, idx, K)                    # (B, K, N, D)
    upd = attn_fn(ev.reshape(B * K, N, D)).reshape(B, K, N, D)
    return scatter_events_padded(states, upd, idx)


def naive_sparse_event_attention(states: torch.Tensor, event_mask: torch.Tensor, attn_fn: Callable,
                                 max_events: int | None = None) -> torch.Tensor:
    """Gather events -> attn_fn -> scatter back (reference :35-86; rule mask != 0)."""
    return _run(states, event_mask, attn_fn, max_events, "nonzero")


def sparse_event_attention(states: torch.Tensor, event_mask: torch.Tensor, attn_fn: Callable,
                           max_events: int | None = None) -> torch.Tensor:
    """Vectorised variant (reference :153-188; rule mask > 0.5)."""
    return _run(states, event_mask, attn_fn, max_events, "gt_half")


def sparse_event_attn_fn(states: torch.Tensor, event_mask: torch.Tensor, attn_fn: Callable,
                         max_events: int | None = None, backend: str = "auto") -> torch.Tensor:
    """Dispatcher (reference :242-263): "naive" -> nonzero rule, anything else -> > 0.5 rule."""
    if backend == "naive":
        return naive_sparse_event_attention(states, event_mask, attn_fn, max_events)
    return sparse_event_attention(states, event_mask, attn_fn, max_events)


def _vectorized_gather(states: torch.Tensor, event_mask: torch.Tensor, max_events: int):
    """Reference :93-131: returns (event_states (B,K,N,D), pad_mask (B,K) bool, indices (B,K) long).
    Index entries past a row's count are 0 (the reference leaves them tie-dependent)."""
    idx = build_event_index(event_mask, "gt_half")
    K = int(max_events)
    ev = gather_events_padded(states, idx, K)
    pad = pad_mask_from_index(idx, K, torch.bool)
    t_idx = gather_events_padded(torch.arange(idx.T, device=states.device, dtype=torch.int32)
                                 .expand(idx.B, idx.T).contiguous().unsqueeze(-1), idx, K).squeeze(-1).long()
    return ev, pad, t_idx


def _vectorized_scatter(output: torch.Tensor, updated_events: torch.Tensor, event_indices: torch.Tensor,
                        event_pad_mask: torch.Tensor) -> torch.Tensor:
    """Reference :134-150: writes updated_events[b, k] to output[b, event_indices[b, k]] where the
    pad mask is set (in place on ``output``, which is also returned).  Any index order works:
    the (B, T) slot table is built from the given indices, then one scatter kernel runs."""
    require_gpu("_vectorized_scatter", output, updated_events)
    B, T = output.shape[:2]
    K = updated_events.shape[1]
    valid = event_pad_mask.bool()
    slot_of = torch.full((B, T), -1, dtype=torch.int32, device=output.device)
    ks = torch.arange(K, dtype=torch.int32, device=output.device).expand(B, K)
    tgt = torch.where(valid, event_indices.long(), torch.full_like(event_indices.long(), T))
    slot_pad = torch.cat([slot_of, slot_of[:, :1]], dim=1)            # column T absorbs invalid writes
    slot_pad.scatter_(1, tgt, torch.where(valid, ks, torch.full_like(ks, -1)))
    slot_of = slot_pad[:, :T].contiguous()
    out = output.contiguous()
    upd = updated_events.to(out.dtype).contiguous()
    rc = _lib.lib().hclsm_event_scatter(_lib.ptr(out), _lib.ptr(upd), _lib.ptr(out), _row_bytes(out), B, T, K,
                                        _lib.ptr(slot_of), _lib.stream_of(out))
    _lib.check(rc, "hclsm_event_scatter")
    if out.data_ptr() != output.data_ptr():
        output.copy_(out)
    return output
