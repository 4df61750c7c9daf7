"""Variable-length event attention on MFMA (libhclsm_amd.so: hclsm_event_attention).

Two semantics over the same kernel:

  * ``track_causal``: for each track, causal softmax attention among that track's event
    timesteps (the sparse Level-1 event attention of the benchmark configurations: per-track
    segments packed by int32 prefix-sum offsets).
  * ``slots``: for each (batch, event) problem, attention across its N slot rows with a key
    padding mask -- the attention core of ``nn.MultiheadAttention`` inside
    ``EventTransformerBlock`` (reference dynamics/level1_event.py:37-52; projections stay
    outside, as in MHA's in_proj / out_proj).

Inputs are (P, T, H, dh) tensors on the GPU (bf16, fp16 or fp32; softmax and accumulation
in fp32); dh in {16, 32, 64, 128}.
"""

from __future__ import annotations

import torch

from hclsm_amd import _lib
from hclsm_amd.kernels._common import require_gpu
from hclsm_amd.kernels.sparse_event_attn import EventIndex, _mask_code, build_event_index

_MODES = {"track_causal": _lib.ATTN_TRACK_CAUSAL, "slots": _lib.ATTN_SLOTS}
_RULES = {"gt_half": _lib.EVENT_GT_HALF, "nonzero": _lib.EVENT_NONZERO}


def _check_qkv(q, k, v):
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q, k, v must share a (P, T, H, dh) shape, got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError("q, k, v must share one dtype among bfloat16, float16, float32")


def event_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, index: EventIndex,
                    mode: str = "track_causal", scale: float | None = None,
                    key_pad: torch.Tensor | None = None, out: str = "packed",
                    capacity: int | None = None, out_grid: torch.Tensor | None = None) -> torch.Tensor:
    """Attention over the segments of ``index`` (segment p = rows (p, indices[offsets[p]:offsets[p+1]])).

    out="packed": returns (capacity, H, dh) with row offsets[p] + i = query i of segment p
        (capacity defaults to index.total(), one host read);
    out="grid":   returns (P, T, H, dh) holding the outputs at the query rows; other rows are
        copied from ``out_grid`` if given (written in place) or zero.
    """
    require_gpu("event_attention", q, k, v, key_pad)
    _check_qkv(q, k, v)
    P, T, H, dh = q.shape
    if (index.B, index.T) != (P, T):
        raise ValueError(f"event index is for ({index.B}, {index.T}) but q is ({P}, {T}, ...)")
    qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
    kp = None
    if key_pad is not None:
        if key_pad.shape != (P, T):
            raise ValueError(f"key_pad must be ({P}, {T}), got {tuple(key_pad.shape)}")
        kp = key_pad.to(torch.uint8).contiguous()
    if scale is None:
        scale = dh ** -0.5
    outp = outg = None
    cap = 0
    if out == "packed":
        cap = index.total() if capacity is None else int(capacity)
        outp = torch.empty((max(cap, 0), H, dh), dtype=q.dtype, device=q.device)
        result = outp
    elif out == "grid":
        outg = out_grid if out_grid is not None else torch.zeros_like(qc)
        if outg.shape != qc.shape or outg.dtype != qc.dtype or not outg.is_contiguous():
            raise ValueError("out_grid must be a contiguous tensor shaped and typed like q")
        result = outg
    else:
        raise ValueError(f"out must be 'packed' or 'grid', got {out!r}")
    rc = _lib.lib().hclsm_event_attention(
        _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), _lib.ptr(outp), _lib.ptr(outg),
        index.ptr("offsets"), index.ptr("indices"), _lib.ptr(kp), P, T, H, dh, max(cap, 0), float(scale),
        _lib.dtype_code(q.dtype), _MODES[mode], _lib.stream_of(qc))
    _lib.check(rc, "hclsm_event_attention")
    return result


def track_causal_event_attention(q, k, v, event_mask, scale=None, out="packed", rule="gt_half", capacity=None,
                                 *, out_packed=None, index=None):
    """Per-track causal attention among the event timesteps of ``event_mask`` (P, T).
    Returns (packed output, event index).  With out="packed" and a known ``capacity`` (rows of the packed
    output; events past it are dropped) the index build and the attention are one library call
    (hclsm_track_causal_attention) with no host synchronisation; otherwise the index is built first and
    the output sized by its total (one host read).

    A loop over steps of one shape can pass back the buffers of an earlier call: ``out_packed`` (a
    contiguous (capacity, H, dh) tensor of q's dtype; capacity defaults to its rows) and ``index`` (an
    EventIndex of this (P, T) from EventIndex.allocate or an earlier call, rewritten in place).  Nothing
    is allocated then."""
    if out != "packed" or (capacity is None and out_packed is None):
        idx = build_event_index(event_mask, rule)
        return event_attention(q, k, v, idx, "track_causal", scale=scale, out=out, capacity=capacity), idx
    require_gpu("track_causal_event_attention", q, k, v, event_mask, out_packed)
    _check_qkv(q, k, v)
    P, T, H, dh = q.shape
    if tuple(event_mask.shape) != (P, T):
        raise ValueError(f"event_mask must be ({P}, {T}) to match q, got {tuple(event_mask.shape)}")
    cap = int(capacity) if capacity is not None else out_packed.shape[0]
    if cap < 0:
        raise ValueError(f"capacity must be >= 0, got {cap}")
    m, code = _mask_code(event_mask.detach().contiguous())
    qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
    if index is None:
        idx = EventIndex.allocate(P, T, q.device)
    elif index._buf is None or (index.B, index.T) != (P, T) or index._buf.device != q.device:
        raise ValueError(f"index must be an EventIndex.allocate({P}, {T}) buffer on {q.device}")
    else:
        idx = index
    if out_packed is None:
        outp = torch.empty((cap, H, dh), dtype=q.dtype, device=q.device)
    elif (out_packed.dtype != q.dtype or not out_packed.is_contiguous() or out_packed.dim() != 3
          or tuple(out_packed.shape[1:]) != (H, dh) or out_packed.shape[0] < cap):
        raise ValueError(f"out_packed must be a contiguous ({cap}, {H}, {dh}) {q.dtype} tensor")
    else:
        outp = out_packed
    rc = _lib.lib().hclsm_track_causal_attention(
        m.data_ptr(), code, _RULES[rule], qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), outp.data_ptr(), P, T, H, dh,
        cap, float(dh ** -0.5 if scale is None else scale), _lib.dtype_code(q.dtype), idx.ptr("stats"),
        _lib.stream_of(qc))
    _lib.check(rc, "hclsm_track_causal_attention")
    return outp, idx


class TrackCausalPlan:
    """track_causal_event_attention prepared for a loop over steps of one shape (a serving loop): the tensors
    are checked and the output and index buffers allocated once, and each call is the one library call
    (hclsm_track_causal_attention) on torch's current stream, reading whatever q, k, v and the mask hold at
    that moment.  The caller keeps those tensors alive and updates them in place between calls.

        plan = TrackCausalPlan(q, k, v, event_mask, capacity)
        out, index = plan()      # the same (out, index) objects every call
    """

    def __init__(self, q, k, v, event_mask, capacity, scale=None, rule="gt_half"):
        require_gpu("TrackCausalPlan", q, k, v, event_mask)
        _check_qkv(q, k, v)
        P, T, H, dh = q.shape
        if tuple(event_mask.shape) != (P, T):
            raise ValueError(f"event_mask must be ({P}, {T}) to match q, got {tuple(event_mask.shape)}")
        if not (q.is_contiguous() and k.is_contiguous() and v.is_contiguous() and event_mask.is_contiguous()):
            raise ValueError("TrackCausalPlan binds device pointers: q, k, v and the mask must be contiguous")
        cap = int(capacity)
        if cap < 0:
            raise ValueError(f"capacity must be >= 0, got {cap}")
        m, code = _mask_code(event_mask.detach())
        if m.data_ptr() != event_mask.data_ptr():
            raise TypeError("TrackCausalPlan needs a float32, bfloat16, float16, bool or uint8 mask")
        self.out = torch.empty((cap, H, dh), dtype=q.dtype, device=q.device)
        self.index = EventIndex.allocate(P, T, q.device)
        self._keep = (q, k, v, event_mask)
        self._fn = _lib.lib().hclsm_track_causal_attention
        self._dev = q.get_device()
        self._args = (m.data_ptr(), code, _RULES[rule], q.data_ptr(), k.data_ptr(), v.data_ptr(),
                      self.out.data_ptr(), P, T, H, dh, cap, float(dh ** -0.5 if scale is None else scale),
                      _lib.dtype_code(q.dtype), self.index.ptr("stats"))

    def __call__(self):
        rc = self._fn(*self._args, _lib.stream_of_device(self._dev))
        if rc:
            _lib.check(rc, "hclsm_track_causal_attention")
        return self.out, self.index


_DENSE_CACHE: dict = {}


def _dense_index(P: int, N: int, device) -> EventIndex:
    key = (P, N, str(device))
    idx = _DENSE_CACHE.get(key)
    if idx is None:
        i32 = dict(dtype=torch.int32, device=device)
        offsets = torch.arange(0, (P + 1) * N, N, **i32)
        indices = torch.arange(N, **i32).repeat(P)
        rows = torch.arange(P, **i32).repeat_interleave(N)
        slot_of = torch.arange(N, **i32).repeat(P, 1)
        stats = torch.tensor([P * N, N], **i32)
        idx = EventIndex(P, N, torch.full((P,), N, **i32), offsets, indices, rows, slot_of, stats)
        if len(_DENSE_CACHE) > 64:
            _DENSE_CACHE.clear()
        _DENSE_CACHE[key] = idx
    return idx


def _slots_attention_raw(q, k, v, key_padding_mask, scale):
    P, N = q.shape[:2]
    idx = _dense_index(P, N, q.device)
    return event_attention(q, k, v, idx, "slots", scale=scale, key_pad=key_padding_mask, out="grid",
                           out_grid=torch.empty(q.shape, dtype=q.dtype, device=q.device))


class _SlotsAttention(torch.autograd.Function):
    """HIP forward; backward recomputes the (small, N x N) softmax in fp32 with torch on the GPU."""

    @staticmethod
    def forward(ctx, q, k, v, key_padding_mask, scale):
        ctx.save_for_backward(q, k, v, key_padding_mask if key_padding_mask is not None else torch.empty(0))
        ctx.has_kp = key_padding_mask is not None
        ctx.scale = scale
        return _slots_attention_raw(q, k, v, key_padding_mask, scale)

    @staticmethod
    def backward(ctx, go):
        q, k, v, kp = ctx.saved_tensors
        qf, kf, vf, gf = (t.float().permute(0, 2, 1, 3).contiguous() for t in (q, k, v, go))   # (P, H, N, dh)
        s = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * ctx.scale
        if ctx.has_kp:
            s = s.masked_fill(kp.bool()[:, None, None, :], float("-inf"))
        p = torch.softmax(s, dim=-1)
        dv = torch.matmul(p.transpose(-1, -2).contiguous(), gf)
        dp = torch.matmul(gf, vf.transpose(-1, -2).contiguous())
        ds = p * (dp - (dp * p).sum(dim=-1, keepdim=True))
        dq = torch.matmul(ds, kf) * ctx.scale
        dk = torch.matmul(ds.transpose(-1, -2).contiguous(), qf) * ctx.scale
        back = lambda t, like: t.permute(0, 2, 1, 3).contiguous().to(like.dtype)
        return back(dq, q), back(dk, k), back(dv, v), None, None


def slots_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    key_padding_mask: torch.Tensor | None = None, scale: float | None = None) -> torch.Tensor:
    """Attention across the N slot rows of each of P problems: q, k, v (P, N, H, dh);
    key_padding_mask (P, N) bool, True = ignore that key (nn.MultiheadAttention's convention).
    Returns (P, N, H, dh).  A query with every key padded returns NaN, like the reference.
    Differentiable (forward on the HIP kernel)."""
    require_gpu("slots_attention", q, k, v, key_padding_mask)
    if scale is None:
        scale = q.shape[-1] ** -0.5
    kp = None if key_padding_mask is None else key_padding_mask.to(torch.bool).contiguous()
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        return _SlotsAttention.apply(q, k, v, kp, float(scale))
    return _slots_attention_raw(q, k, v, kp, float(scale))
