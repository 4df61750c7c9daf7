"""Slot tracking (matching MLP, Sinkhorn, reorder + GRU carry) in C calls (``hclsm_slot_track_*``).

Counterparts of SlotTracker (hclsm/objects/slot_tracker.py:46-158) and of the frame loop of
hclsm/model.py:229-252:

* ``track_cost``            compute_cost_matrix (:74-107): the pair features (frames, N, N, 3D) are never
                            materialised; the [a; b] blocks of the first layer are per-node projections and
                            only W1c |a_i - b_j| is contracted per pair, on MFMA pair tiles.
* ``track_match``           forward after the cost (:122-135): clamp, Sinkhorn (:15-43), argmax, matched.
* ``track_reorder_update``  reorder_and_update (:137-158).
* ``track_sequence``        the whole loop: one launch for the costs of every (t-1, t) frame pair (the
                            previous perm only reorders cost rows), then one workgroup per clip runs the
                            Sinkhorn steps in sequence; the GRU carry is optional (the model discards it).

Inference only; fp32 inputs, matrices in the compute dtype.
"""

from __future__ import annotations

import ctypes

import torch

from hclsm_amd import _lib
from hclsm_amd.kernels._common import require_gpu
from hclsm_amd.kernels.slot_iteration import _workspace

# parameter order of the C entries = the module's state-dict order (slot_tracker.py:59-72)
TRACK_PARAM_ORDER = ("match_mlp.0.weight", "match_mlp.0.bias", "match_mlp.2.weight", "match_mlp.2.bias",
                     "match_mlp.4.weight", "match_mlp.4.bias", "hidden_gru.weight_ih", "hidden_gru.weight_hh",
                     "hidden_gru.bias_ih", "hidden_gru.bias_hh")
_MATRICES = {"match_mlp.0.weight", "match_mlp.2.weight", "hidden_gru.weight_ih", "hidden_gru.weight_hh"}

SINKHORN_ITERS = 20         # slot_tracker.py:127
SINKHORN_TEMPERATURE = 0.05


class TrackerWeights:
    """Device copies of a SlotTracker's parameters in TRACK_PARAM_ORDER: matrices in the compute dtype, the
    rest fp32 (match_mlp.4.weight as a vector)."""

    def __init__(self, tensors: list, dtype: torch.dtype, d_slot: int) -> None:
        self.tensors = tensors
        ptrs = [t.data_ptr() for t in tensors]
        self.ptrs = (ctypes.c_void_p * 10)(*ptrs)
        self.match_ptrs = (ctypes.c_void_p * 6)(*ptrs[:6])
        self.gru_ptrs = (ctypes.c_void_p * 4)(*ptrs[6:])
        self.dtype, self.d_slot = dtype, d_slot

    @classmethod
    def from_dict(cls, w: dict, dtype: torch.dtype, device="cuda") -> "TrackerWeights":
        t = []
        for name in TRACK_PARAM_ORDER:
            v = torch.as_tensor(w[name]).detach()
            v = v.to(device=device, dtype=dtype if name in _MATRICES else torch.float32)
            t.append(v.contiguous() if name in _MATRICES else v.reshape(-1).contiguous())
        return cls(t, dtype, t[0].shape[0])

    @classmethod
    def from_module(cls, m, dtype: torch.dtype) -> "TrackerWeights":
        key = (dtype,) + tuple((p.data_ptr(), p._version) for p in m.parameters())
        hit = getattr(m, "_hclsm_track_weights", None)
        if hit is not None and hit[0] == key:
            return hit[1]
        W = cls.from_dict(dict(m.named_parameters()), dtype, m.match_mlp[0].weight.device)
        m._hclsm_track_weights = (key, W)
        return W


def track_supported(N: int, d_slot: int, dtype: torch.dtype, sequence: bool = False) -> bool:
    """Whether the tracker entries take this shape: d_slot a multiple of 64 and at most 384; the Sinkhorn
    entries also N <= 128."""
    code = _lib.dtype_code(dtype)
    L = _lib.lib()
    if sequence:
        return int(L.hclsm_slot_track_sequence_workspace(1, 2, N, d_slot, 0, code)) >= 0
    return int(L.hclsm_slot_track_cost_workspace(1, N, d_slot, code)) >= 0 and N <= 128


def _f32(t):
    return None if t is None else t.detach().to(torch.float32).contiguous()


def track_cost(slots_t, slots_t1, alive_t, alive_t1, W: TrackerWeights) -> torch.Tensor:
    """(F, N, D) x2, alive (F, N) x2 (or both None) -> cost (F, N, N) fp32, lower = better (unclamped)."""
    require_gpu("track_cost", slots_t, slots_t1, alive_t, alive_t1)
    F, N, D = slots_t.shape
    if slots_t1.shape != slots_t.shape:
        raise ValueError(f"slots_t {tuple(slots_t.shape)} and slots_t1 {tuple(slots_t1.shape)} differ")
    a, b, at, at1 = _f32(slots_t), _f32(slots_t1), _f32(alive_t), _f32(alive_t1)
    cost = torch.empty((F, N, N), dtype=torch.float32, device=a.device)
    L = _lib.lib()
    code = _lib.dtype_code(W.dtype)
    wsb = L.hclsm_slot_track_cost_workspace(F, N, D, code)
    _lib.check(wsb if wsb < 0 else 0, "hclsm_slot_track_cost_workspace")
    ws = _workspace(int(wsb), a.device)
    rc = L.hclsm_slot_track_cost(_lib.ptr(a), _lib.ptr(b), _lib.ptr(at), _lib.ptr(at1), _lib.ptr(cost), F, N, D,
                                 W.match_ptrs, code, _lib.ptr(ws), ws.numel(), _lib.stream_of(a))
    _lib.check(rc, "hclsm_slot_track_cost")
    return cost


def track_match(cost, alive_t=None, alive_t1=None, n_iters: int = SINKHORN_ITERS,
                temperature: float = SINKHORN_TEMPERATURE):
    """cost (F, N, N) -> (perm (F, N) int64, matched (F, N) fp32, confidence (F, N) fp32)."""
    require_gpu("track_match", cost, alive_t, alive_t1)
    F, N, _ = cost.shape
    c, at, at1 = _f32(cost), _f32(alive_t), _f32(alive_t1)
    perm = torch.empty((F, N), dtype=torch.int64, device=c.device)
    matched = torch.empty((F, N), dtype=torch.float32, device=c.device)
    conf = torch.empty((F, N), dtype=torch.float32, device=c.device)
    rc = _lib.lib().hclsm_slot_track_match(_lib.ptr(c), _lib.ptr(at), _lib.ptr(at1), _lib.ptr(perm),
                                           _lib.ptr(matched), _lib.ptr(conf), F, N, int(n_iters),
                                           float(temperature), _lib.stream_of(c))
    _lib.check(rc, "hclsm_slot_track_match")
    return perm, matched, conf


def track_reorder_update(slots_t1, perm, hidden_t, matched, W: TrackerWeights):
    """-> (reordered (F, N, D), hidden_t1 (F, N, D)) fp32.  perm entries outside [0, N) give NaN rows."""
    require_gpu("track_reorder_update", slots_t1, perm, hidden_t, matched)
    F, N, D = slots_t1.shape
    x, h, m = _f32(slots_t1), _f32(hidden_t), _f32(matched)
    p = perm.detach().to(torch.int64).contiguous()
    re = torch.empty_like(x)
    h1 = torch.empty_like(x)
    L = _lib.lib()
    code = _lib.dtype_code(W.dtype)
    wsb = L.hclsm_slot_track_reorder_update_workspace(F, N, D, code)
    _lib.check(wsb if wsb < 0 else 0, "hclsm_slot_track_reorder_update_workspace")
    ws = _workspace(int(wsb), x.device)
    rc = L.hclsm_slot_track_reorder_update(_lib.ptr(x), _lib.ptr(p), _lib.ptr(h), _lib.ptr(m), _lib.ptr(re),
                                           _lib.ptr(h1), F, N, D, W.gru_ptrs, code, _lib.ptr(ws), ws.numel(),
                                           _lib.stream_of(x))
    _lib.check(rc, "hclsm_slot_track_reorder_update")
    return re, h1


def track_sequence(slots, alive, W: TrackerWeights, with_hidden: bool = False, n_iters: int = SINKHORN_ITERS,
                   temperature: float = SINKHORN_TEMPERATURE) -> dict:
    """The tracking loop of model.py:229-252 for slots (B, T, N, D), alive (B, T, N) or None.  Returns a dict
    with ``tracked`` (B, T, N, D), ``alive`` (B, T, N) reordered alongside, ``perm`` (B, T, N) int64 (frame 0:
    identity), ``matched`` (B, T, N) (frame 0: zeros) and, with with_hidden, ``hidden`` (B, N, D), the GRU
    state after the last frame."""
    require_gpu("track_sequence", slots, alive)
    B, T, N, D = slots.shape
    x, al = _f32(slots), _f32(alive)
    dev = x.device
    tracked = torch.empty_like(x)
    alive_out = torch.empty((B, T, N), dtype=torch.float32, device=dev)
    perm = torch.empty((B, T, N), dtype=torch.int64, device=dev)
    matched = torch.empty((B, T, N), dtype=torch.float32, device=dev)
    hidden = torch.empty((B, N, D), dtype=torch.float32, device=dev) if with_hidden else None
    L = _lib.lib()
    code = _lib.dtype_code(W.dtype)
    wsb = L.hclsm_slot_track_sequence_workspace(B, T, N, D, int(with_hidden), code)
    _lib.check(wsb if wsb < 0 else 0, "hclsm_slot_track_sequence_workspace")
    ws = _workspace(int(wsb), dev)
    rc = L.hclsm_slot_track_sequence(_lib.ptr(x), _lib.ptr(al), _lib.ptr(tracked),
                                     _lib.ptr(alive_out) if al is not None else None, _lib.ptr(perm),
                                     _lib.ptr(matched), _lib.ptr(hidden), B, T, N, D, int(n_iters),
                                     float(temperature), W.ptrs, code, _lib.ptr(ws), ws.numel(), _lib.stream_of(x))
    _lib.check(rc, "hclsm_slot_track_sequence")
    if al is None:
        alive_out = None
    return {"tracked": tracked, "alive": alive_out, "perm": perm, "matched": matched, "hidden": hidden}
