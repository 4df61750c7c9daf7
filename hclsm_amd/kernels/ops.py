"""torch.library registration of the hot-path entry points (namespace ``hclsm_hip``).

Each op calls the same C ABI as the eager functions of ``hclsm_amd.kernels`` and carries a fake
kernel, so the ops propagate shapes under FakeTensorMode / torch.compile tracing and on ``meta``
tensors.  The eager functions call the C ABI directly rather than through these ops: a custom op
adds tens of microseconds of Python dispatch per call, which is the size of the kernels.

    hclsm_hip::ssm_scan_fwd(x, dt, A_log, B, C, D?, mode, want_h) -> (y, h_final)
        y in x.dtype; h_final (batch, d_inner, d_state) fp32, or shape (0,) when want_h is False
        (ssm_scan_kernel.py:294-319 forward; mode 0 raw, 1 clamped model form)
    hclsm_hip::ssm_block_scan_fwd(z, dt_in, A_log, B, C, gate) -> (y, y_pre)
        y = silu(gate) * clamped scan with dt = clamp(softplus(dt_in), 1e-3, 1) (level0_ssm.py:72-103)
    hclsm_hip::ssm_scan_bwd(x, dt, A_log, B, C, D?, gy, mode) -> (gx, gdt, gA_log, gB, gC, gD)
        gD has shape (0,) when D is None (ssm_scan_kernel.py:321-377)
    hclsm_hip::slot_attn_core(Q, K, V, scale, denom_eps, logit_clamp, renorm_eps) -> (out, attn)
        softmax over the slot axis; logit_clamp 0 = none, renorm_eps < 0 = none
        (slot_attention_kernel.py:43-152, dynamic_slots.py:116-121)
    hclsm_hip::event_index(mask, rule) -> (counts, offsets, indices, rows, slot_of, stats)
        int32; rule 0 = mask > 0.5 (hierarchy_manager.py:61), 1 = nonzero (sparse_event_attn.py:64)
    hclsm_hip::event_gather(states, counts, offsets, indices, K) -> (B, K, ...)
        zero rows past each count (hierarchy_manager.py:66-75)
    hclsm_hip::event_scatter(base, updates, slot_of) -> (B, T, ...)
        (hierarchy_manager.py:103-116)
    hclsm_hip::event_attention(q, k, v, offsets, indices, key_pad?, scale, mode, capacity) -> (capacity, H, dh)
        mode 0 track-causal, 1 slots with key padding (level1_event.py:37-52)
    hclsm_hip::slot_attention_forward(inputs, slots0, weights, n_iter, scale, logit_clamp, renorm_eps,
                                      slot_clamp, compute_dtype) -> slots fp32
        weights in the order of SLOT_WEIGHT_ORDER (dynamic_slots.py:98-164)
    hclsm_hip::event_gather_packed(states, rows, indices, stats) -> (B*T, ...)
        packed event rows, zero past the live count stats[0] (no host sync)
    hclsm_hip::event_scatter_packed(base, packed, offsets, slot_of) -> (B, T, ...)
    hclsm_hip::event_top_down(level0, events, offsets, slot_of, kpad, level2_context?, obj_mask?, params,
                              compute_dtype) -> fp32 (B, T, N, D)
        HierarchyManager.forward after the Level-1 pass (hierarchy_manager.py:120-162): scatter, Level-2 gate
        and alive mask; events packed (kpad = 0) or padded (B, kpad, N, D); params = l2_to_l1.weight,
        gate_l2_l0.0.weight[, gate_l2_l0.0.bias]
    hclsm_hip::level1_forward(ev, stats, rows, obj_mask?, params, n_heads, ln_eps, compute_dtype) -> fp32
        Level1EventDynamics over the live packed events (level1_event.py:17-133); params in the order of
        Level1Weights (4 + 9 per layer); rows past the live count are zero
    hclsm_hip::relation_graph_forward(nodes, alive?, params, n_rounds, chunked, ln_eps, compute_dtype)
        -> (nodes', causal) fp32: RelationGraph.forward (objects/relation_graph.py:68-193); params in the
        module's state-dict order (18 tensors)
    hclsm_hip::slot_track_sequence(slots, alive?, params, with_hidden, n_iters, temperature, compute_dtype)
        -> (tracked, alive', perm, matched, hidden): the tracking loop of model.py:229-252 over
        SlotTracker's 10 tensors (state-dict order); alive' is empty without alive, hidden without with_hidden
"""

from __future__ import annotations

from typing import Optional

import torch

from hclsm_amd import _lib
from hclsm_amd.kernels._common import require_gpu
from hclsm_amd.kernels.event_attention import event_attention as _event_attention
from hclsm_amd.kernels.slot_attention_kernel import _core_raw
from hclsm_amd.kernels.slot_iteration import SlotMode, SlotWeights, slot_attention_forward as _slot_forward
from hclsm_amd.kernels.level1_packed import Level1Weights, level1_forward_packed
from hclsm_amd.kernels.relation_graph import GNN_PARAM_ORDER, GnnWeights, relation_graph_forward as _gnn_forward
from hclsm_amd.kernels.slot_tracker import TRACK_PARAM_ORDER, TrackerWeights, track_sequence as _track_sequence
from hclsm_amd.kernels.sparse_event_attn import (EventIndex, _gather_padded_raw, _mask_code, _scatter_padded_raw,
                                                 gather_packed, scatter_packed)
from hclsm_amd.kernels.ssm_scan_bwd import scan_backward
from hclsm_amd.kernels.top_down import TopDownWeights, event_top_down as _event_top_down
from hclsm_amd.kernels.ssm_scan_kernel import _block_forward, _scan_forward

Tensor = torch.Tensor
SLOT_WEIGHT_ORDER = ("w_q", "w_k", "w_v", "w_ih", "w_hh", "w1", "w2", "b_ih", "b_hh", "b1", "b2",
                     "ln_pre_w", "ln_pre_b", "ln_mlp_w", "ln_mlp_b", "ln_in_w", "ln_in_b")
_ATTN_MODES = ("track_causal", "slots")


def _index_of(B, T, counts, offsets, indices, slot_of=None):
    return EventIndex(B, T, counts, offsets, indices, None, slot_of, None)


# --------------------------------------------------------------------------- scan

@torch.library.custom_op("hclsm_hip::ssm_scan_fwd", mutates_args=())
def ssm_scan_fwd(x: Tensor, dt: Tensor, A_log: Tensor, B: Tensor, C: Tensor, D: Optional[Tensor],
                 mode: int, want_h: bool) -> tuple[Tensor, Tensor]:
    y, h, _ = _scan_forward(x, dt, A_log, B, C, D, int(mode), bool(want_h))
    return y, (h if h is not None else x.new_empty((0,), dtype=torch.float32))


@ssm_scan_fwd.register_fake
def _(x, dt, A_log, B, C, D, mode, want_h):
    h = x.new_empty((x.shape[0], x.shape[2], B.shape[2]) if want_h else (0,), dtype=torch.float32)
    return torch.empty_like(x), h


@torch.library.custom_op("hclsm_hip::ssm_block_scan_fwd", mutates_args=())
def ssm_block_scan_fwd(z: Tensor, dt_in: Tensor, A_log: Tensor, B: Tensor, C: Tensor,
                       gate: Tensor) -> tuple[Tensor, Tensor]:
    y, y_pre, _ = _block_forward(z, dt_in, A_log, B, C, gate, True)
    return y, y_pre


@ssm_block_scan_fwd.register_fake
def _(z, dt_in, A_log, B, C, gate):
    return torch.empty_like(z), torch.empty_like(z)


@torch.library.custom_op("hclsm_hip::ssm_scan_bwd", mutates_args=())
def ssm_scan_bwd(x: Tensor, dt: Tensor, A_log: Tensor, B: Tensor, C: Tensor, D: Optional[Tensor], gy: Tensor,
                 mode: int) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    g = scan_backward(x, dt, A_log, B, C, D, gy, int(mode))
    gD = g.get("D")
    return (g["x"], g["dt"], g["A_log"], g["B"], g["C"],
            gD if gD is not None else x.new_empty((0,), dtype=torch.float32))


@ssm_scan_bwd.register_fake
def _(x, dt, A_log, B, C, D, gy, mode):
    f32 = torch.float32
    return (torch.empty_like(x), torch.empty_like(dt), torch.empty_like(A_log, dtype=f32), torch.empty_like(B),
            torch.empty_like(C), x.new_empty((x.shape[2],) if D is not None else (0,), dtype=f32))


# --------------------------------------------------------------------------- slot attention

@torch.library.custom_op("hclsm_hip::slot_attn_core", mutates_args=())
def slot_attn_core(Q: Tensor, K: Tensor, V: Tensor, scale: float, denom_eps: float, logit_clamp: float,
                   renorm_eps: float) -> tuple[Tensor, Tensor]:
    out, attn = _core_raw(Q, K, V, scale, denom_eps, logit_clamp=logit_clamp or None,
                          renorm_eps=renorm_eps if renorm_eps >= 0 else None)
    return out.to(Q.dtype), attn.to(Q.dtype)


@slot_attn_core.register_fake
def _(Q, K, V, scale, denom_eps, logit_clamp, renorm_eps):
    return torch.empty_like(Q), Q.new_empty((Q.shape[0], Q.shape[1], K.shape[1]))


@torch.library.custom_op("hclsm_hip::slot_attention_forward", mutates_args=())
def slot_attention_forward(inputs: Tensor, slots0: Tensor, weights: list[Tensor], n_iter: int, scale: float,
                           logit_clamp: float, renorm_eps: float, slot_clamp: float,
                           compute_dtype: torch.dtype) -> Tensor:
    if len(weights) != len(SLOT_WEIGHT_ORDER):
        raise ValueError(f"expected {len(SLOT_WEIGHT_ORDER)} weights in the order {SLOT_WEIGHT_ORDER}")
    W = SlotWeights.from_dict(dict(zip(SLOT_WEIGHT_ORDER, weights)), compute_dtype, inputs.device)
    mode = SlotMode(logit_clamp=logit_clamp or None, renorm_eps=renorm_eps if renorm_eps >= 0 else None,
                    slot_clamp=slot_clamp or None)
    return _slot_forward(inputs, slots0, W, int(n_iter), mode, scale=scale)


@slot_attention_forward.register_fake
def _(inputs, slots0, weights, n_iter, scale, logit_clamp, renorm_eps, slot_clamp, compute_dtype):
    return torch.empty_like(slots0, dtype=torch.float32)


# --------------------------------------------------------------------------- events

@torch.library.custom_op("hclsm_hip::event_index", mutates_args=())
def event_index(mask: Tensor, rule: int) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    # separate allocations: a custom op's outputs may not alias each other (the eager
    # build_event_index carves all six tables out of one buffer)
    require_gpu("event_index", mask)
    if mask.dim() != 2:
        raise ValueError(f"event_mask must be (B, T), got {tuple(mask.shape)}")
    m, code = _mask_code(mask.detach().contiguous())
    B, T = m.shape
    i32 = dict(dtype=torch.int32, device=m.device)
    cap = max(B * T, 1)
    t = (torch.empty(B, **i32), torch.empty(B + 1, **i32), torch.empty(cap, **i32), torch.empty(cap, **i32),
         torch.empty((B, T), **i32), torch.empty(2, **i32))
    rc = _lib.lib().hclsm_event_index(_lib.ptr(m), code, B, T, (_lib.EVENT_GT_HALF, _lib.EVENT_NONZERO)[rule],
                                      *(_lib.ptr(x) for x in t), _lib.stream_of(m))
    _lib.check(rc, "hclsm_event_index")
    return t


@event_index.register_fake
def _(mask, rule):
    B, T = mask.shape
    i32 = dict(dtype=torch.int32, device=mask.device)
    n = max(B * T, 1)
    return (torch.empty(B, **i32), torch.empty(B + 1, **i32), torch.empty(n, **i32), torch.empty(n, **i32),
            torch.empty((B, T), **i32), torch.empty(2, **i32))


@torch.library.custom_op("hclsm_hip::event_gather", mutates_args=())
def event_gather(states: Tensor, counts: Tensor, offsets: Tensor, indices: Tensor, K: int) -> Tensor:
    return _gather_padded_raw(states, _index_of(states.shape[0], states.shape[1], counts, offsets, indices), int(K))


@event_gather.register_fake
def _(states, counts, offsets, indices, K):
    return states.new_empty((states.shape[0], K) + tuple(states.shape[2:]))


@torch.library.custom_op("hclsm_hip::event_scatter", mutates_args=())
def event_scatter(base: Tensor, updates: Tensor, slot_of: Tensor) -> Tensor:
    B, T = slot_of.shape
    idx = _index_of(B, T, None, None, None, slot_of)
    return _scatter_padded_raw(base, updates.to(base.dtype), idx, updates.shape[1], base)


@event_scatter.register_fake
def _(base, updates, slot_of):
    return torch.empty_like(base)


@torch.library.custom_op("hclsm_hip::event_attention", mutates_args=())
def event_attention(q: Tensor, k: Tensor, v: Tensor, offsets: Tensor, indices: Tensor, key_pad: Optional[Tensor],
                    scale: float, mode: int, capacity: int) -> Tensor:
    idx = _index_of(q.shape[0], q.shape[1], None, offsets, indices)
    return _event_attention(q, k, v, idx, _ATTN_MODES[mode], scale=scale, key_pad=key_pad, out="packed",
                            capacity=int(capacity))


@event_attention.register_fake
def _(q, k, v, offsets, indices, key_pad, scale, mode, capacity):
    return q.new_empty((capacity, q.shape[2], q.shape[3]))


@torch.library.custom_op("hclsm_hip::event_gather_packed", mutates_args=())
def event_gather_packed(states: Tensor, rows: Tensor, indices: Tensor, stats: Tensor) -> Tensor:
    idx = EventIndex(states.shape[0], states.shape[1], None, None, indices, rows, None, stats)
    return gather_packed(states, idx, zero_fill=True)


@event_gather_packed.register_fake
def _(states, rows, indices, stats):
    return states.new_empty((states.shape[0] * states.shape[1],) + tuple(states.shape[2:]))


@torch.library.custom_op("hclsm_hip::event_scatter_packed", mutates_args=())
def event_scatter_packed(base: Tensor, packed: Tensor, offsets: Tensor, slot_of: Tensor) -> Tensor:
    B, T = slot_of.shape
    idx = EventIndex(B, T, None, offsets, None, None, slot_of, None)
    return scatter_packed(base, packed.to(base.dtype), idx)


@event_scatter_packed.register_fake
def _(base, packed, offsets, slot_of):
    return torch.empty_like(base)


@torch.library.custom_op("hclsm_hip::event_top_down", mutates_args=())
def event_top_down(level0: Tensor, events: Tensor, offsets: Tensor, slot_of: Tensor, kpad: int,
                   level2_context: Optional[Tensor], obj_mask: Optional[Tensor], params: list[Tensor],
                   compute_dtype: torch.dtype) -> Tensor:
    B, T = slot_of.shape
    idx = EventIndex(B, T, None, offsets, None, None, slot_of, None)
    W = None
    if level2_context is not None:
        if len(params) not in (2, 3):
            raise ValueError("event_top_down: params are l2_to_l1.weight, gate_l2_l0.0.weight[, its bias]")
        W = TopDownWeights.from_tensors(params[0], params[1], params[2] if len(params) == 3 else None, compute_dtype)
    return _event_top_down(level0, events, idx, W, level2_context, obj_mask, kpad=int(kpad))


@event_top_down.register_fake
def _(level0, events, offsets, slot_of, kpad, level2_context, obj_mask, params, compute_dtype):
    return torch.empty(level0.shape, dtype=torch.float32, device=level0.device)


@torch.library.custom_op("hclsm_hip::level1_forward", mutates_args=())
def level1_forward(ev: Tensor, stats: Tensor, rows: Tensor, obj_mask: Optional[Tensor], params: list[Tensor],
                   n_heads: int, ln_eps: float, compute_dtype: torch.dtype) -> Tensor:
    if len(params) < 4 or (len(params) - 4) % 9:
        raise ValueError("level1_forward: params are proj_in, norm.w, norm.b, proj_out, then 9 per layer")
    n_layers = (len(params) - 4) // 9
    mats = {0, 3} | {4 + 9 * l + j for l in range(n_layers) for j in (2, 3, 6, 7, 8)}
    t = [p.detach().to(compute_dtype if i in mats else torch.float32).contiguous() for i, p in enumerate(params)]
    d_model, d_slot = t[0].shape
    hidden = t[10].shape[0] if n_layers else 32
    W = Level1Weights(t, compute_dtype, d_slot, d_model, hidden, n_layers, int(n_heads), float(ln_eps))
    cap, N = ev.shape[0], ev.shape[1]
    B = obj_mask.shape[0] if obj_mask is not None else max(cap, 1)
    idx = EventIndex(B, max(cap // max(B, 1), 1), None, None, None, rows, None, stats)
    idx.B, idx.T = B, (cap + B - 1) // B if B else 1
    out = level1_forward_packed(ev, idx, obj_mask, W, out_dtype=torch.float32)
    live = torch.arange(cap, device=ev.device) < stats[0]          # device-side: rows past the count -> 0
    return torch.where(live[:, None, None], out, out.new_zeros(()))


@level1_forward.register_fake
def _(ev, stats, rows, obj_mask, params, n_heads, ln_eps, compute_dtype):
    return ev.new_empty(ev.shape, dtype=torch.float32)


# --------------------------------------------------------------------------- object layer

@torch.library.custom_op("hclsm_hip::relation_graph_forward", mutates_args=())
def relation_graph_forward(nodes: Tensor, alive: Optional[Tensor], params: list[Tensor], n_rounds: int,
                           chunked: bool, ln_eps: float, compute_dtype: torch.dtype) -> tuple[Tensor, Tensor]:
    if len(params) != len(GNN_PARAM_ORDER):
        raise ValueError(f"relation_graph_forward: {len(GNN_PARAM_ORDER)} parameters in state-dict order")
    W = GnnWeights.from_dict(dict(zip(GNN_PARAM_ORDER, params)), compute_dtype, float(ln_eps), nodes.device)
    return _gnn_forward(nodes, alive, W, int(n_rounds), chunked=bool(chunked))


@relation_graph_forward.register_fake
def _(nodes, alive, params, n_rounds, chunked, ln_eps, compute_dtype):
    F, N, D = nodes.shape
    return nodes.new_empty((F, N, D), dtype=torch.float32), nodes.new_empty((F, N, N), dtype=torch.float32)


@torch.library.custom_op("hclsm_hip::slot_track_sequence", mutates_args=())
def slot_track_sequence(slots: Tensor, alive: Optional[Tensor], params: list[Tensor], with_hidden: bool,
                        n_iters: int, temperature: float,
                        compute_dtype: torch.dtype) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    if len(params) != len(TRACK_PARAM_ORDER):
        raise ValueError(f"slot_track_sequence: {len(TRACK_PARAM_ORDER)} parameters in state-dict order")
    W = TrackerWeights.from_dict(dict(zip(TRACK_PARAM_ORDER, params)), compute_dtype, slots.device)
    r = _track_sequence(slots, alive, W, with_hidden=bool(with_hidden), n_iters=int(n_iters),
                        temperature=float(temperature))
    empty = slots.new_empty((0,), dtype=torch.float32)
    return (r["tracked"], r["alive"] if r["alive"] is not None else empty, r["perm"], r["matched"],
            r["hidden"] if r["hidden"] is not None else empty)


@slot_track_sequence.register_fake
def _(slots, alive, params, with_hidden, n_iters, temperature, compute_dtype):
    B, T, N, D = slots.shape
    f32 = dict(dtype=torch.float32)
    return (slots.new_empty((B, T, N, D), **f32),
            slots.new_empty((B, T, N) if alive is not None else (0,), **f32),
            slots.new_empty((B, T, N), dtype=torch.int64), slots.new_empty((B, T, N), **f32),
            slots.new_empty((B, N, D) if with_hidden else (0,), **f32))
