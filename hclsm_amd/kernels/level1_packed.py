"""Level-1 event dynamics on packed events in one C call (``hclsm_level1_forward``).

Counterpart of ``Level1EventDynamics.forward`` (hclsm/dynamics/level1_event.py:57-133) for the live
rows of the packed event layout: event e < stats[0] of an EventIndex is rows e*N .. e*N+N-1 of a
(capacity, N, d_slot) tensor.  Every launch inside is sized for the capacity and reads the live count on
the device, so the call never waits on the host.  Inference only: the differentiable path is the
module's torch ops (``Level1EventDynamics.forward_packed``).
"""

from __future__ import annotations

import ctypes

import torch

from hclsm_amd import _lib
from hclsm_amd.kernels._common import require_gpu
from hclsm_amd.kernels.slot_iteration import _workspace
from hclsm_amd.kernels.sparse_event_attn import EventIndex


class Level1Weights:
    """Device copies of a Level1EventDynamics' parameters in the order hclsm_level1_forward takes them:
    proj_in, norm.w, norm.b, proj_out, then per block norm1.w, norm1.b, attn.in_proj_weight,
    attn.out_proj.weight, norm2.w, norm2.b, ffn.w1, ffn.w3, ffn.w2.  Matrices in the compute dtype,
    LayerNorm vectors fp32."""

    def __init__(self, tensors: list, dtype: torch.dtype, d_slot: int, d_model: int, hidden: int, n_layers: int,
                 n_heads: int, ln_eps: float, fold: list | None = None) -> None:
        self.tensors = tensors
        self.ptrs = (ctypes.c_void_p * len(tensors))(*[t.data_ptr() for t in tensors])
        # the folded LayerNorms (16-bit): proj_out diag(g), its row sums, proj_out b; per block in_proj diag(g1),
        # its row sums, in_proj b1, w1 diag(g2), w3 diag(g2), their row sums and w1 b2 | w3 b2 (the C call's fold
        # array)
        self.fold = fold
        self.fold_ptrs = None if fold is None else (ctypes.c_void_p * len(fold))(*[t.data_ptr() for t in fold])
        self.dtype, self.d_slot, self.d_model, self.hidden = dtype, d_slot, d_model, hidden
        self.n_layers, self.n_heads, self.ln_eps = n_layers, n_heads, ln_eps

    @staticmethod
    def _key(m, dtype):
        return (dtype,) + tuple((p.data_ptr(), p._version) for p in m.parameters())

    @classmethod
    def from_module(cls, m, dtype: torch.dtype = torch.bfloat16) -> "Level1Weights":
        """From a Level1EventDynamics-shaped module (attribute names of level1_event.py:57-85); cached
        on the module until a parameter changes."""
        key = cls._key(m, dtype)
        hit = getattr(m, "_hclsm_level1_weights", None)
        if hit is not None and hit[0] == key:
            return hit[1]

        def mat(w):
            return w.detach().to(dtype).contiguous()

        def vec(w):
            return w.detach().to(torch.float32).contiguous()

        eps = {m.norm.eps} | {b.norm1.eps for b in m.blocks} | {b.norm2.eps for b in m.blocks}
        if len(eps) != 1:
            raise ValueError("hclsm_level1_forward takes one LayerNorm eps for every norm")
        t = [mat(m.proj_in.weight), vec(m.norm.weight), vec(m.norm.bias), mat(m.proj_out.weight)]
        for b in m.blocks:
            if b.attn.in_proj_bias is not None or b.attn.out_proj.bias is not None:
                raise ValueError("hclsm_level1_forward: attention without biases (bias=False, level1_event.py:37-39)")
            t += [vec(b.norm1.weight), vec(b.norm1.bias), mat(b.attn.in_proj_weight), mat(b.attn.out_proj.weight),
                  vec(b.norm2.weight), vec(b.norm2.bias), mat(b.ffn.w1.weight), mat(b.ffn.w3.weight),
                  mat(b.ffn.w2.weight)]
        n_heads = m.blocks[0].attn.num_heads if len(m.blocks) else 1
        hidden = m.blocks[0].ffn.w1.weight.shape[0] if len(m.blocks) else 32
        fold = None
        if dtype in (torch.bfloat16, torch.float16) and len(m.blocks):
            # LN(x) W^T = rstd (x (W diag g)^T - mean rowsum(W diag g)) + W b, from the fp32 weights, rounded once
            def folded(w, ln):
                with torch.autocast(w.device.type, enabled=False):
                    w32 = w.detach().float()
                    wn = (w32 * ln.weight.detach().float()[None, :]).to(dtype).contiguous()
                    return wn, wn.float().sum(1), w32 @ ln.bias.detach().float()
            po, po_s, po_b = folded(m.proj_out.weight, m.norm)
            fold = [po, po_s.contiguous(), po_b.contiguous()]
            for b in m.blocks:
                qkv, qkv_s, qkv_b = folded(b.attn.in_proj_weight, b.norm1)
                w1, w1_s, w1_b = folded(b.ffn.w1.weight, b.norm2)
                w3, w3_s, w3_b = folded(b.ffn.w3.weight, b.norm2)
                fold += [qkv, qkv_s.contiguous(), qkv_b.contiguous(),
                         w1, w3, torch.cat([w1_s, w3_s]).contiguous(), torch.cat([w1_b, w3_b]).contiguous()]
        W = cls(t, dtype, m.d_slot, m.d_model, hidden, len(m.blocks), n_heads, float(eps.pop()), fold)
        m._hclsm_level1_weights = (key, W)
        return W


def level1_forward_packed(ev: torch.Tensor, idx: EventIndex, obj_mask: torch.Tensor | None, W: Level1Weights,
                          out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """ev (capacity, N, d_slot) fp32 or W.dtype, events packed as by gather_packed(states, idx);
    obj_mask (B, N) or None.  Returns (capacity, N, d_slot) in out_dtype: rows of the idx.total() live
    events hold Level1EventDynamics' output, later rows are left uninitialised.  No host sync."""
    require_gpu("level1_forward_packed", ev, obj_mask)
    cap, N, d_slot = ev.shape
    if d_slot != W.d_slot:
        raise ValueError(f"ev has d_slot {d_slot}, the weights {W.d_slot}")
    if cap > idx.B * idx.T:
        raise ValueError("more packed rows than the index's capacity")
    x = ev if ev.dtype in (torch.float32, W.dtype) else ev.to(torch.float32)
    x = x.contiguous()
    om = None
    if obj_mask is not None:
        if obj_mask.shape != (idx.B, N):
            raise ValueError(f"obj_mask must be (B, N) = {(idx.B, N)}, got {tuple(obj_mask.shape)}")
        om = obj_mask.detach().to(torch.float32).contiguous()
    out = torch.empty((cap, N, d_slot), dtype=out_dtype, device=ev.device)
    L = _lib.lib()
    code = _lib.dtype_code(W.dtype)
    wsb = L.hclsm_level1_forward_workspace(cap, N, W.d_model, W.hidden, code)
    _lib.check(wsb if wsb < 0 else 0, "hclsm_level1_forward_workspace")
    ws = _workspace(int(wsb), ev.device)
    rc = L.hclsm_level1_forward(_lib.ptr(x), _lib.dtype_code(x.dtype), _lib.ptr(out), _lib.dtype_code(out_dtype),
                                idx.ptr("stats"), cap, N, idx.ptr("rows"), _lib.ptr(om), d_slot, W.d_model,
                                W.n_heads, W.hidden, W.n_layers, W.ptrs, W.fold_ptrs, W.ln_eps, code, _lib.ptr(ws),
                                ws.numel(), _lib.stream_of(x))
    _lib.check(rc, "hclsm_level1_forward")
    return out


_DENSE_TABLES: dict = {}


def _dense_tables(B: int, K: int, device) -> tuple:
    """Device tables of a dense (B, K) event layout, cached per shape: the event count B*K (int32 [1]) and the
    batch row of each event, e // K (int32 [B*K])."""
    key = (B, K, device)
    hit = _DENSE_TABLES.get(key)
    if hit is None:
        n = torch.full((1,), B * K, dtype=torch.int32, device=device)
        rows = torch.arange(B * K, dtype=torch.int32, device=device).div_(K, rounding_mode="floor")
        hit = (n, rows)
        _DENSE_TABLES[key] = hit
    return hit


def level1_forward_dense(ev: torch.Tensor, obj_mask: torch.Tensor | None, W: Level1Weights,
                         out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Level1EventDynamics' stack over every event of a padded (B, K, N, d_slot) batch (the layout of
    HierarchyManager.gather_events), padded events included, in one hclsm_level1_forward call; obj_mask (B, N)
    or None.  Returns (B, K, N, d_slot) in out_dtype.  The caller applies the event padding mask."""
    require_gpu("level1_forward_dense", ev, obj_mask)
    B, K, N, d_slot = ev.shape
    if d_slot != W.d_slot:
        raise ValueError(f"ev has d_slot {d_slot}, the weights {W.d_slot}")
    out = torch.empty((B, K, N, d_slot), dtype=out_dtype, device=ev.device)
    if B * K == 0:
        return out
    x = ev if ev.dtype in (torch.float32, W.dtype) else ev.to(torch.float32)
    x = x.contiguous()
    om = None
    if obj_mask is not None:
        if obj_mask.shape != (B, N):
            raise ValueError(f"obj_mask must be (B, N) = {(B, N)}, got {tuple(obj_mask.shape)}")
        om = obj_mask.detach().to(torch.float32).contiguous()
    n_dev, rows = _dense_tables(B, K, ev.device)
    L = _lib.lib()
    code = _lib.dtype_code(W.dtype)
    cap = B * K
    wsb = L.hclsm_level1_forward_workspace(cap, N, W.d_model, W.hidden, code)
    _lib.check(wsb if wsb < 0 else 0, "hclsm_level1_forward_workspace")
    ws = _workspace(int(wsb), ev.device)
    rc = L.hclsm_level1_forward(_lib.ptr(x), _lib.dtype_code(x.dtype), _lib.ptr(out), _lib.dtype_code(out_dtype),
                                _lib.ptr(n_dev), cap, N, _lib.ptr(rows), _lib.ptr(om), d_slot, W.d_model, W.n_heads,
                                W.hidden, W.n_layers, W.ptrs, W.fold_ptrs, W.ln_eps, code, _lib.ptr(ws), ws.numel(),
                                _lib.stream_of(x))
    _lib.check(rc, "hclsm_level1_forward")
    return out
