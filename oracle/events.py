"""Oracle: event index, gather/scatter and event attention.  TEST INFRASTRUCTURE ONLY.

Event index (integer, bit-exact):
  * event rule "gt_half": mask > 0.5 -- HierarchyManager.gather_events (dynamics/hierarchy_manager.py:61)
    and the pad test of _vectorized_gather (kernels/sparse_event_attn.py:124).
  * event rule "nonzero": mask != 0 (NaN counts as an event) -- naive_sparse_event_attention's
    ``nonzero`` (sparse_event_attn.py:65).
  * counts[b] = number of events in row b; offsets = exclusive prefix sum (length B+1);
    indices = event timesteps of each row in ascending t, rows concatenated (the ``nonzero``
    order of sparse_event_attn.py:65, the canonical order here; the reference's sort/topk
    order at hierarchy_manager.py:66 and sparse_event_attn.py:117 is tie-dependent, and no
    output depends on it); rows[e] = the row of packed event e; slot_of[b, t] = rank of t
    among row b's events, or -1.

Gather / scatter (byte moves, bit-exact):
  * padded gather -> (B, K, ...) with zero rows for k >= count[b]
    (hierarchy_manager.py:69-75, sparse_event_attn.py:59-70, :121-128);
  * scatter: out = base, except out[b, t] = upd[b, slot_of[b, t]] where 0 <= slot < K
    (hierarchy_manager.py:79-118, sparse_event_attn.py:78-84, :134-150).

Event attention (float):
  * "track_causal": per track, causal softmax attention among that track's event rows
    (the benchmark's config 3/4 semantics).
  * "slots": per (row, head), attention across the N slot rows with a key padding mask --
    the core of nn.MultiheadAttention in EventTransformerBlock (dynamics/level1_event.py:37-52),
    without its projections.
"""

from __future__ import annotations

import numpy as np


def event_bool(mask, rule="gt_half"):
    m = np.asarray(mask)
    if m.dtype == np.bool_:
        return m.copy()
    if rule == "gt_half":
        return m.astype(np.float64) > 0.5
    if rule == "nonzero":
        return ~(m.astype(np.float64) == 0)   # NaN != 0 -> event, like torch.nonzero
    raise ValueError(rule)


def event_index(mask, rule="gt_half"):
    """Returns dict of int32 arrays: counts (B,), offsets (B+1,), indices (total,),
    rows (total,), slot_of (B, T); and ints total, kmax."""
    ev = event_bool(mask, rule)
    B, T = ev.shape
    counts = ev.sum(axis=1).astype(np.int32)
    offsets = np.zeros(B + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(counts)
    idx_rows, idx_t = np.nonzero(ev)          # row-major => ascending t within each row
    slot_of = np.full((B, T), -1, dtype=np.int32)
    rank = np.arange(len(idx_t)) - offsets[idx_rows]
    slot_of[idx_rows, idx_t] = rank
    return dict(counts=counts, offsets=offsets.astype(np.int32), indices=idx_t.astype(np.int32),
                rows=idx_rows.astype(np.int32), slot_of=slot_of,
                total=int(offsets[-1]), kmax=int(counts.max()) if B else 0)


def event_index_scalar(mask, rule="gt_half"):
    """Pure-Python loop version (independent of numpy's nonzero/cumsum) for pinning."""
    ev = event_bool(mask, rule)
    B, T = ev.shape
    counts, offsets, indices, rows = [], [0], [], []
    slot_of = [[-1] * T for _ in range(B)]
    for b in range(B):
        c = 0
        for t in range(T):
            if ev[b, t]:
                slot_of[b][t] = c
                indices.append(t)
                rows.append(b)
                c += 1
        counts.append(c)
        offsets.append(offsets[-1] + c)
    return dict(counts=np.array(counts, np.int32), offsets=np.array(offsets, np.int32),
                indices=np.array(indices, np.int32), rows=np.array(rows, np.int32),
                slot_of=np.array(slot_of, np.int32).reshape(B, T), total=offsets[-1],
                kmax=max(counts) if counts else 0)


def gather_padded(states, index, K):
    """(B, T, ...) -> (B, K, ...): event rows in ascending order, zero rows past count."""
    states = np.asarray(states)
    B = states.shape[0]
    out = np.zeros((B, K) + states.shape[2:], dtype=states.dtype)
    for b in range(B):
        o, c = index["offsets"][b], index["counts"][b]
        k = min(int(c), K)
        if k:
            out[b, :k] = states[b, index["indices"][o:o + k]]
    return out


def pad_mask(index, K):
    return (np.arange(K)[None, :] < index["counts"][:, None]).astype(np.float32)


def gather_packed(states, index):
    states = np.asarray(states)
    return states[index["rows"], index["indices"]]


def scatter(base, upd_padded, index):
    """out = base; out[b, t] = upd[b, slot_of[b,t]] for 0 <= slot < K."""
    out = np.array(base, copy=True)
    K = upd_padded.shape[1]
    b, t = np.nonzero((index["slot_of"] >= 0) & (index["slot_of"] < K))
    out[b, t] = upd_padded[b, index["slot_of"][b, t]]
    return out


def scatter_packed(base, packed, index):
    out = np.array(base, copy=True)
    out[index["rows"], index["indices"]] = packed
    return out


def naive_sparse_event_attention(states, event_mask, attn_fn, max_events=None):
    """Restates sparse_event_attn.py:35-86 with numpy arrays and a numpy attn_fn."""
    states = np.asarray(states)
    B, T = states.shape[:2]
    if max_events is None:
        max_events = int(np.asarray(event_mask, np.float64).sum(axis=1).max())   # :56
    K = max(max_events, 1)                                                      # :57
    idx = event_index(event_mask, rule="nonzero")
    ev = gather_padded(states, idx, K)
    upd = attn_fn(ev.reshape((B * K,) + states.shape[2:])).reshape(ev.shape)
    return scatter(states, upd, idx)


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

def _softmax_rows(s):
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    return e / e.sum(axis=-1, keepdims=True)


def track_causal_attention(q, k, v, index, scale=None):
    """q, k, v: (tracks, T, H, dh) (any float dtype, upcast to float64).
    Returns packed O (total, H, dh) float64: for each track, causal attention among its
    event rows in ascending order."""
    q, k, v = (np.asarray(t) for t in (q, k, v))
    rows, ts = index["rows"], index["indices"]
    return track_causal_attention_packed(q[rows, ts], k[rows, ts], v[rows, ts], index["offsets"], scale)


def track_causal_attention_packed(qp, kp, vp, offsets, scale=None):
    """The same on packed event rows: qp, kp, vp (total, H, dh), track b owning rows
    offsets[b] .. offsets[b+1]-1 in ascending t (the gather_packed order)."""
    q = np.asarray(qp, np.float64)
    k = np.asarray(kp, np.float64)
    v = np.asarray(vp, np.float64)
    total, H, dh = q.shape
    if scale is None:
        scale = dh ** -0.5
    out = np.zeros((total, H, dh))
    for b in range(len(offsets) - 1):
        o, c = int(offsets[b]), int(offsets[b + 1]) - int(offsets[b])
        if c == 0:
            continue
        Q, Kk, V = q[o:o + c], k[o:o + c], v[o:o + c]      # (c, H, dh)
        causal = np.tril(np.ones((c, c), bool))
        for h in range(H):
            s = Q[:, h] @ Kk[:, h].T * scale               # (c, c)
            s = np.where(causal, s, -np.inf)
            out[o:o + c, h] = _softmax_rows(s) @ V[:, h]
    return out


def slots_attention(q, k, v, key_pad=None, scale=None):
    """q, k, v: (P, N, H, dh); key_pad: (P, N) bool, True = ignore this key (the
    key_padding_mask convention of nn.MultiheadAttention).  Returns (P, N, H, dh) float64.
    A row whose keys are all padded gives NaN, as softmax over all -inf does."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    P, N, H, dh = q.shape
    if scale is None:
        scale = dh ** -0.5
    s = np.einsum("pihd,pjhd->phij", q, k) * scale
    if key_pad is not None:
        s = np.where(np.asarray(key_pad, bool)[:, None, None, :], -np.inf, s)
    with np.errstate(invalid="ignore"):
        p = _softmax_rows(s)
    return np.einsum("phij,pjhd->pihd", p, v)
