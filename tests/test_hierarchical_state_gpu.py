"""GPU checks of hclsm_amd.kernels.hierarchical_state against a float64 CPU restatement of the reference's
steps (hclsm/kernels/hierarchical_state.py:25-221) with the same callables.

The callables are the reference's roles built from this package's kernels: gather_fn = the padded event gather
(ascending t), level1_fn / level2_fn = elementwise and reducing maps that depend on the event order and on the
pad mask, scatter_fn = an additive combine.  The fused and streamed forms gather the events themselves in
descending score order (the reference's topk(sorted=True)); the restatement sorts the same way (ties by
ascending t).  Comparisons: gathered rows and masks bit-exact; float outputs within 1e-6 (fp32)."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(B=5, T=24, N=3, D=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    level0 = torch.randn(B, T, N, D, generator=g)
    scores = torch.rand(B, T, generator=g)
    scores[1] = 0.0                               # a row with no event
    scores[2, 3] = scores[2, 7] = 0.9             # a tie: ascending t breaks it
    return level0, scores


def _callables():
    def gather_fn(states, mask):
        from hclsm_amd.dynamics import HierarchyManager
        return HierarchyManager(states.shape[-1], 4).to(states.device).gather_events(states, mask)

    def level1_fn(ev, pad):
        k = torch.arange(ev.shape[1], device=ev.device, dtype=ev.dtype)[None, :, None, None]
        return (ev * 2.0 + k) * pad.to(ev.dtype)[:, :, None, None]   # depends on the event order

    def level2_fn(ev, pad):
        w = pad.to(ev.dtype)[:, :, None, None]
        return (ev * w).sum(dim=1) / w.sum(dim=1).clamp(min=1.0)       # (B, N, D)

    def scatter_fn(level0, l1, l2, mask):
        return level0 + l2[:, None] + mask[:, :, None, None] * l1.sum(dim=1, keepdim=True)

    return gather_fn, level1_fn, level2_fn, scatter_fn


def _reference(level0, scores, thr, order):
    """The reference's steps on CPU float64 tensors; order "time" (a gather_fn over ascending t) or "score"."""
    level0 = level0.double()
    mask = (scores > thr).double()
    B, T = mask.shape
    K = max(int(mask.sum(1).max()), 1)
    ev = torch.zeros((B, K) + tuple(level0.shape[2:]), dtype=torch.float64)
    pad = torch.zeros(B, K, dtype=torch.bool)
    for b in range(B):
        ts = [t for t in range(T) if mask[b, t] > 0]
        if order == "score":
            ts = sorted(ts, key=lambda t: (-float(scores[b, t]), t))
        for k, t in enumerate(ts):
            ev[b, k] = level0[b, t]
            pad[b, k] = True
    _, l1f, l2f, scf = _callables()
    l1 = l1f(ev, pad)
    l2 = l2f(ev, pad)
    return scf(level0, l1, l2, mask), mask, l1, l2, ev, pad


@pytest.mark.parametrize("backend", ["naive", "fused", "streamed", "auto"])
def test_forms_match_the_restatement(backend):
    from hclsm_amd.kernels import hierarchical_state_fn
    level0, scores = _case()
    thr = 0.55
    got = hierarchical_state_fn(level0.cuda(), scores.cuda(), thr, *_callables(), backend=backend)
    torch.cuda.synchronize()
    order = "time" if backend == "naive" else "score"
    want = _reference(level0, scores, thr, order)
    for g, w in zip(got, want[:4]):
        assert g.shape == w.shape
        torch.testing.assert_close(g.double().cpu(), w, rtol=1e-6, atol=1e-6)


def test_score_ordered_gather_is_bit_exact():
    from hclsm_amd.kernels.hierarchical_state import _gather_by_score
    level0, scores = _case(B=7, T=40, N=4, D=6, seed=3)
    mask = (scores > 0.3).float()
    ev, pad = _gather_by_score(level0.cuda(), scores.cuda(), mask.cuda())
    _, _, _, _, ev_ref, pad_ref = _reference(level0, scores, 0.3, "score")
    assert torch.equal(pad.cpu(), pad_ref)
    assert torch.equal(ev.cpu(), ev_ref.float())             # byte moves; pads exact zeros


def test_shape_mismatch_raises():
    from hclsm_amd.kernels import hierarchical_state_fused
    level0, scores = _case()
    with pytest.raises(ValueError):
        hierarchical_state_fused(level0[:, :-1].cuda(), scores.cuda(), 0.5, *_callables())
