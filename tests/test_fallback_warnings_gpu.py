"""The object- and dynamics-layer modules say when a call runs torch ops instead of their HIP kernels:
a HipFallbackWarning under autograd (none of the fused forwards has a backward) and for shapes outside
the kernels; the no-grad calls inside the kernels' shapes warn nothing."""

from __future__ import annotations

import warnings
from types import SimpleNamespace

import pytest
import torch

pytestmark = pytest.mark.gpu


def _reset():
    from hclsm_amd.kernels import _common
    _common._WARNED.clear()


def _silent(fn):
    with torch.no_grad(), warnings.catch_warnings():
        warnings.simplefilter("error")
        return fn()


def test_relation_graph():
    from hclsm_amd.kernels import HipFallbackWarning
    from hclsm_amd.objects import RelationGraph
    _reset()
    m = RelationGraph(SimpleNamespace(d_slot=64, d_edge=32, gnn_rounds=1, n_max_slots=8)).cuda()
    x, alive = torch.randn(2, 8, 64, device="cuda"), torch.ones(2, 8, device="cuda")
    _silent(lambda: m(x, alive))
    with pytest.warns(HipFallbackWarning, match="autograd"):
        m(x.requires_grad_(), alive)
    odd = RelationGraph(SimpleNamespace(d_slot=48, d_edge=24, gnn_rounds=1, n_max_slots=8)).cuda()
    with torch.no_grad(), pytest.warns(HipFallbackWarning, match="shape outside"):
        odd(torch.randn(2, 8, 48, device="cuda"), alive)


def test_slot_tracker():
    from hclsm_amd.kernels import HipFallbackWarning
    from hclsm_amd.objects import SlotTracker
    _reset()
    m = SlotTracker(SimpleNamespace(d_slot=64, n_max_slots=8)).cuda()
    a, b = torch.randn(2, 8, 64, device="cuda"), torch.randn(2, 8, 64, device="cuda")
    al = torch.ones(2, 8, device="cuda")
    _silent(lambda: m(a, b, al, al))
    with pytest.warns(HipFallbackWarning, match="autograd"):
        m(a.requires_grad_(), b, al, al)


def test_dynamic_slots():
    from hclsm_amd.kernels import HipFallbackWarning
    from hclsm_amd.objects import DynamicSlotAttention
    _reset()
    cfg = SimpleNamespace(d_slot=128, n_max_slots=16, n_iterations=2, existence_threshold=0.5, birth_threshold=0.7)
    m = DynamicSlotAttention(cfg, 256).cuda()
    x = torch.randn(2, 50, 256, device="cuda")
    _silent(lambda: m(x))
    with pytest.warns(HipFallbackWarning, match="autograd"):
        m(x)


def test_level1_packed_and_top_down():
    from hclsm_amd.dynamics import HierarchyManager, Level1EventDynamics
    from hclsm_amd.kernels import HipFallbackWarning
    _reset()
    D = 128
    hm = HierarchyManager(D, 384).cuda()
    l1 = Level1EventDynamics(SimpleNamespace(d_model=256, n_layers=1, n_heads=4), D).cuda()
    states = torch.randn(2, 6, 8, D, device="cuda")
    mask = torch.zeros(2, 6, device="cuda")
    mask[:, 1] = 1
    mask[:, 4] = 1

    def run():
        ev, idx = hm.gather_events_packed(states, mask)
        out = l1.forward_packed(ev, idx)
        return hm.forward_packed(states, out, idx, torch.randn(2, 4, 384, device="cuda"))
    _silent(run)
    with pytest.warns(HipFallbackWarning) as rec:
        run()
    msgs = " ".join(str(w.message) for w in rec)
    assert "Level1EventDynamics.forward_packed" in msgs and "HierarchyManager" in msgs
