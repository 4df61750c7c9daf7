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


def test_level1_padded_forward_is_native():
    """Level1EventDynamics.forward -- the reference's padded call (model.py:302, level1_event.py:85-133) -- runs
    without autograd as one hclsm_level1_forward call over every (b, k) of the padded batch: no
    HipFallbackWarning, the oracle's values (fp32 at 1e-5; bf16 autocast at 2e-2), a padded event exactly zero.
    Under autograd it warns.  The HierarchyManager says why it leaves its fused step for non-fp32 states."""
    from hclsm_amd.dynamics import HierarchyManager, Level1EventDynamics
    from hclsm_amd.kernels import HipFallbackWarning
    from oracle import modules as om
    from oracle.ssm_scan import normwise_rel_err
    _reset()
    torch.manual_seed(3)
    cfg = SimpleNamespace(d_model=256, n_layers=2, n_heads=4)
    l1 = Level1EventDynamics(cfg, 128).cuda()
    B, K, N, D = 2, 3, 16, 128
    x = torch.randn(B, K, N, D, device="cuda")
    pad = torch.ones(B, K, device="cuda")
    pad[1, 2] = 0.0
    obj = torch.ones(B, N, device="cuda")
    obj[0, 11:] = 0.0
    sd = {k: v.detach().double().cpu().numpy() for k, v in l1.state_dict().items()}
    ref = om.level1_ref(x.double().cpu().numpy(), pad.double().cpu().numpy(), obj.double().cpu().numpy(), sd,
                        cfg.n_layers, cfg.n_heads)
    out = _silent(lambda: l1(x, pad, obj))
    assert out.shape == (B, K, N, D) and out.dtype == torch.float32
    assert normwise_rel_err(out.double().cpu().numpy(), ref) <= 1e-5
    assert out[1, 2].abs().sum() == 0

    def bf():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            return l1(x, pad, obj)
    out_bf = _silent(bf)
    assert normwise_rel_err(out_bf.double().cpu().numpy(), ref) <= 2e-2
    with pytest.warns(HipFallbackWarning, match="Level1EventDynamics.forward"):
        l1(x.requires_grad_(), pad, obj)
    hm = HierarchyManager(D, 384).cuda()
    mask = torch.zeros(B, 6, device="cuda")
    mask[:, 1] = 1
    with torch.no_grad(), pytest.warns(HipFallbackWarning, match="HierarchyManager"):
        hm(torch.randn(B, 6, N, D, device="cuda").half(), torch.randn(B, 1, N, D, device="cuda").half(), None,
           mask)
