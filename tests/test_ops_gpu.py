"""torch.library ops (namespace hclsm_hip) on the GPU: each op returns what the eager function
of hclsm_amd.kernels returns (same kernels, bit for bit) and passes torch.library.opcheck's
schema and fake-tensor checks."""

from __future__ import annotations

import pytest
import torch

import hclsm_amd.kernels.ops as hops

pytestmark = pytest.mark.gpu
OPS = torch.ops.hclsm_hip


def test_scan_ops_equal_eager():
    from hclsm_amd.kernels import ssm_scan_fn
    from hclsm_amd.kernels.ssm_scan_bwd import scan_backward
    from hclsm_amd.workloads import scan_inputs
    d = {k: v.cuda() for k, v in scan_inputs(3, 20, 64, 16, dtype=torch.bfloat16, seed=2).items()}
    args = (d["x"], d["dt"], d["A_log"], d["B"], d["C"])
    y, h = OPS.ssm_scan_fwd(*args, d["D"], 0, True)
    ye, he = ssm_scan_fn(*args, backend="hip", D=d["D"], return_h_final=True)
    assert torch.equal(y, ye) and torch.equal(h, he)
    gy = torch.randn_like(y)
    g = OPS.ssm_scan_bwd(*args, d["D"], gy, 1)
    ge = scan_backward(*args, d["D"], gy, 1)
    for t, n in zip(g, ("x", "dt", "A_log", "B", "C", "D")):
        assert torch.equal(t, ge[n]), n
    torch.library.opcheck(OPS.ssm_scan_fwd.default, (*args, d["D"], 0, True), test_utils=("test_schema", "test_faketensor"))


def test_event_ops_equal_eager():
    from hclsm_amd.kernels.event_attention import event_attention
    from hclsm_amd.kernels.sparse_event_attn import build_event_index, gather_events_padded, scatter_events_padded
    g = torch.Generator().manual_seed(4)
    m = (torch.rand(6, 21, generator=g) < 0.3).float().cuda()
    idx = build_event_index(m)
    t = OPS.event_index(m, 0)
    n = idx.total()
    for a, b in zip(t, (idx.counts, idx.offsets, idx.indices[:n], idx.rows[:n], idx.slot_of, idx.stats)):
        assert torch.equal(a[: b.numel()] if a.dim() == 1 else a, b)   # entries past the total are unused
    K = max(idx.kmax(), 1)
    st = torch.randn(6, 21, 3, 8, generator=g).cuda()
    gp = OPS.event_gather(st, t[0], t[1], t[2], K)
    assert torch.equal(gp, gather_events_padded(st, idx, K))
    upd = torch.randn(6, K, 3, 8, generator=g).cuda()
    assert torch.equal(OPS.event_scatter(st, upd, t[4]), scatter_events_padded(st, upd, idx))
    q, k, v = (torch.randn(6, 21, 2, 32, generator=g).to(torch.bfloat16).cuda() for _ in range(3))
    tot = idx.total()
    o = OPS.event_attention(q, k, v, t[1], t[2], None, 32 ** -0.5, 0, tot)
    assert torch.equal(o, event_attention(q, k, v, idx, capacity=tot))
    torch.library.opcheck(OPS.event_gather.default, (st, t[0], t[1], t[2], K), test_utils=("test_schema", "test_faketensor"))


def test_slot_ops_equal_eager():
    from hclsm_amd.kernels import naive_slot_attention
    from hclsm_amd.kernels import slot_iteration as si
    from hclsm_amd.workloads import slot_config
    g = torch.Generator().manual_seed(6)
    Q, K, V = (torch.randn(s, generator=g).cuda() for s in ((2, 8, 64), (2, 40, 64), (2, 40, 64)))
    out, attn = OPS.slot_attn_core(Q, K, V, 0.125, 0.0, 0.0, -1.0)
    oe, ae = naive_slot_attention(Q, K, V, scale=0.125)
    assert torch.equal(out, oe) and torch.equal(attn, ae)
    tokens, slots0, w = slot_config(B=2)
    ws = [w[n].cuda() for n in hops.SLOT_WEIGHT_ORDER]
    s = OPS.slot_attention_forward(tokens.cuda(), slots0.cuda(), ws, 3, 384 ** -0.5, 0.0, 1e-8, 0.0, torch.bfloat16)
    W = si.SlotWeights.from_dict(w, torch.bfloat16)
    assert torch.equal(s, si.slot_attention_forward(tokens.cuda(), slots0.cuda(), W, 3, si.CONFIG2_MODE))
    torch.library.opcheck(OPS.slot_attn_core.default, (Q, K, V, 0.125, 0.0, 0.0, -1.0),
                          test_utils=("test_schema", "test_faketensor"))


def test_block_scan_op_equals_eager():
    from hclsm_amd.kernels import ssm_block_scan
    g = torch.Generator().manual_seed(8)
    z, dt_in, gate = (torch.randn(2, 16, 64, generator=g).to(torch.bfloat16).cuda() for _ in range(3))
    A_log = (-torch.rand(64, 16, generator=g) * 0.5).cuda()
    Bm, Cm = (torch.randn(2, 16, 16, generator=g).to(torch.bfloat16).cuda() for _ in range(2))
    y, y_pre = OPS.ssm_block_scan_fwd(z, dt_in, A_log, Bm, Cm, gate)
    assert torch.equal(y, ssm_block_scan(z, dt_in, A_log, Bm, Cm, gate))
    assert torch.allclose(y.float(), (y_pre.float() * torch.nn.functional.silu(gate.float())), rtol=1e-2, atol=1e-2)


def test_packed_level1_ops_equal_eager():
    """hclsm_hip::event_gather_packed / level1_forward / event_scatter_packed against the eager packed
    path, and opcheck of their schemas and fake kernels."""
    from types import SimpleNamespace
    from hclsm_amd.dynamics import HierarchyManager, Level1EventDynamics
    from hclsm_amd.kernels.level1_packed import Level1Weights
    torch.manual_seed(12)
    B, T, N, D = 3, 9, 8, 64
    hm = HierarchyManager(D, 96).cuda()
    l1 = Level1EventDynamics(SimpleNamespace(d_model=64, n_layers=2, n_heads=4), D).cuda()
    g = torch.Generator().manual_seed(13)
    states = torch.randn(B, T, N, D, generator=g).cuda()
    mask = (torch.rand(B, T, generator=g) < 0.4).float().cuda()
    obj = torch.ones(B, N, device="cuda")
    obj[0, 5:] = 0.0
    with torch.no_grad():
        ev, idx = hm.gather_events_packed(states, mask)
        want = l1.forward_packed(ev, idx, obj)
        t = OPS.event_index(mask, 0)
        evo = OPS.event_gather_packed(states, t[3], t[2], t[5])
        n = idx.total()
        # live rows equal; the op zero-fills the rest (the eager gather does so only in grad mode)
        assert torch.equal(evo[:n], ev[:n]) and evo[n:].abs().sum() == 0
        W = Level1Weights.from_module(l1, torch.float32)
        got = OPS.level1_forward(evo, t[5], t[3], obj, W.tensors, 4, W.ln_eps, torch.float32)
        assert torch.equal(got[:n], want[:n]) and got[n:].abs().sum() == 0
        comb = OPS.event_scatter_packed(states, got, t[1], t[4])
        assert torch.equal(comb, hm.forward_packed(states, want, idx))
        # the whole output step: against the module's fused call, and the padded-row form
        l2 = torch.randn(B, 3, 96, generator=g).cuda()
        td_params = [p.detach() for p in (hm.l2_to_l1.weight, hm.gate_l2_l0[0].weight, hm.gate_l2_l0[0].bias)]
        td = OPS.event_top_down(states, got, t[1], t[4], 0, l2, obj, td_params, torch.float32)
        assert torch.equal(td, hm.forward_packed(states, got, idx, l2, obj))
    torch.library.opcheck(OPS.event_top_down.default,
                          (states, got, t[1], t[4], 0, l2, obj, td_params, torch.float32),
                          test_utils=("test_schema", "test_faketensor"))
    torch.library.opcheck(OPS.event_gather_packed.default, (states, t[3], t[2], t[5]),
                          test_utils=("test_schema", "test_faketensor"))
    torch.library.opcheck(OPS.level1_forward.default, (evo, t[5], t[3], obj, W.tensors, 4, W.ln_eps, torch.float32),
                          test_utils=("test_schema", "test_faketensor"))


def test_object_layer_ops_equal_eager():
    """hclsm_hip::relation_graph_forward / slot_track_sequence against the module calls, and opcheck of their
    schemas and fake kernels."""
    from types import SimpleNamespace
    from hclsm_amd.objects import RelationGraph, SlotTracker
    torch.manual_seed(14)
    cfg = SimpleNamespace(d_slot=64, d_edge=32, gnn_rounds=2, n_max_slots=16)
    rg, trk = RelationGraph(cfg).cuda(), SlotTracker(cfg).cuda()
    g = torch.Generator().manual_seed(15)
    nodes = torch.randn(4, 16, 64, generator=g).cuda()
    alive = (torch.rand(4, 16, generator=g) > 0.25).float().cuda()
    slots = torch.randn(2, 5, 16, 64, generator=g).cuda()
    salive = (torch.rand(2, 5, 16, generator=g) > 0.2).float().cuda()
    gp = [p.detach() for p in rg.state_dict().values()]
    tp = [p.detach() for p in trk.state_dict().values()]
    with torch.no_grad():
        wn, wc = rg(nodes, alive)
        gn, gc = OPS.relation_graph_forward(nodes, alive, gp, 2, False, rg.pair_norm.eps, torch.float32)
        assert torch.equal(gn, wn) and torch.equal(gc, wc)
        wt, wa, wh = trk.track(slots, salive, return_hidden=True)
        t, a, p, mt, h = OPS.slot_track_sequence(slots, salive, tp, True, 20, 0.05, torch.float32)
        assert torch.equal(t, wt) and torch.equal(a, wa) and torch.equal(h, wh)
        assert torch.equal(torch.gather(slots, 2, p[..., None].expand_as(slots)), t)
    torch.library.opcheck(OPS.relation_graph_forward.default, (nodes, alive, gp, 2, False, 1e-5, torch.float32),
                          test_utils=("test_schema", "test_faketensor"))
    torch.library.opcheck(OPS.slot_track_sequence.default, (slots, salive, tp, True, 20, 0.05, torch.float32),
                          test_utils=("test_schema", "test_faketensor"))
