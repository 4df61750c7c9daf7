"""GPU tests of the module counterparts (hclsm_amd.dynamics / hclsm_amd.objects).

Ports of the reference's tests/test_dynamics.py:21-116 and tests/test_objects.py:20-41 (same
shapes, the tiny config of hclsm/config.py:193-212), plus parity against oracle/modules.py and
the slot-attention oracle (fp32: normwise 1e-5 relative) and gradient checks against float64
torch autograd of the same modules' math on the CPU."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import modules as om
from oracle import slot_attention as sa
from oracle.ssm_scan import normwise_rel_err

pytestmark = pytest.mark.gpu

# HCLSMConfig.tiny() (reference hclsm/config.py:193-212 with dataclass defaults :31-59)
TINY = SimpleNamespace(
    d_world=256,
    objects=SimpleNamespace(d_slot=128, n_max_slots=16, n_iterations=3, existence_threshold=0.5, birth_threshold=0.7),
    level0=SimpleNamespace(d_state=32, n_blocks=2, expand_ratio=2),
    level1=SimpleNamespace(d_model=256, n_layers=2, n_heads=4),
    level2_d_model=384,
)
D_SLOT = TINY.objects.d_slot


def _np(t):
    return t.detach().double().cpu().numpy()


def _sd(m):
    return {k: _np(v) for k, v in m.state_dict().items()}


# ---------------------------------------------------------------- Level 0 (test_dynamics.py:21-45)

def test_level0_output_shape_and_oracle():
    from hclsm_amd.dynamics import Level0SSM
    torch.manual_seed(0)
    ssm = Level0SSM(TINY.level0, D_SLOT).cuda()
    B, N, T, D = 2, 16, 8, D_SLOT
    x = torch.randn(B, N, T, D, device="cuda")
    mask = torch.ones(B, N, device="cuda")
    mask[1, 5:] = 0.0
    with torch.no_grad():
        out = ssm(x, mask)
    assert out.shape == (B, N, T, D)
    ref = om.level0_ssm_ref(_np(x), _np(mask), _sd(ssm), TINY.level0.n_blocks)
    assert normwise_rel_err(_np(out), ref) <= 1e-5


def test_level0_dead_objects_masked():
    from hclsm_amd.dynamics import Level0SSM
    ssm = Level0SSM(TINY.level0, D_SLOT).cuda()
    x = torch.randn(2, 16, 4, D_SLOT, device="cuda")
    mask = torch.zeros(2, 16, device="cuda")
    mask[:, :3] = 1.0
    out = ssm(x, mask)
    assert out[:, 3:].abs().sum() < 1e-5


def _block_math_f64(blk, x):
    """float64 autograd of the same block on the CPU: sequential clamped scan (level0_ssm.py:82-101)."""
    p = {k: v.detach().double().cpu().requires_grad_() for k, v in blk.named_parameters()}
    h = F.layer_norm(x, (x.shape[-1],), p["norm.weight"], p["norm.bias"])
    z = h @ p["in_proj.weight"].T
    gate = F.silu(h @ p["gate_proj.weight"].T)
    dt = F.softplus(z @ p["dt_proj.weight"].T + p["dt_proj.bias"]).clamp(1e-3, 1.0)
    Bm, Cm = z @ p["B_proj.weight"].T, z @ p["C_proj.weight"].T
    A = -torch.exp(p["A_log"]).clamp(1e-6, 1.0)
    st = torch.zeros(x.shape[0], z.shape[-1], Bm.shape[-1], dtype=torch.float64)
    ys = []
    for t in range(x.shape[1]):
        dA = torch.exp((dt[:, t, :, None] * A).clamp(-20.0, 0.0))
        st = st * dA + (dt[:, t] * z[:, t])[:, :, None] * Bm[:, t, None, :]
        ys.append((st * Cm[:, t, None, :]).sum(-1))
    y = torch.stack(ys, 1)
    return x + (y * gate) @ p["out_proj.weight"].T, p


def test_ssm_block_gradients_match_float64_autograd():
    from hclsm_amd.dynamics import SimplifiedSSMBlock
    torch.manual_seed(3)
    blk = SimplifiedSSMBlock(32, 16).cuda()
    x = torch.randn(3, 24, 32)
    w = torch.randn(3, 24, 32)
    xg = x.cuda().requires_grad_()
    (blk(xg) * w.cuda()).sum().backward()
    x64 = x.double().requires_grad_()
    out64, p64 = _block_math_f64(blk, x64)
    (out64 * w.double()).sum().backward()
    assert normwise_rel_err(_np(blk(x.cuda())), _np(out64)) <= 1e-5
    assert normwise_rel_err(_np(xg.grad), _np(x64.grad)) <= 1e-5
    for name, prm in blk.named_parameters():
        assert normwise_rel_err(_np(prm.grad), _np(p64[name].grad)) <= 1e-5, name


def test_level0_gradient_flow():
    from hclsm_amd.dynamics import Level0SSM
    ssm = Level0SSM(TINY.level0, D_SLOT).cuda()
    x = torch.randn(1, 4, 4, D_SLOT, device="cuda", requires_grad=True)
    out = ssm(x, torch.ones(1, 4, device="cuda"))
    out.sum().backward()
    assert x.grad is not None and torch.isfinite(x.grad).all()


# ---------------------------------------------------------------- event mask rule

def test_event_mask_rule_matches_oracle_and_straight_through():
    from hclsm_amd.dynamics import event_mask_rule
    g = torch.Generator().manual_seed(5)
    tl = torch.tensor(0.4)
    for probs in (torch.rand(4, 9, generator=g), torch.rand(3, 7, generator=g) * 0.3):
        pc = probs.cuda().requires_grad_()
        m = event_mask_rule(pc, tl.cuda())
        np.testing.assert_allclose(_np(m), om.event_mask_rule_ref(_np(probs), 0.4), atol=1e-6)
        m.sum().backward()
        assert torch.allclose(pc.grad[:, 1:], torch.ones_like(pc.grad[:, 1:]))


def test_at_least_one_event():
    """test_dynamics.py:56-61: threshold 0.99 on zero features -> every row still has an event."""
    from hclsm_amd.dynamics import event_mask_rule
    probs = torch.full((2, 8), 0.5, device="cuda")
    mask = event_mask_rule(probs, torch.logit(torch.tensor(0.99, device="cuda")))
    assert mask.sum(dim=1).min() >= 1


# ---------------------------------------------------------------- Level 1 (test_dynamics.py:64-72)

def test_level1_shape_and_oracle():
    from hclsm_amd.dynamics import Level1EventDynamics
    torch.manual_seed(1)
    l1 = Level1EventDynamics(TINY.level1, D_SLOT).cuda()
    B, K, N, D = 2, 3, 16, D_SLOT
    x = torch.randn(B, K, N, D, device="cuda")
    pad = torch.ones(B, K, device="cuda")
    pad[1, 2] = 0.0
    obj = torch.ones(B, N, device="cuda")
    obj[0, 11:] = 0.0
    with torch.no_grad():
        out = l1(x, pad, obj)
    assert out.shape == (B, K, N, D)
    ref = om.level1_ref(_np(x), _np(pad), _np(obj), _sd(l1), TINY.level1.n_layers, TINY.level1.n_heads)
    assert normwise_rel_err(_np(out), ref) <= 1e-5
    assert out[1, 2].abs().sum() == 0


def test_event_block_matches_multihead_attention_with_grads():
    """The block's attention (HIP kernel forward, torch backward) against nn.MultiheadAttention
    with the same weights, forward and gradients, key padding included."""
    from hclsm_amd.dynamics import EventTransformerBlock
    torch.manual_seed(2)
    blk = EventTransformerBlock(64, 4).cuda()
    x = torch.randn(6, 10, 64, device="cuda")
    kp = torch.rand(6, 10, device="cuda") < 0.3
    kp[:, 0] = False
    w = torch.randn(6, 10, 64, device="cuda")
    xa = x.clone().requires_grad_()
    (blk(xa, kp) * w).sum().backward()
    ga = {n: p.grad.clone() for n, p in blk.named_parameters()}
    blk.zero_grad()
    xb = x.clone().requires_grad_()
    h = blk.norm1(xb)
    a, _ = blk.attn(h, h, h, key_padding_mask=kp, need_weights=False)
    y = xb + a
    y = y + blk.ffn(blk.norm2(y))
    (y * w).sum().backward()
    assert normwise_rel_err(_np(blk(x, kp)), _np(y)) <= 1e-5
    assert normwise_rel_err(_np(xa.grad), _np(xb.grad)) <= 1e-5
    for n, p in blk.named_parameters():
        assert normwise_rel_err(_np(ga[n]), _np(p.grad)) <= 1e-5, n


# ---------------------------------------------------------------- hierarchy manager (test_dynamics.py:90-116)

def test_gather_scatter_roundtrip():
    from hclsm_amd.dynamics import HierarchyManager
    hm = HierarchyManager(D_SLOT, TINY.level2_d_model).cuda()
    B, T, N, D = 2, 8, 16, D_SLOT
    states = torch.randn(B, T, N, D, device="cuda")
    em = torch.zeros(B, T, device="cuda")
    em[:, 2] = 1.0
    em[:, 5] = 1.0
    gathered, pad, K = hm.gather_events(states, em)
    assert gathered.shape[1] == K and K == 2
    assert torch.equal(gathered, states[:, [2, 5]])
    assert torch.equal(pad, torch.ones(B, 2, device="cuda"))
    back = hm.scatter_events(torch.zeros_like(states), gathered, em)
    assert torch.equal(back[:, [2, 5]], states[:, [2, 5]]) and back[:, [0, 1, 3, 4, 6, 7]].abs().sum() == 0


def test_ragged_gather_scatter_matches_oracle():
    from hclsm_amd.dynamics import HierarchyManager
    from oracle import events as oe
    hm = HierarchyManager(32, 48).cuda()
    g = torch.Generator().manual_seed(4)
    B, T, N, D = 3, 11, 5, 32
    states = torch.randn(B, T, N, D, generator=g)
    em = (torch.rand(B, T, generator=g) > 0.6).float()
    em[2] = 0.0
    ev, pad, K = hm.gather_events(states.cuda(), em.cuda())
    index = oe.event_index(em.numpy(), "gt_half")
    Kr = max(int(index["counts"].max()), 1)
    assert K == Kr
    np.testing.assert_array_equal(ev.cpu().numpy(), oe.gather_padded(states.numpy(), index, K))
    np.testing.assert_array_equal(pad.cpu().numpy(), oe.pad_mask(index, K))
    upd = torch.randn(B, K, N, D, generator=g)
    out = hm.scatter_events(states.cuda(), upd.cuda(), em.cuda())
    np.testing.assert_array_equal(out.cpu().numpy(), oe.scatter(states.numpy(), upd.numpy(), index))


def test_gating_range():
    from hclsm_amd.dynamics import HierarchyManager
    hm = HierarchyManager(D_SLOT, TINY.level2_d_model).cuda()
    B, T, N, D = 2, 8, 16, D_SLOT
    l0 = torch.randn(B, T, N, D, device="cuda")
    l1 = torch.randn(B, 2, N, D, device="cuda")
    l2 = torch.randn(B, 8, TINY.level2_d_model, device="cuda")
    em = torch.zeros(B, T, device="cuda")
    em[:, 0] = 1.0
    em[:, 4] = 1.0
    out = hm(l0, l1, l2, em)
    assert out.shape == (B, T, N, D) and torch.isfinite(out).all()


# ---------------------------------------------------------------- DynamicSlotAttention (test_objects.py:20-41)

def test_dynamic_slots_shapes_and_alive_range():
    from hclsm_amd.objects import DynamicSlotAttention
    sa_m = DynamicSlotAttention(TINY.objects, TINY.d_world).cuda()
    slots, alive = sa_m(torch.randn(4, 196, TINY.d_world, device="cuda"))
    assert slots.shape == (4, 16, D_SLOT) and alive.shape == (4, 16)
    _, alive = sa_m(torch.randn(2, 196, TINY.d_world, device="cuda"))
    assert alive.min() >= 0.0 and alive.max() <= 1.0


def test_dynamic_slots_gradient_flow():
    from hclsm_amd.objects import DynamicSlotAttention
    sa_m = DynamicSlotAttention(TINY.objects, TINY.d_world).cuda()
    slots, alive = sa_m(torch.randn(2, 50, TINY.d_world, device="cuda"))
    (slots.sum() + alive.sum()).backward()
    assert sa_m.slot_mu.grad is not None and torch.isfinite(sa_m.slot_mu.grad).all()


def test_dynamic_slots_fused_forward_matches_oracle_and_grad_path():
    """No-grad path (fused C entry) and autograd path (torch + HIP core) against the oracle's
    forward with the in-model semantics (logits clamped to +-30, slots to +-50, no renorm eps)."""
    from hclsm_amd.objects import DynamicSlotAttention
    torch.manual_seed(6)
    m = DynamicSlotAttention(TINY.objects, TINY.d_world).cuda()
    m.birth_threshold = 10.0            # birth off: compare the iterations alone
    x = torch.randn(3, 100, TINY.d_world, device="cuda")
    torch.manual_seed(7)
    with torch.no_grad():
        s_fused, a_fused = m(x)
    torch.manual_seed(7)
    s_grad, a_grad = m(x)
    torch.manual_seed(7)
    with torch.no_grad():
        slots0 = m._init_slots(3, "cuda")
    W = {"ln_in_w": m.norm_input.weight, "ln_in_b": m.norm_input.bias, "w_k": m.project_k.weight,
         "w_v": m.project_v.weight, "ln_pre_w": m.norm_pre_attn.weight, "ln_pre_b": m.norm_pre_attn.bias,
         "w_q": m.project_q.weight, "w_ih": m.gru.weight_ih, "w_hh": m.gru.weight_hh, "b_ih": m.gru.bias_ih,
         "b_hh": m.gru.bias_hh, "ln_mlp_w": m.norm_slots.weight, "ln_mlp_b": m.norm_slots.bias,
         "w1": m.mlp[0].weight, "b1": m.mlp[0].bias, "w2": m.mlp[2].weight, "b2": m.mlp[2].bias}
    ref = sa.slot_attention_forward(_np(x), _np(slots0), {k: _np(v) for k, v in W.items()}, 3,
                                    logit_clamp=30.0, renorm_eps=None, slot_clamp=50.0)
    assert normwise_rel_err(_np(s_fused), ref) <= 1e-5
    assert normwise_rel_err(_np(s_grad), ref) <= 1e-5
    assert normwise_rel_err(_np(a_fused), _np(a_grad)) <= 1e-5


def _dyn_weights(m):
    W = {"ln_in_w": m.norm_input.weight, "ln_in_b": m.norm_input.bias, "w_k": m.project_k.weight,
         "w_v": m.project_v.weight, "ln_pre_w": m.norm_pre_attn.weight, "ln_pre_b": m.norm_pre_attn.bias,
         "w_q": m.project_q.weight, "w_ih": m.gru.weight_ih, "w_hh": m.gru.weight_hh, "b_ih": m.gru.bias_ih,
         "b_hh": m.gru.bias_hh, "ln_mlp_w": m.norm_slots.weight, "ln_mlp_b": m.norm_slots.bias,
         "w1": m.mlp[0].weight, "b1": m.mlp[0].bias, "w2": m.mlp[2].weight, "b2": m.mlp[2].bias,
         "e1_w": m.existence_head[0].weight, "e1_b": m.existence_head[0].bias, "e2_w": m.existence_head[2].weight,
         "e2_b": m.existence_head[2].bias, "birth_w": m.birth_proj.weight, "birth_b": m.birth_proj.bias}
    return {k: _np(v) for k, v in W.items()}


@pytest.mark.parametrize("grad", [False, True])
def test_dynamic_slots_birth_matches_oracle(grad):
    """Slot birth (dynamic_slots.py:180-199) on, in the fused no-grad path and the autograd path, against
    oracle/slot_attention.py::dynamic_slots_forward_ref: one input token (the residual's argmax is token 0
    exactly), a birth threshold every clip exceeds, an existence threshold between two alive values of every
    clip (so some slots are dormant and the decision is far from rounding); then a threshold no residual
    reaches (the residual is rounding noise) leaves the slots as the iterations made them."""
    from hclsm_amd.objects import DynamicSlotAttention
    torch.manual_seed(31)
    m = DynamicSlotAttention(TINY.objects, TINY.d_world).cuda()
    x = torch.randn(4, 1, TINY.d_world, device="cuda")
    W = _dyn_weights(m)
    torch.manual_seed(32)
    with torch.no_grad():
        slots0 = m._init_slots(4, "cuda")
    _, alive_ref = sa.dynamic_slots_forward_ref(_np(x), _np(slots0), W, m.n_iterations, 0.0, 10.0)
    a = np.sort(alive_ref, axis=1)
    gaps = a[:, 1:] - a[:, :-1]
    k = int(np.argmax(gaps.min(axis=0)))              # the rank whose gap is widest in the worst clip
    thr = float(np.clip(0.5 * (a[:, k].max() + a[:, k + 1].min()), 1e-6, 1 - 1e-6))
    if not (a[:, k].max() + 1e-4 < thr < a[:, k + 1].min() - 1e-4):
        thr = float(np.median(alive_ref))
    m.existence_threshold = thr
    m.birth_threshold = -1.0
    ref, _ = sa.dynamic_slots_forward_ref(_np(x), _np(slots0), W, m.n_iterations, thr, -1.0)
    torch.manual_seed(32)
    with torch.set_grad_enabled(grad):
        s, alive = m(x)
    assert normwise_rel_err(_np(alive), alive_ref) <= 1e-5
    assert normwise_rel_err(_np(s), ref) <= 1e-5
    born = np.abs(ref - sa.dynamic_slots_forward_ref(_np(x), _np(slots0), W, m.n_iterations, thr, 10.0)[0])
    assert (born.max(axis=-1) > 1e-3).sum() >= 1     # at least one slot was born
    m.birth_threshold = 1e-3
    torch.manual_seed(32)
    with torch.set_grad_enabled(grad):
        s2, _ = m(torch.randn(4, 9, TINY.d_world, device="cuda"))
    torch.manual_seed(32)
    m.birth_threshold = 10.0
    with torch.set_grad_enabled(grad):
        s3, _ = m(torch.randn(4, 9, TINY.d_world, device="cuda"))
    assert torch.isfinite(s2).all() and torch.equal(s2, s3)


def test_dynamic_slots_bf16_birth_attention_from_kq():
    """Under a bf16 autocast the fused forward forms kq = k W_q instead of k (TINY's 128-wide slots take the
    fused core), and the birth step takes its attention as softmax over slots of LN_pre(slots) kq^T scale,
    without project_q.  The final attention map, the residual-driven birth and the slots agree with the fp32
    forward (keys k, then project_q) within the bf16 bar."""
    from hclsm_amd.kernels import slot_iteration as si
    from hclsm_amd.objects import DynamicSlotAttention
    torch.manual_seed(41)
    m = DynamicSlotAttention(TINY.objects, TINY.d_world).cuda()
    x = torch.randn(3, 100, TINY.d_world, device="cuda")
    assert si.forms_kq(3, TINY.objects.n_max_slots, 100, TINY.d_world, si.SlotWeights.from_module(m, torch.bfloat16))
    out = {}
    for bf16 in (False, True):
        torch.manual_seed(42)
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=bf16):
            out[bf16] = m(x, return_attention=True)
    (s32, a32, attn32), (s16, a16, attn16) = out[False], out[True]
    assert attn16.shape == attn32.shape == (3, TINY.objects.n_max_slots, 100)
    assert torch.allclose(attn16.float().sum(1), attn32.float().sum(1), atol=2e-2)
    assert normwise_rel_err(_np(attn16), _np(attn32)) <= 2e-2
    assert normwise_rel_err(_np(a16), _np(a32)) <= 2e-2
    assert normwise_rel_err(_np(s16), _np(s32)) <= 2e-2


def test_hot_path_from_reference_checkpoint_matches_oracle(tmp_path):
    """step_N.pt with the reference's layout (distributed.py:295-304) -> build_hot_path -> Level-0 and
    packed Level-1 forwards against oracle/modules.py with the checkpoint's weights."""
    from hclsm_amd.checkpoint import build_hot_path, module_state, preset_config, read_model_state
    from hclsm_amd.dynamics import HierarchyManager, Level0SSM, Level1EventDynamics
    torch.manual_seed(21)
    cfg = preset_config("tiny")
    src = {"level0_ssm": Level0SSM(cfg.dynamics.level0, D_SLOT),
           "level1_event": Level1EventDynamics(cfg.dynamics.level1, D_SLOT),
           "hierarchy_manager": HierarchyManager(D_SLOT, cfg.dynamics.level2.d_model)}
    from hclsm_amd.objects import DynamicSlotAttention, RelationGraph, SlotTracker
    src["slot_attention"] = DynamicSlotAttention(cfg.objects, cfg.d_world)
    src["slot_tracker"] = SlotTracker(cfg.objects)
    src["relation_graph"] = RelationGraph(cfg.objects)
    with torch.no_grad():      # trained-looking A_log: spread over the clamp's range
        for blk in list(src["level0_ssm"].object_blocks) + list(src["level0_ssm"].global_blocks):
            blk.A_log.uniform_(-3.0, 0.5)
    state = {f"{n}.{k}": v for n, m in src.items() for k, v in m.state_dict().items()}
    path = tmp_path / "step_100.pt"
    torch.save({"model": state, "optimizer": {}, "scheduler": None, "scaler": None, "global_step": 100,
                "is_fsdp": False}, path)
    mods = build_hot_path(path, cfg)
    sd = read_model_state(path)
    B, N, T = 2, 16, 8
    x = torch.randn(B, N, T, D_SLOT, device="cuda")
    mask = torch.ones(B, N, device="cuda")
    with torch.no_grad():
        out0 = mods["level0_ssm"](x, mask)
    ref0 = om.level0_ssm_ref(_np(x), _np(mask), {k: _np(v) for k, v in module_state(sd, "level0_ssm").items()},
                             cfg.dynamics.level0.n_blocks)
    assert normwise_rel_err(_np(out0), ref0) <= 1e-5
    states = torch.randn(B, T, N, D_SLOT, device="cuda")
    em = torch.zeros(B, T, device="cuda")
    em[:, [0, 3, 5]] = 1.0
    with torch.no_grad():
        ev, idx = mods["hierarchy_manager"].gather_events_packed(states, em)
        out1 = mods["level1_event"].forward_packed(ev, idx, mask)
    ref1 = om.level1_ref(_np(states[:, [0, 3, 5]]), None, _np(mask),
                         {k: _np(v) for k, v in module_state(sd, "level1_event").items()},
                         cfg.dynamics.level1.n_layers, cfg.dynamics.level1.n_heads)
    assert normwise_rel_err(_np(out1[:6]).reshape(B, 3, N, D_SLOT), ref1) <= 1e-5
    # object layer: tracker cost and relation graph with the checkpoint's weights
    from oracle import objects as ob
    a, b = torch.randn(B, N, D_SLOT, device="cuda"), torch.randn(B, N, D_SLOT, device="cuda")
    al = torch.ones(B, N, device="cuda")
    with torch.no_grad():
        cost = mods["slot_tracker"].compute_cost_matrix(a, b, al, al)
        nodes, causal = mods["relation_graph"](a, al)
    pt = {k: _np(v) for k, v in module_state(sd, "slot_tracker").items()}
    assert normwise_rel_err(_np(cost), ob.tracker_cost_ref(_np(a), _np(b), _np(al), _np(al), pt)) <= 1e-5
    pg = {k: _np(v) for k, v in module_state(sd, "relation_graph").items()}
    rn, rc = ob.relation_graph_ref(_np(a), _np(al), pg, cfg.objects.gnn_rounds)
    assert normwise_rel_err(_np(nodes), rn) <= 1e-5 and normwise_rel_err(_np(causal), rc) <= 1e-5


@pytest.mark.parametrize("autocast", [False, True])
def test_ssm_block_out_projection_residual_fused(autocast):
    """SimplifiedSSMBlock's out-projection and residual add run as one hclsm_linear launch (no fallback warning,
    raised as an error here): in fp32 the block matches its torch form (the same scan, then residual + out_proj)
    at 1e-5, under a bf16 autocast within the bf16 bar, and the gradients reach x and every weight.  The oracle and
    float64-autograd checks of the block run through the same path (test_level0_output_shape_and_oracle,
    test_ssm_block_gradients_match_float64_autograd)."""
    import warnings
    from hclsm_amd.dynamics import SimplifiedSSMBlock
    from hclsm_amd.kernels import HipFallbackWarning
    torch.manual_seed(5)
    blk = SimplifiedSSMBlock(192, 16).cuda()
    x = torch.randn(4, 40, 192, device="cuda")
    with warnings.catch_warnings():
        warnings.simplefilter("error", HipFallbackWarning)
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            out = blk(x)
            xr = x.clone().requires_grad_()
            (blk(xr) ** 2).mean().backward()
    assert out.dtype == torch.float32
    # the torch form of the same block: the scan output from the same kernel, then residual + out_proj
    from hclsm_amd.kernels import ssm_block_scan
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        h = blk.norm(x)
        z, gate = blk.in_proj(h), blk.gate_proj(h)
        y = ssm_block_scan(z, blk.dt_proj(z), blk.A_log, blk.B_proj(z), blk.C_proj(z), gate)
        want = x + blk.out_proj(y.to(h.dtype))
    assert normwise_rel_err(_np(out), _np(want.float())) <= (2e-2 if autocast else 1e-5)
    assert xr.grad is not None and torch.isfinite(xr.grad).all()
    for name, prm in blk.named_parameters():
        assert prm.grad is not None and torch.isfinite(prm.grad).all(), name
