"""GPU tests of the packed, sync-free Level-1 path: hclsm_level1_forward (one C call for
Level1EventDynamics over the live events), the differentiable packed gather / scatter, and
level1_events_packed (index, gather, Level-1, scatter and top-down gating without a host read).

Parity: the Level-1 output of every live event against oracle/modules.py::level1_ref on the padded
events (fp32: normwise 1e-5; bf16 compute: 2e-2); the whole packed step against the reference-shaped
padded flow (gather_events with its K_max host read, Level-1, HierarchyManager.forward), outputs and
gradients."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import modules as om
from oracle.ssm_scan import normwise_rel_err

pytestmark = pytest.mark.gpu

L1 = SimpleNamespace(d_model=256, n_layers=2, n_heads=4)     # HCLSMConfig.tiny() level1 (config.py:206)
D_SLOT, D_L2 = 128, 384


def _np(t):
    return t.detach().double().cpu().numpy()


def _sd(m):
    return {k: _np(v) for k, v in m.state_dict().items()}


def _case(B, T, N, seed, p=0.35, empty_row=True, dead=True):
    g = torch.Generator().manual_seed(seed)
    states = torch.randn(B, T, N, D_SLOT, generator=g)
    mask = (torch.rand(B, T, generator=g) < p).float()
    if empty_row and B > 1:
        mask[1] = 0.0
    obj = torch.ones(B, N)
    if dead:
        for b in range(B):
            k = int(torch.randint(0, N // 2, (1,), generator=g))
            obj[b, N - k:] = 0.0
    return states.cuda(), mask.cuda(), obj.cuda()


def _modules(seed):
    from hclsm_amd.dynamics import HierarchyManager, Level1EventDynamics
    torch.manual_seed(seed)
    return HierarchyManager(D_SLOT, D_L2).cuda(), Level1EventDynamics(L1, D_SLOT).cuda()


def _live_rows(out, idx):
    """Packed rows of the live events, in (b, k) order, and the (b, k) list."""
    counts = idx.counts.cpu().tolist()
    offs = idx.offsets.cpu().tolist()
    rows, bk = [], []
    for b, c in enumerate(counts):
        for k in range(c):
            rows.append(offs[b] + k)
            bk.append((b, k))
    return out[rows], bk


@pytest.mark.parametrize("B,T,N,seed", [(3, 7, 16, 0), (4, 12, 16, 1), (2, 5, 32, 2)])
def test_level1_packed_matches_oracle_fp32(B, T, N, seed):
    hm, l1 = _modules(seed)
    states, mask, obj = _case(B, T, N, seed)
    with torch.no_grad():
        ev, idx = hm.gather_events_packed(states, mask)
        out = l1.forward_packed(ev, idx, obj)
        ev_pad, pad, K = hm.gather_events(states, mask)
    ref = om.level1_ref(_np(ev_pad), _np(pad), _np(obj), _sd(l1), L1.n_layers, L1.n_heads)
    got, bk = _live_rows(out, idx)
    assert len(bk) == idx.total() and len(bk) > 0
    want = np.stack([ref[b, k] for b, k in bk])
    assert normwise_rel_err(_np(got), want) <= 1e-5


def test_level1_packed_bf16_autocast():
    hm, l1 = _modules(3)
    states, mask, obj = _case(4, 16, 16, 3)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        ev, idx = hm.gather_events_packed(states, mask)
        out = l1.forward_packed(ev, idx, obj)
    with torch.no_grad():
        ev_pad, pad, K = hm.gather_events(states, mask)
    ref = om.level1_ref(_np(ev_pad), _np(pad), _np(obj), _sd(l1), L1.n_layers, L1.n_heads)
    got, bk = _live_rows(out, idx)
    assert out.dtype == torch.float32
    assert normwise_rel_err(_np(got), np.stack([ref[b, k] for b, k in bk])) <= 2e-2


def test_level1_packed_bf16_autocast_wide_tiles():
    """A capacity of 65,536 rows: the paired SwiGLU GEMM (w1 / w3 interleaved, one launch) runs on the
    128x128-tile kernel, the other layers on their usual kernels; against the oracle at the bf16 bar."""
    hm, l1 = _modules(11)
    states, mask, obj = _case(16, 128, 32, 11, p=0.1)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        ev, idx = hm.gather_events_packed(states, mask)
        out = l1.forward_packed(ev, idx, obj)
    with torch.no_grad():
        ev_pad, pad, K = hm.gather_events(states, mask)
    ref = om.level1_ref(_np(ev_pad), _np(pad), _np(obj), _sd(l1), L1.n_layers, L1.n_heads)
    got, bk = _live_rows(out, idx)
    assert ev.shape[0] * ev.shape[1] == 65536
    assert normwise_rel_err(_np(got), np.stack([ref[b, k] for b, k in bk])) <= 2e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_level1_fused_qkv_attention_32_slots(dtype):
    """32 slots per event and 64-wide heads with 16-bit operands: the QKV projection and the slot attention run as
    one launch (q / k / v never leave the chip).  Against the oracle at the 16-bit bar, with a clip whose slots
    are all dead (its events' rows NaN, as softmax over all -inf), dead slots elsewhere, and a capacity whose
    128-row blocks are partly live."""
    from hclsm_amd.kernels.level1_packed import Level1Weights, level1_forward_packed
    hm, l1 = _modules(21)
    states, mask, obj = _case(5, 9, 32, 21, p=0.45)
    obj[2] = 0.0
    mask[2, 0] = 1.0
    with torch.no_grad():
        ev, idx = hm.gather_events_packed(states, mask)
        out = level1_forward_packed(ev, idx, obj, Level1Weights.from_module(l1, dtype))
        ev_pad, pad, K = hm.gather_events(states, mask)
    ref = om.level1_ref(_np(ev_pad), _np(pad), _np(obj), _sd(l1), L1.n_layers, L1.n_heads)
    got, bk = _live_rows(out, idx)
    assert len(bk) % 4 != 0 and ev.shape[0] * 32 % 128 != 0
    dead = torch.tensor([b == 2 for b, _ in bk], device="cuda")
    assert bool(dead.any()) and torch.isnan(got[dead]).all() and torch.isfinite(got[~dead]).all()
    keep = [i for i, (b, _) in enumerate(bk) if b != 2]
    want = np.stack([ref[b, k] for b, k in bk if b != 2])
    assert normwise_rel_err(_np(got[keep]), want) <= 2e-2


@pytest.mark.parametrize("dtype,N,B,T", [(torch.bfloat16, 32, 5, 9), (torch.float16, 16, 4, 12),
                                         (torch.bfloat16, 32, 16, 128)])
def test_level1_folded_layernorms(dtype, N, B, T):
    """16-bit calls fold the LayerNorms before the SwiGLU inputs, before proj_out and (32 slots: the fused QKV
    attention) LN1 of every block after the first into those layers' weights (Level1Weights' fold array: W diag(gamma),
    its row sums, W beta); the out-projection and W2 write the rows' LayerNorm partials.  With non-trivial gamma / beta in every LayerNorm and a mean offset on the events,
    the output matches the oracle at the 16-bit bar and the call without the fold array within 1e-2; the last case
    has a 65,536-row capacity."""
    from hclsm_amd.kernels.level1_packed import Level1Weights, level1_forward_packed
    hm, l1 = _modules(31 + N)
    g = torch.Generator().manual_seed(N + T)
    with torch.no_grad():
        for ln in [l1.norm] + [m for b in l1.blocks for m in (b.norm1, b.norm2)]:
            ln.weight.copy_(torch.rand(ln.weight.shape, generator=g) + 0.5)
            ln.bias.copy_(torch.randn(ln.bias.shape, generator=g) * 0.2)
    states, mask, obj = _case(B, T, N, 31 + N, p=0.3)
    states = states + 0.7
    W = Level1Weights.from_module(l1, dtype)
    assert W.fold is not None and len(W.fold) == 3 + 7 * L1.n_layers
    W0 = Level1Weights(W.tensors, W.dtype, W.d_slot, W.d_model, W.hidden, W.n_layers, W.n_heads, W.ln_eps)
    print(f"level1 fold {dtype} N={N} B={B} T={T}", flush=True)
    with torch.no_grad():
        ev, idx = hm.gather_events_packed(states, mask)
        out = level1_forward_packed(ev, idx, obj, W)
        out0 = level1_forward_packed(ev, idx, obj, W0)
        ev_pad, pad, K = hm.gather_events(states, mask)
    ref = om.level1_ref(_np(ev_pad), _np(pad), _np(obj), _sd(l1), L1.n_layers, L1.n_heads)
    got, bk = _live_rows(out, idx)
    got0, _ = _live_rows(out0, idx)
    want = np.stack([ref[b, k] for b, k in bk])
    assert normwise_rel_err(_np(got), want) <= 2e-2
    assert normwise_rel_err(_np(got), _np(got0)) <= 1e-2


def test_level1_fold_array_past_the_partials_limit():
    """d_model = 1088 (17 heads of 64) has 17 64-column LayerNorm partials per row, one more than the folded kernels
    combine: with the fold array given, the 16-bit call takes the LayerNorm launches instead and still matches the
    oracle at the 16-bit bar (and the call without the fold array within 1e-2)."""
    from hclsm_amd.dynamics import Level1EventDynamics
    from hclsm_amd.kernels.level1_packed import Level1Weights, level1_forward_packed
    cfg = SimpleNamespace(d_model=1088, n_layers=2, n_heads=17)
    hm, _ = _modules(41)
    torch.manual_seed(41)
    l1 = Level1EventDynamics(cfg, D_SLOT).cuda()
    states, mask, obj = _case(3, 6, 32, 41, p=0.5)
    mask[0, :2] = 1.0   # live events in clip 0 whatever the draw (clip 1 has none)
    W = Level1Weights.from_module(l1, torch.bfloat16)
    assert W.fold is not None
    W0 = Level1Weights(W.tensors, W.dtype, W.d_slot, W.d_model, W.hidden, W.n_layers, W.n_heads, W.ln_eps)
    print("level1 fold past the partials limit: d_model 1088", flush=True)
    with torch.no_grad():
        ev, idx = hm.gather_events_packed(states, mask)
        out = level1_forward_packed(ev, idx, obj, W)
        out0 = level1_forward_packed(ev, idx, obj, W0)
        ev_pad, pad, K = hm.gather_events(states, mask)
    ref = om.level1_ref(_np(ev_pad), _np(pad), _np(obj), _sd(l1), cfg.n_layers, cfg.n_heads)
    got, bk = _live_rows(out, idx)
    got0, _ = _live_rows(out0, idx)
    want = np.stack([ref[b, k] for b, k in bk])
    assert normwise_rel_err(_np(got), want) <= 2e-2
    assert normwise_rel_err(_np(got), _np(got0)) <= 1e-2


def test_level1_padded_forward_bf16_fused_attention():
    """The reference-shaped padded call (Level1EventDynamics.forward over (B, K_max, N, d_slot), level1_event.py:85-133)
    under a bf16 autocast with 32 slots: the dense event index feeds the fused QKV projection + slot attention
    (key padding through obj_mask of each event's clip).  Against the oracle at the bf16 bar, padded events zero."""
    hm, l1 = _modules(23)
    states, mask, obj = _case(3, 11, 32, 23, p=0.4)
    with torch.no_grad():
        ev_pad, pad, K = hm.gather_events(states, mask)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out = l1(ev_pad, pad, obj)
    ref = om.level1_ref(_np(ev_pad), _np(pad), _np(obj), _sd(l1), L1.n_layers, L1.n_heads)
    real = _np(pad) > 0.5
    assert normwise_rel_err(_np(out.float())[real], ref[real]) <= 2e-2
    assert bool((out.float()[~torch.as_tensor(real, device="cuda")] == 0).all())


def test_level1_packed_all_slots_dead_gives_nan_like_softmax():
    """An event whose slots are all dead: every key excluded, softmax over all -inf -> NaN rows, as
    nn.MultiheadAttention gives; other rows unaffected."""
    hm, l1 = _modules(4)
    states, mask, obj = _case(2, 6, 16, 4, empty_row=False, dead=False)
    mask[:, 0] = 1.0
    obj[1] = 0.0
    with torch.no_grad():
        ev, idx = hm.gather_events_packed(states, mask)
        out = l1.forward_packed(ev, idx, obj)
    got, bk = _live_rows(out, idx)
    dead_rows = torch.tensor([b == 1 for b, _ in bk], device="cuda")
    assert torch.isnan(got[dead_rows]).all()
    assert torch.isfinite(got[~dead_rows]).all()


def test_level1_packed_no_events():
    hm, l1 = _modules(5)
    states, mask, obj = _case(2, 6, 16, 5)
    mask.zero_()
    from hclsm_amd.dynamics import level1_events_packed
    with torch.no_grad():
        comb = level1_events_packed(hm, l1, states, mask, obj)
    assert torch.equal(comb, states * obj[:, None, :, None])


def _padded_flow(hm, l1, states, mask, obj, l2):
    ev, pad, K = hm.gather_events(states, mask)
    return hm(states, l1(ev, pad, obj), l2, mask, obj)


def test_level1_events_packed_matches_padded_flow_without_host_sync():
    from hclsm_amd.dynamics import level1_events_packed
    hm, l1 = _modules(6)
    states, mask, obj = _case(3, 10, 16, 6)
    l2 = torch.randn(3, 4, D_L2, device="cuda")
    with torch.no_grad():
        want = _padded_flow(hm, l1, states, mask, obj, l2)
        level1_events_packed(hm, l1, states, mask, obj, l2)   # warm caches (weights, workspace)
        torch.cuda.synchronize()
        torch.cuda.set_sync_debug_mode("error")
        try:
            got = level1_events_packed(hm, l1, states, mask, obj, l2)
        finally:
            torch.cuda.set_sync_debug_mode("default")
    assert normwise_rel_err(_np(got), _np(want)) <= 1e-5


def test_level1_events_packed_gradients_match_padded_flow():
    from hclsm_amd.dynamics import level1_events_packed
    hm, l1 = _modules(7)
    states, mask, obj = _case(2, 8, 16, 7)
    l2 = torch.randn(2, 3, D_L2, device="cuda")
    w = torch.randn(2, 8, 16, D_SLOT, device="cuda")
    xa = states.clone().requires_grad_()
    (level1_events_packed(hm, l1, xa, mask, obj, l2) * w).sum().backward()
    ga = {n: None if p.grad is None else p.grad.clone()
          for n, p in list(hm.named_parameters()) + list(l1.named_parameters())}
    hm.zero_grad()
    l1.zero_grad()
    xb = states.clone().requires_grad_()
    (_padded_flow(hm, l1, xb, mask, obj, l2) * w).sum().backward()
    assert normwise_rel_err(_np(xa.grad), _np(xb.grad)) <= 1e-5
    for n, p in list(hm.named_parameters()) + list(l1.named_parameters()):
        if p.grad is None:
            assert ga[n] is None or ga[n].abs().sum() == 0, n
            continue
        assert normwise_rel_err(_np(ga[n]), _np(p.grad)) <= 1e-5, n


@pytest.mark.parametrize("autocast", [False, True])
def test_level1_events_packed_small_preset_matches_padded_flow(autocast):
    """The bench's small-preset shape (32 clips x T=64 x 32 slots, d_slot 192, d_model 384, 3 layers,
    6 heads): large enough for the LDS-tiled GEMM kernels (64x64, 128x128, fp32) with device row counts
    and the gated epilogue.  fp32: 1e-5 normwise against the padded flow; bf16 autocast: 2e-2."""
    from hclsm_amd.dynamics import HierarchyManager, Level1EventDynamics, level1_events_packed
    torch.manual_seed(8)
    B, T, N, D, DL2 = 32, 64, 32, 192, 512
    hm = HierarchyManager(D, DL2).cuda()
    l1 = Level1EventDynamics(SimpleNamespace(d_model=384, n_layers=3, n_heads=6), D).cuda()
    g = torch.Generator(device="cuda").manual_seed(9)
    states = torch.randn(B, T, N, D, generator=g, device="cuda")
    mask = (torch.rand(B, T, generator=g, device="cuda") < 0.15).float()
    mask[:, 0] = 1.0
    obj = (torch.rand(B, N, generator=g, device="cuda") < 0.8).float()
    obj[:, 0] = 1.0
    l2 = torch.randn(B, 4, DL2, generator=g, device="cuda")
    with torch.no_grad():
        want = _padded_flow(hm, l1, states, mask, obj, l2)
        if autocast:
            with torch.autocast("cuda", dtype=torch.bfloat16):
                got = level1_events_packed(hm, l1, states, mask, obj, l2)
        else:
            got = level1_events_packed(hm, l1, states, mask, obj, l2)
    assert normwise_rel_err(_np(got.float()), _np(want)) <= (2e-2 if autocast else 1e-5)
