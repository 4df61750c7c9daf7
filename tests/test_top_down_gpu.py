"""GPU parity of the fused hierarchy output step (hclsm_event_top_down) against the float64 oracle of
HierarchyManager.forward (hierarchy_manager.py:120-162): packed and padded Level-1 rows, ragged row counts,
d_slot 32..384, fp32 / bf16 / fp16 gate GEMMs, no Level-2 context (bit-exact), in place, and the module
paths against their torch math."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import events as oe
from oracle import modules as om

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}

# (B, T, N, D, d_l2, n_summary, event probability)
CASES = [(4, 16, 32, 192, 512, 4, 0.15), (3, 5, 7, 64, 96, 1, 0.5), (2, 9, 32, 256, 512, 4, 0.3),
         (2, 6, 16, 384, 640, 2, 0.4), (1, 1, 1, 32, 32, 1, 1.0), (5, 7, 3, 128, 200, 3, 0.0)]


def _case(B, T, N, D, DL2, S2, p, seed=0, no_bias=False):
    from hclsm_amd.dynamics import HierarchyManager
    torch.manual_seed(seed)
    hm = HierarchyManager(D, DL2)
    with torch.no_grad():
        hm.gate_l2_l0[0].bias.normal_(0.0, 0.5)
    if no_bias:
        hm.gate_l2_l0[0].bias = None
    g = torch.Generator().manual_seed(seed + 1)
    mask = (torch.rand(B, T, generator=g) < p).float()
    if B > 2:
        mask[0] = 1.0           # every frame an event
        mask[1] = 0.0           # no event
    K = max(int(mask.sum(dim=1).max()), 1)
    level0 = torch.randn(B, T, N, D, generator=g)
    level1 = torch.randn(B, K, N, D, generator=g)
    ctx = torch.randn(B, S2, DL2, generator=g)
    obj = (torch.rand(B, N, generator=g) < 0.75).float()
    return hm, mask, level0, level1, ctx, obj


def _packed(level1, mask):
    """Level-1 rows in the packed layout: row offsets[b] + s holds event s of clip b (capacity B*T rows)."""
    B, K, N, D = level1.shape
    ref = oe.event_index(mask.numpy())
    packed = torch.zeros(B * mask.shape[1], N, D)
    for b in range(B):
        c = int(ref["counts"][b])
        packed[ref["offsets"][b]:ref["offsets"][b] + c] = level1[b, :c]
    return packed, ref


def _oracle(hm, level0, level1, ref, ctx, obj):
    bias = hm.gate_l2_l0[0].bias
    return om.hierarchy_forward_ref(level0.numpy(), level1.numpy(), ref, hm.l2_to_l1.weight.detach().numpy(),
                                    hm.gate_l2_l0[0].weight.detach().numpy(),
                                    None if bias is None else bias.detach().numpy(),
                                    None if ctx is None else ctx.numpy(), None if obj is None else obj.numpy())


def _err(got, want):
    want = np.asarray(want, np.float64)
    return float(np.linalg.norm(got.double().cpu().numpy() - want) / max(np.linalg.norm(want), 1e-30))


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_packed_matches_oracle(case, dtype):
    from hclsm_amd.kernels.sparse_event_attn import build_event_index
    from hclsm_amd.kernels.top_down import TopDownWeights, event_top_down
    hm, mask, level0, level1, ctx, obj = _case(*case)
    packed, ref = _packed(level1, mask)
    want = _oracle(hm, level0, level1, ref, ctx, obj)
    hm = hm.cuda()
    idx = build_event_index(mask.cuda(), "gt_half")
    print(f"top_down packed case={case} dtype={dtype}", flush=True)
    out = event_top_down(level0.cuda(), packed.cuda(), idx, TopDownWeights.from_module(hm, dtype), ctx.cuda(),
                         obj.cuda())
    torch.cuda.synchronize()
    assert out.dtype == torch.float32 and out.shape == level0.shape
    assert torch.isfinite(out).all()
    assert _err(out, want) < TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_padded_rows_short_capacity_and_no_bias(dtype):
    """Padded Level-1 rows with fewer slots than some clip's events: the later events keep Level-0
    (hierarchy_manager.py:109-116); a gate Linear without bias."""
    from hclsm_amd.kernels.sparse_event_attn import build_event_index
    from hclsm_amd.kernels.top_down import TopDownWeights, event_top_down
    hm, mask, level0, level1, ctx, obj = _case(4, 12, 32, 192, 256, 2, 0.5, seed=3, no_bias=True)
    short = level1[:, :2].contiguous()
    ref = oe.event_index(mask.numpy())
    assert int(ref["counts"].max()) > 2
    want = _oracle(hm, level0, short, ref, ctx, obj)
    hm = hm.cuda()
    print(f"top_down padded K=2 dtype={dtype}", flush=True)
    out = event_top_down(level0.cuda(), short.cuda(), build_event_index(mask.cuda(), "gt_half"),
                         TopDownWeights.from_module(hm, dtype), ctx.cuda(), obj.cuda(), kpad=2)
    torch.cuda.synchronize()
    assert _err(out, want) < TOL[dtype]


@pytest.mark.parametrize("case", CASES)
def test_no_context_is_the_masked_scatter(case):
    """Without a Level-2 context the step is the scatter times the alive mask: bit-exact (fp32 products)."""
    from hclsm_amd.kernels.sparse_event_attn import build_event_index
    from hclsm_amd.kernels.top_down import event_top_down
    hm, mask, level0, level1, ctx, obj = _case(*case, seed=5)
    packed, ref = _packed(level1, mask)
    want = oe.scatter(level0.numpy(), level1.numpy(), ref) * obj.numpy()[:, None, :, None]
    idx = build_event_index(mask.cuda(), "gt_half")
    print(f"top_down no-context case={case}", flush=True)
    out = event_top_down(level0.cuda(), packed.cuda(), idx, None, None, obj.cuda())
    out_nomask = event_top_down(level0.cuda(), packed.cuda(), idx, None, None, None)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), want.astype(np.float32))
    np.testing.assert_array_equal(out_nomask.cpu().numpy(), oe.scatter(level0.numpy(), level1.numpy(), ref))


def test_in_place_over_level0():
    from hclsm_amd.kernels.sparse_event_attn import build_event_index
    from hclsm_amd.kernels.top_down import TopDownWeights, event_top_down
    hm, mask, level0, level1, ctx, obj = _case(3, 10, 32, 192, 512, 4, 0.3, seed=7)
    packed, _ = _packed(level1, mask)
    hm = hm.cuda()
    W = TopDownWeights.from_module(hm, torch.float32)
    idx = build_event_index(mask.cuda(), "gt_half")
    x = level0.cuda()
    print("top_down in place", flush=True)
    want = event_top_down(x, packed.cuda(), idx, W, ctx.cuda(), obj.cuda())
    got = event_top_down(x, packed.cuda(), idx, W, ctx.cuda(), obj.cuda(), out=x)
    torch.cuda.synchronize()
    assert got.data_ptr() == x.data_ptr()
    assert torch.equal(got, want)


def test_module_paths_match_torch_math():
    """HierarchyManager.forward (padded) and forward_packed take the fused call without autograd; they agree
    with the module's torch math (scatter kernel + torch gate) and, under a bf16 autocast, with the oracle."""
    from hclsm_amd.kernels.sparse_event_attn import build_event_index
    hm, mask, level0, level1, ctx, obj = _case(4, 16, 32, 192, 512, 4, 0.2, seed=9)
    packed, ref = _packed(level1, mask)
    want = _oracle(hm, level0, level1, ref, ctx, obj)
    hm = hm.cuda()
    l0, l1, pk, c, o, m = level0.cuda(), level1.cuda(), packed.cuda(), ctx.cuda(), obj.cuda(), mask.cuda()
    print("top_down module paths", flush=True)
    with torch.no_grad():
        torch_math = hm._top_down(hm.scatter_events(l0, l1, m), c, o)
        padded = hm(l0, l1, c, m, o)
        packed_out = hm.forward_packed(l0, pk, build_event_index(m, "gt_half"), c, o)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            padded_bf = hm(l0, l1, c, m, o)
    torch.cuda.synchronize()
    assert _err(torch_math, want) < 1e-5
    assert _err(padded, want) < 1e-5 and _err(packed_out, want) < 1e-5
    assert padded_bf.dtype == torch.float32 and _err(padded_bf, want) < 2e-2
    # with autograd the module keeps the torch math, and its gradient flows
    l0g = l0.clone().requires_grad_(True)
    out = hm(l0g, l1, c, m, o)
    out.sum().backward()
    assert l0g.grad is not None and _err(out.detach(), want) < 1e-5
