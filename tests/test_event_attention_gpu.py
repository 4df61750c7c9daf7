"""GPU parity of the MFMA event attention against the numpy oracle (oracle/events.py).

Tolerances, normwise relative (max|got-ref|/max|ref|): fp32 1e-5; bf16/fp16 inputs with fp32
softmax 2e-2 (oracle fed the rounded inputs)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import events as ev
from oracle.ssm_scan import normwise_rel_err

pytestmark = pytest.mark.gpu


def _data(P, T, H, dh, dtype, p, seed, force0=True):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(P, T, H, dh, generator=g).to(dtype) for _ in range(3))
    m = (torch.rand(P, T, generator=g) < p).float()
    if force0:
        m[:, 0] = 1
    return q, k, v, m


def _np(t):
    return t.float().cpu().numpy().astype(np.float64)


def _run_causal(q, k, v, m, out="packed"):
    from hclsm_amd.kernels.event_attention import track_causal_event_attention
    o, idx = track_causal_event_attention(q.cuda(), k.cuda(), v.cuda(), m.cuda(), out=out)
    torch.cuda.synchronize()
    return o, idx


def test_config3_bf16():
    """benchmark config 3: 1024 tracks, T=64, 6 heads x 64, p=0.15 with t=0 forced."""
    q, k, v, m = _data(1024, 64, 6, 64, torch.bfloat16, 0.15, seed=1003)
    o, _ = _run_causal(q, k, v, m)
    i = ev.event_index(m.numpy())
    ref = ev.track_causal_attention(_np(q), _np(k), _np(v), i)
    assert o.shape == ref.shape
    err = normwise_rel_err(_np(o), ref)
    assert err <= 2e-2, f"config 3 normwise err {err:.3e}"


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.float16, 2e-2), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("dh", [16, 32, 64, 128])
def test_dtypes_and_head_dims(dtype, tol, dh):
    q, k, v, m = _data(9, 40, 3, dh, dtype, 0.5, seed=dh)
    o, _ = _run_causal(q, k, v, m)
    ref = ev.track_causal_attention(_np(q), _np(k), _np(v), ev.event_index(m.numpy()))
    err = normwise_rel_err(_np(o), ref)
    assert err <= tol, f"{dtype} dh={dh}: {err:.3e}"


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_long_segments_cross_many_key_tiles(dtype, tol):
    q, k, v, m = _data(5, 300, 2, 64, dtype, 0.9, seed=7)
    m[3] = 0                          # an empty track
    m[4] = 0
    m[4, 299] = 1                     # a single event at the last step
    o, _ = _run_causal(q, k, v, m)
    i = ev.event_index(m.numpy())
    ref = ev.track_causal_attention(_np(q), _np(k), _np(v), i)
    assert normwise_rel_err(_np(o), ref) <= tol
    # segment of length one: output equals v at that row
    last = i["offsets"][4]
    np.testing.assert_allclose(_np(o[last]), _np(v[4, 299]), rtol=0, atol=0)


def test_grid_output_leaves_other_rows():
    from hclsm_amd.kernels.event_attention import event_attention
    from hclsm_amd.kernels.sparse_event_attn import build_event_index
    q, k, v, m = _data(6, 50, 2, 32, torch.float32, 0.3, seed=9)
    base = torch.randn(6, 50, 2, 32)
    idx = build_event_index(m.cuda())
    og = base.cuda().clone()
    event_attention(q.cuda(), k.cuda(), v.cuda(), idx, out="grid", out_grid=og)
    i = ev.event_index(m.numpy())
    ref = ev.scatter_packed(_np(base), ev.track_causal_attention(_np(q), _np(k), _np(v), i), i)
    assert normwise_rel_err(_np(og), ref) <= 1e-5
    nonev = (m < 0.5)
    assert torch.equal(og.cpu()[nonev], base[nonev])


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_slots_mode_with_key_padding(dtype, tol):
    from hclsm_amd.kernels.event_attention import slots_attention
    g = torch.Generator().manual_seed(13)
    P, N, H, dh = 40, 32, 6, 64               # small preset: 32 slots, 6 heads x 64
    q, k, v = (torch.randn(P, N, H, dh, generator=g).to(dtype) for _ in range(3))
    pad = torch.rand(P, N, generator=g) < 0.25
    pad[:, 0] = False
    out = slots_attention(q.cuda(), k.cuda(), v.cuda(), pad.cuda())
    ref = ev.slots_attention(_np(q), _np(k), _np(v), key_pad=pad.numpy())
    assert normwise_rel_err(_np(out), ref) <= tol
    allpad = torch.ones(1, N, dtype=torch.bool)
    o2 = slots_attention(q[:1].cuda(), k[:1].cuda(), v[:1].cuda(), allpad.cuda())
    assert torch.isnan(o2).all()


def test_against_torch_sdpa_on_gpu():
    """Independent library check: per-track torch SDPA (fp32, math) on the GPU."""
    import torch.nn.functional as F
    q, k, v, m = _data(8, 48, 4, 64, torch.float32, 0.4, seed=21)
    o, idx = _run_causal(q, k, v, m)
    offs = idx.offsets.cpu().tolist()
    for b in range(8):
        ts = torch.nonzero(m[b] > 0.5).flatten()
        qq, kk, vv = (t[b, ts].permute(1, 0, 2).cuda() for t in (q, k, v))
        ref = F.scaled_dot_product_attention(qq, kk, vv, is_causal=True).permute(1, 0, 2)
        assert torch.allclose(o[offs[b]:offs[b + 1]], ref, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("P,T,H,dh,p,dtype", [(1024, 64, 6, 64, 0.15, torch.bfloat16), (37, 300, 2, 32, 0.3, torch.float32),
                                              (5, 1, 1, 16, 1.0, torch.float16), (64, 128, 4, 64, 0.0, torch.bfloat16),
                                              (8, 1024, 3, 64, 0.05, torch.bfloat16), (700, 16, 2, 128, 0.5, torch.float32),
                                              (3, 1500, 1, 16, 0.3, torch.bfloat16),
                                              (5000, 32, 1, 16, 0.3, torch.bfloat16)])   # past the in-launch track bound
def test_one_call_matches_two_calls(P, T, H, dh, p, dtype):
    """hclsm_track_causal_attention (index + attention in one call, capacity given: for T <= 1024 the row
    counts, then the attention building each track's event list from the mask and filling the tables; past
    that the separate index build) against the index build followed by hclsm_event_attention: identical
    packed output and identical index tables; with a capacity below the event total the rows past it are
    not written."""
    from hclsm_amd.kernels.event_attention import event_attention, track_causal_event_attention
    from hclsm_amd.kernels.sparse_event_attn import build_event_index
    q, k, v, m = _data(P, T, H, dh, dtype, p, seed=P + T)
    q, k, v, m = q.cuda(), k.cuda(), v.cuda(), m.cuda()
    ref_idx = build_event_index(m)
    total = ref_idx.total()
    ref = event_attention(q, k, v, ref_idx, capacity=total)
    o, idx = track_causal_event_attention(q, k, v, m, capacity=total)
    torch.cuda.synchronize()
    assert o.shape == (total, H, dh) and torch.equal(o, ref)
    for name in ("counts", "offsets", "slot_of", "stats"):
        assert torch.equal(getattr(idx, name), getattr(ref_idx, name)), name
    assert torch.equal(idx.indices[:total], ref_idx.indices[:total])
    assert torch.equal(idx.rows[:total], ref_idx.rows[:total])
    if total > 1:
        cut = total // 2
        o2, _ = track_causal_event_attention(q, k, v, m, capacity=cut)
        assert o2.shape == (cut, H, dh) and torch.equal(o2, ref[:cut])


def test_one_call_reuses_buffers():
    """Passing back the output and the index of an earlier call: a second mask of the same shape gives the
    same result as fresh buffers, written into the same memory; mismatched buffers raise before any launch."""
    from hclsm_amd.kernels.event_attention import track_causal_event_attention
    from hclsm_amd.kernels.sparse_event_attn import EventIndex, build_event_index
    P, T, H, dh = 96, 80, 3, 64
    q, k, v, m = (t.cuda() for t in _data(P, T, H, dh, torch.bfloat16, 0.3, seed=11))
    _, _, _, m2 = (t.cuda() for t in _data(P, T, H, dh, torch.bfloat16, 0.2, seed=12))
    cap = P * T
    o, idx = track_causal_event_attention(q, k, v, m, capacity=cap)
    ptr_o, ptr_i = o.data_ptr(), idx.ptr("stats")
    o2, idx2 = track_causal_event_attention(q, k, v, m2, out_packed=o, index=idx)
    ref, ref_idx = track_causal_event_attention(q, k, v, m2, capacity=cap)
    torch.cuda.synchronize()
    total = build_event_index(m2).total()
    assert o2.data_ptr() == ptr_o and idx2.ptr("stats") == ptr_i
    assert torch.equal(o2[:total], ref[:total])
    for name in ("counts", "offsets", "slot_of", "stats"):
        assert torch.equal(getattr(idx2, name), getattr(ref_idx, name)), name
    with pytest.raises(ValueError):
        track_causal_event_attention(q, k, v, m2, out_packed=o[:, :, :32], index=idx)
    with pytest.raises(ValueError):
        track_causal_event_attention(q, k, v, m2, out_packed=o, index=EventIndex.allocate(P, T + 1, q.device))


def test_plan_matches_the_function_and_follows_updates():
    """TrackCausalPlan: the same output and tables as track_causal_event_attention, written into the same
    buffers each call, and a mask / q updated in place between calls is what the next call reads."""
    from hclsm_amd.kernels.event_attention import TrackCausalPlan, track_causal_event_attention
    P, T, H, dh = 200, 64, 6, 64
    q, k, v, m = (t.cuda() for t in _data(P, T, H, dh, torch.bfloat16, 0.15, seed=31))
    cap = P * T
    plan = TrackCausalPlan(q, k, v, m, capacity=cap)
    for step in range(3):
        if step:
            _, _, _, m_new = _data(P, T, H, dh, torch.bfloat16, 0.1 * step, seed=40 + step)
            m.copy_(m_new.cuda())
            q.mul_(0.5)
        out, idx = plan()
        ref, ref_idx = track_causal_event_attention(q, k, v, m, capacity=cap)
        torch.cuda.synchronize()
        total = int(ref_idx.stats[0])
        assert out.data_ptr() == plan.out.data_ptr() and idx is plan.index
        assert torch.equal(out[:total], ref[:total])
        for name in ("counts", "offsets", "slot_of", "stats"):
            assert torch.equal(getattr(idx, name), getattr(ref_idx, name)), name
    with pytest.raises(ValueError):
        TrackCausalPlan(q[:, :, :, :32], k[:, :, :, :32], v[:, :, :, :32], m, capacity=cap)


@pytest.mark.parametrize("mdtype", [torch.bool, torch.uint8, torch.bfloat16])
def test_plan_mask_dtypes(mdtype):
    """TrackCausalPlan over bool / uint8 / bf16 masks gives the fp32-mask result; a float64 mask, which the
    plan cannot bind without a copy, raises."""
    from hclsm_amd.kernels.event_attention import TrackCausalPlan, track_causal_event_attention
    P, T, H, dh = 40, 48, 2, 32
    q, k, v, m = (t.cuda() for t in _data(P, T, H, dh, torch.float32, 0.3, seed=77))
    cap = P * T
    ref, ref_idx = track_causal_event_attention(q, k, v, m, capacity=cap)
    out, idx = TrackCausalPlan(q, k, v, (m > 0.5).to(mdtype).contiguous(), capacity=cap)()
    torch.cuda.synchronize()
    total = int(ref_idx.stats[0])
    assert torch.equal(out[:total], ref[:total])
    assert torch.equal(idx.offsets, ref_idx.offsets)
    with pytest.raises(TypeError):
        TrackCausalPlan(q, k, v, m.double(), capacity=cap)


@pytest.mark.parametrize("P,T,H,dh,p,dtype", [(16, 256, 3, 64, 0.3, torch.bfloat16),    # ~77 events: past the 64 staged rows
                                              (12, 1024, 2, 64, 0.05, torch.bfloat16),  # config 4's density
                                              (10, 200, 2, 32, 0.6, torch.float16),     # 128 staged rows
                                              (6, 300, 2, 128, 0.4, torch.bfloat16),    # 32 staged rows
                                              (9, 150, 3, 64, 0.5, torch.float32),      # fp32: 32 staged rows
                                              (7, 130, 2, 16, 0.7, torch.float32),
                                              (33, 65, 1, 64, 1.0, torch.bfloat16)])    # 65 events, 5 tiles
def test_staged_kv_kernel_matches_direct_kernel(P, T, H, dh, p, dtype):
    """Tracks longer than 64 steps with a packed output take the kernel that stages each (track, head)'s K/V rows
    in LDS once; the grid output is still written by the kernel that reads K/V from global memory per tile.  Both
    compute each query tile in the same order, so the packed rows equal the grid rows at the event positions bit
    for bit; the packed result is also checked against the oracle (a track with no events, and one with a
    single event, included)."""
    from hclsm_amd.kernels.event_attention import event_attention
    from hclsm_amd.kernels.sparse_event_attn import build_event_index
    q, k, v, m = _data(P, T, H, dh, dtype, p, seed=P * T + dh)
    m[1] = 0
    m[2] = 0
    m[2, T - 1] = 1
    q, k, v, m = q.cuda(), k.cuda(), v.cuda(), m.cuda()
    idx = build_event_index(m)
    packed = event_attention(q, k, v, idx)
    grid = event_attention(q, k, v, idx, out="grid")
    torch.cuda.synchronize()
    ev_rows = grid[m > 0.5]                      # (total, H, dh) in (track, ascending t) order = packed order
    assert torch.equal(packed, ev_rows)
    i = ev.event_index(m.cpu().numpy())
    ref = ev.track_causal_attention(_np(q), _np(k), _np(v), i)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert normwise_rel_err(_np(packed), ref) <= tol
