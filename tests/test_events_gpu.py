"""GPU parity of the event index / gather / scatter kernels (bit-exact) and the reference's
sparse-event tests (tests/test_kernels.py:182-232, tests/test_dynamics.py:91-102) on the HIP path."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import events as ev

pytestmark = pytest.mark.gpu


def _mask(B, T, p, seed, force0=False):
    g = torch.Generator().manual_seed(seed)
    m = (torch.rand(B, T, generator=g) < p).float()
    if force0:
        m[:, 0] = 1
    return m


def _check_index(m_cpu, rule="gt_half", dtype=None):
    from hclsm_amd.kernels.sparse_event_attn import build_event_index
    mg = m_cpu.to(dtype) if dtype is not None else m_cpu
    idx = build_event_index(mg.cuda(), rule)
    ref = ev.event_index(mg.float().numpy() if mg.dtype != torch.bool else mg.numpy(), rule)
    total = ref["total"]
    np.testing.assert_array_equal(idx.counts.cpu().numpy(), ref["counts"])
    np.testing.assert_array_equal(idx.offsets.cpu().numpy(), ref["offsets"])
    np.testing.assert_array_equal(idx.indices[:total].cpu().numpy(), ref["indices"])
    np.testing.assert_array_equal(idx.rows[:total].cpu().numpy(), ref["rows"])
    np.testing.assert_array_equal(idx.slot_of.cpu().numpy(), ref["slot_of"])
    assert idx.stats.cpu().tolist() == [total, ref["kmax"]]
    return idx, ref


@pytest.mark.parametrize("B,T,p", [(1, 1, 1.0), (3, 7, 0.4), (1024, 64, 0.15), (7, 130, 0.3), (5, 64, 0.0),
                                   (2, 200, 1.0), (9000, 3, 0.5), (1024, 1024, 0.05),
                                   (8192, 32, 0.3), (4096, 65, 0.2),
                                   (20000, 3, 0.5)])   # past the two-launch row limit: separate scan
def test_index_bit_exact(B, T, p):
    _check_index(_mask(B, T, p, seed=B + T, force0=(p == 0.15)))


def _index_equal(idx, ref):
    total = ref.total()
    for name in ("counts", "offsets", "slot_of", "stats"):
        assert torch.equal(getattr(idx, name), getattr(ref, name)), name
    for name in ("indices", "rows"):            # entries past the total are unwritten capacity
        assert torch.equal(getattr(idx, name)[:total], getattr(ref, name)[:total]), name


@pytest.mark.parametrize("B,T,p", [(1, 4, 1.0), (63, 8, 0.5), (65, 16, 0.5), (200, 32, 0.3), (129, 64, 1.0),
                                   (1024, 64, 0.15), (4096, 64, 0.1), (4000, 4, 0.7), (3000, 16, 0.0),
                                   (2049, 32, 0.6), (4097, 64, 0.2), (10, 60, 0.5)])
def test_one_call_index(B, T, p):
    """The index hclsm_track_causal_attention leaves in its table buffer: the same tables as
    build_event_index, which is checked against the oracle; empty and full masks, ragged sizes."""
    from hclsm_amd.kernels.event_attention import track_causal_event_attention
    from hclsm_amd.kernels.sparse_event_attn import build_event_index
    m = _mask(B, T, p, seed=B + T, force0=(p == 0.15)).cuda()
    q = torch.zeros(B, T, 1, 16, dtype=torch.bfloat16, device="cuda")
    ref, _ = _check_index(m.cpu())
    _, idx = track_causal_event_attention(q, q, q, m, capacity=max(ref.total(), 1))
    _index_equal(idx, build_event_index(m))


@pytest.mark.parametrize("B,T", [(1024, 64), (77, 16)])
def test_one_call_index_nonzero_rule_and_misaligned_mask(B, T):
    """The one-call index under rule "nonzero" (negative, NaN and tiny values count), and from a mask whose
    storage is not 16-byte aligned: both bit-exact against build_event_index."""
    from hclsm_amd.kernels.event_attention import track_causal_event_attention
    from hclsm_amd.kernels.sparse_event_attn import build_event_index
    q = torch.zeros(B, T, 1, 16, dtype=torch.bfloat16, device="cuda")
    m = _mask(B, T, 0.3, seed=B)
    m = m * torch.where(torch.rand(B, T, generator=torch.Generator().manual_seed(1)) < 0.5, -1e-3, 1.0)
    m[0, 1] = float("nan")
    _check_index(m, rule="nonzero")
    mg = m.cuda()
    _, idx = track_causal_event_attention(q, q, q, mg, rule="nonzero", capacity=B * T)
    _index_equal(idx, build_event_index(mg, "nonzero"))
    m2 = _mask(B, T, 0.4, seed=B + 1).cuda()
    buf = torch.zeros(B * T + 1, device="cuda")
    mis = buf[1:].view(B, T)
    mis.copy_(m2)
    assert mis.data_ptr() % 16 != 0
    _, idx2 = track_causal_event_attention(q, q, q, mis, capacity=B * T)
    _index_equal(idx2, build_event_index(m2))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.bool, torch.uint8])
def test_index_mask_dtypes(dtype):
    _check_index(_mask(33, 70, 0.3, seed=2), dtype=dtype)


def test_index_rules_and_special_values():
    m = _mask(6, 40, 0.3, seed=3)
    m[0, 3] = float("nan")
    m[1, 4] = 0.5
    m[2, 5] = 1e-8
    m[3, 6] = -1.0
    for rule in ("gt_half", "nonzero"):
        _check_index(m, rule)


def test_index_empty_batch():
    from hclsm_amd.kernels.sparse_event_attn import build_event_index
    idx = build_event_index(torch.zeros(0, 5, device="cuda"))
    assert idx.offsets.cpu().tolist() == [0] and idx.stats.cpu().tolist() == [0, 0]


@pytest.mark.parametrize("shape,dtype", [((4, 20, 3, 5), torch.float32), ((3, 17, 8, 32), torch.bfloat16),
                                         ((5, 9, 3), torch.uint8), ((2, 33, 1, 7), torch.float16)])
def test_gather_scatter_bit_exact(shape, dtype):
    from hclsm_amd.kernels.sparse_event_attn import (build_event_index, gather_events_padded, gather_packed,
                                                     scatter_events_padded, scatter_packed)
    B, T = shape[:2]
    g = torch.Generator().manual_seed(11)
    states = (torch.randn(shape, generator=g) * 50).to(dtype)
    base = (torch.randn(shape, generator=g) * 50).to(dtype)
    m = _mask(B, T, 0.35, seed=12)
    idx = build_event_index(m.cuda())
    ref_i = ev.event_index(m.numpy())
    for K in (ref_i["kmax"], max(ref_i["kmax"] - 1, 1), ref_i["kmax"] + 2):
        got = gather_events_padded(states.cuda(), idx, K).cpu()
        ref = ev.gather_padded(states.numpy() if dtype != torch.bfloat16 else states.view(torch.int16).numpy(), ref_i, K)
        assert torch.equal(got.view(torch.int16) if dtype == torch.bfloat16 else got, torch.from_numpy(ref))
        upd = (torch.randn((B, K) + shape[2:], generator=g) * 50).to(dtype)
        got_s = scatter_events_padded(base.cuda(), upd.cuda(), idx).cpu()
        conv = (lambda t: t.view(torch.int16).numpy()) if dtype == torch.bfloat16 else (lambda t: t.numpy())
        ref_s = ev.scatter(conv(base), conv(upd), ref_i)
        assert np.array_equal(conv(got_s), ref_s)
    pk = gather_packed(states.cuda(), idx)
    tot = ref_i["total"]
    conv = (lambda t: t.view(torch.int16).numpy()) if dtype == torch.bfloat16 else (lambda t: t.numpy())
    assert np.array_equal(conv(pk[:tot].cpu()), ev.gather_packed(conv(states), ref_i))
    rt = scatter_packed(base.cuda(), pk[:tot], idx).cpu()
    assert np.array_equal(conv(rt), ev.scatter_packed(conv(base), ev.gather_packed(conv(states), ref_i), ref_i))


def test_reference_basic_gather_scatter():
    """tests/test_kernels.py:182-201 on the HIP path."""
    from hclsm_amd.kernels import naive_sparse_event_attention
    torch.manual_seed(0)
    states = torch.randn(2, 16, 8, 32, device="cuda")
    mask = torch.zeros(2, 16, device="cuda")
    mask[0, [2, 5, 10]] = 1
    mask[1, [1, 7]] = 1
    out = naive_sparse_event_attention(states, mask, lambda x: x * 2.0)
    assert out.shape == (2, 16, 8, 32)
    assert torch.equal(out[0, 0], states[0, 0]) and torch.equal(out[0, 3], states[0, 3])
    assert torch.allclose(out[0, 2], states[0, 2] * 2.0) and torch.allclose(out[0, 5], states[0, 5] * 2.0)


def test_reference_vectorized_matches_naive():
    """tests/test_kernels.py:203-215."""
    from hclsm_amd.kernels import naive_sparse_event_attention, sparse_event_attention
    states = torch.randn(2, 16, 8, 32, device="cuda")
    mask = torch.zeros(2, 16, device="cuda")
    mask[0, [2, 5, 10]] = 1
    mask[1, [1, 7, 9, 14]] = 1
    a = naive_sparse_event_attention(states, mask, lambda x: x)
    b = sparse_event_attention(states, mask, lambda x: x)
    assert torch.equal(a, b) and torch.equal(a, states)


def test_reference_no_events_and_all_events():
    """tests/test_kernels.py:217-232."""
    from hclsm_amd.kernels import sparse_event_attn_fn
    states = torch.randn(2, 8, 4, 16, device="cuda")
    assert torch.equal(sparse_event_attn_fn(states, torch.zeros(2, 8, device="cuda"), lambda x: x), states)
    out = sparse_event_attn_fn(states, torch.ones(2, 8, device="cuda"), lambda x: x * 0)
    assert torch.equal(out, torch.zeros_like(out))


def test_autograd_through_gather_and_scatter():
    """Gradients of loss = sum(w * scatter(base, f(gather(states)))) match torch autograd of the
    same index arithmetic written with torch.gather/scatter on the CPU."""
    from hclsm_amd.kernels.sparse_event_attn import build_event_index, gather_events_padded, scatter_events_padded
    B, T, N, D = 3, 12, 2, 4
    g = torch.Generator().manual_seed(5)
    m = _mask(B, T, 0.4, seed=6, force0=True)
    s_cpu = torch.randn(B, T, N, D, generator=g, dtype=torch.float64)
    base_cpu = torch.randn(B, T, N, D, generator=g, dtype=torch.float64)
    w = torch.randn(B, T, N, D, generator=g, dtype=torch.float64)
    idx = build_event_index(m.cuda())
    K = idx.kmax()
    s = s_cpu.cuda().requires_grad_()
    base = base_cpu.cuda().requires_grad_()
    out = scatter_events_padded(base, gather_events_padded(s, idx, K) ** 2, idx)
    (out * w.cuda()).sum().backward()
    ev_b = (m > 0.5)[..., None, None]
    expect_s = torch.where(ev_b, 2 * s_cpu * w, torch.zeros_like(w))
    expect_base = torch.where(ev_b, torch.zeros_like(w), w)
    assert torch.allclose(s.grad.cpu(), expect_s) and torch.equal(base.grad.cpu(), expect_base)


def test_hierarchy_gather_count():
    """tests/test_dynamics.py:91-102: two events per row -> K == 2."""
    from hclsm_amd.kernels.sparse_event_attn import build_event_index
    mask = torch.zeros(2, 8, device="cuda")
    mask[:, 2] = 1.0
    mask[:, 5] = 1.0
    assert build_event_index(mask).kmax() == 2


def test_wrappers_reject_tensors_that_do_not_match_the_index():
    """Every gather / scatter wrapper checks its tensors against the event index on the host, before
    any launch: a (B, T) mismatch, a row-shape mismatch or too few packed rows raise ValueError."""
    from hclsm_amd.kernels import sparse_event_attn as sea
    m = _mask(4, 10, 0.5, seed=31, force0=True).cuda()
    idx = sea.build_event_index(m)
    total = idx.total()
    good = torch.randn(4, 10, 3, 8, device="cuda")
    wrong_b = torch.randn(5, 10, 3, 8, device="cuda")
    wrong_t = torch.randn(4, 9, 3, 8, device="cuda")
    for bad in (wrong_b, wrong_t):
        with pytest.raises(ValueError):
            sea.gather_events_padded(bad, idx, 3)
        with pytest.raises(ValueError):
            sea.gather_packed(bad, idx)
        with pytest.raises(ValueError):
            sea.gather_events_packed(bad, idx)
        with pytest.raises(ValueError):
            sea.scatter_events_padded(bad, torch.zeros(bad.shape[0], 3, 3, 8, device="cuda"), idx)
        with pytest.raises(ValueError):
            sea.scatter_packed(bad, torch.zeros(total, 3, 8, device="cuda"), idx)
        with pytest.raises(ValueError):
            sea.scatter_events_packed(bad, torch.zeros(total, 3, 8, device="cuda"), idx)
    # updates with another row shape or batch size
    with pytest.raises(ValueError):
        sea.scatter_events_padded(good, torch.zeros(4, 3, 3, 7, device="cuda"), idx)
    with pytest.raises(ValueError):
        sea.scatter_events_padded(good, torch.zeros(3, 3, 3, 8, device="cuda"), idx)
    # packed with fewer rows than events, or another row shape
    with pytest.raises(ValueError):
        sea.scatter_packed(good, torch.zeros(total - 1, 3, 8, device="cuda"), idx)
    with pytest.raises(ValueError):
        sea.scatter_events_packed(good, torch.zeros(total - 1, 3, 8, device="cuda"), idx)
    with pytest.raises(ValueError):
        sea.scatter_packed(good, torch.zeros(total, 3, 7, device="cuda"), idx)
    with pytest.raises(ValueError):
        sea.gather_events_padded(good, idx, -1)
    # the matching calls still work, and exactly total packed rows suffice
    out = sea.scatter_packed(good, sea.gather_packed(good, idx)[:total].contiguous(), idx)
    assert torch.equal(out, good)
