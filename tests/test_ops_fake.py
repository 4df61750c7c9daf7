"""torch.library ops (namespace hclsm_hip): fake kernels give the C ABI's output shapes and dtypes
on meta tensors and under FakeTensorMode (no GPU needed)."""

from __future__ import annotations

import torch

import hclsm_amd.kernels.ops  # noqa: F401  (registers the ops)

OPS = torch.ops.hclsm_hip


def _m(*s, dt=torch.float32):
    return torch.empty(*s, device="meta", dtype=dt)


def test_scan_ops_fake_shapes():
    bf = torch.bfloat16
    x = _m(2, 8, 32, dt=bf)
    y, h = OPS.ssm_scan_fwd(x, x, _m(32, 16), _m(2, 8, 16, dt=bf), _m(2, 8, 16, dt=bf), None, 0, True)
    assert (y.shape, y.dtype, h.shape, h.dtype) == ((2, 8, 32), bf, (2, 32, 16), torch.float32)
    _, h0 = OPS.ssm_scan_fwd(x, x, _m(32, 16), _m(2, 8, 16, dt=bf), _m(2, 8, 16, dt=bf), None, 1, False)
    assert h0.shape == (0,)
    g = OPS.ssm_scan_bwd(x, x, _m(32, 16), _m(2, 8, 16, dt=bf), _m(2, 8, 16, dt=bf), _m(32), x, 1)
    assert [tuple(t.shape) for t in g] == [(2, 8, 32), (2, 8, 32), (32, 16), (2, 8, 16), (2, 8, 16), (32,)]
    assert g[2].dtype == torch.float32 and g[0].dtype == bf


def test_event_and_slot_ops_fake_shapes():
    i32 = torch.int32
    idx = OPS.event_index(_m(4, 9), 0)
    assert [tuple(t.shape) for t in idx] == [(4,), (5,), (36,), (36,), (4, 9), (2,)]
    assert all(t.dtype == i32 for t in idx)
    assert OPS.event_gather(_m(4, 9, 3, 5), _m(4, dt=i32), _m(5, dt=i32), _m(36, dt=i32), 2).shape == (4, 2, 3, 5)
    assert OPS.event_scatter(_m(4, 9, 3, 5), _m(4, 2, 3, 5), _m(4, 9, dt=i32)).shape == (4, 9, 3, 5)
    q = _m(4, 9, 2, 16)
    assert OPS.event_attention(q, q, q, _m(5, dt=i32), _m(36, dt=i32), None, 0.25, 0, 11).shape == (11, 2, 16)
    out, attn = OPS.slot_attn_core(_m(2, 8, 64), _m(2, 40, 64), _m(2, 40, 64), 0.125, 0.0, 0.0, -1.0)
    assert out.shape == (2, 8, 64) and attn.shape == (2, 8, 40)
    s = OPS.slot_attention_forward(_m(2, 40, 32), _m(2, 8, 64), [_m(1)] * 17, 3, 0.125, 0.0, 1e-8, 0.0, torch.bfloat16)
    assert s.shape == (2, 8, 64) and s.dtype == torch.float32


def test_packed_level1_ops_fake_shapes():
    i32 = torch.int32
    assert OPS.event_gather_packed(_m(4, 9, 3, 5), _m(36, dt=i32), _m(36, dt=i32), _m(2, dt=i32)).shape == (36, 3, 5)
    assert OPS.event_scatter_packed(_m(4, 9, 3, 5), _m(36, 3, 5), _m(5, dt=i32), _m(4, 9, dt=i32)).shape == (4, 9, 3, 5)
    params = [_m(64, 32), _m(64), _m(64), _m(32, 64)] + [_m(1)] * 9
    out = OPS.level1_forward(_m(36, 8, 32), _m(2, dt=i32), _m(36, dt=i32), _m(4, 8), params, 4, 1e-5, torch.bfloat16)
    assert out.shape == (36, 8, 32) and out.dtype == torch.float32
    td = OPS.event_top_down(_m(4, 9, 3, 64), _m(36, 3, 64), _m(5, dt=i32), _m(4, 9, dt=i32), 0, _m(4, 2, 96),
                            _m(4, 3), [_m(64, 96), _m(64, 128), _m(64)], torch.bfloat16)
    assert td.shape == (4, 9, 3, 64) and td.dtype == torch.float32


def test_ops_under_fake_tensor_mode():
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        x = torch.empty(2, 8, 32)
        y, _ = OPS.ssm_scan_fwd(x, x, torch.empty(32, 16), torch.empty(2, 8, 16), torch.empty(2, 8, 16), None, 0, False)
        assert y.shape == (2, 8, 32)


def test_object_layer_ops_fake_shapes():
    nodes, causal = OPS.relation_graph_forward(_m(6, 16, 64), _m(6, 16), [_m(1)] * 18, 2, False, 1e-5, torch.bfloat16)
    assert nodes.shape == (6, 16, 64) and causal.shape == (6, 16, 16) and causal.dtype == torch.float32
    t, a, p, mt, h = OPS.slot_track_sequence(_m(2, 5, 16, 64), _m(2, 5, 16), [_m(1)] * 10, True, 20, 0.05,
                                             torch.bfloat16)
    assert [tuple(x.shape) for x in (t, a, p, mt, h)] == [(2, 5, 16, 64), (2, 5, 16), (2, 5, 16), (2, 5, 16), (2, 16, 64)]
    assert p.dtype == torch.int64
    _, a0, _, _, h0 = OPS.slot_track_sequence(_m(2, 5, 16, 64), None, [_m(1)] * 10, False, 20, 0.05, torch.float32)
    assert a0.shape == (0,) and h0.shape == (0,)
