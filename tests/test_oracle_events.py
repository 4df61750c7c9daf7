"""CPU pins of oracle/events.py.

  * index tables: an independent pure-Python loop, plus closed-form invariants (counts are
    row sums, offsets the exclusive cumsum, indices strictly ascending per row, slot_of the
    inverse map);
  * gather/scatter: round trip and the reference's own sparse-event tests
    (tests/test_kernels.py:182-232) re-run on the oracle;
  * attention: torch's scaled_dot_product_attention (is_causal=True per segment) and
    nn.MultiheadAttention with identity projections and key padding (library routines),
    segment length 1 => out = v, all-keys-padded => NaN.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import events as ev


def _mask(B, T, p, seed, force0=False):
    r = np.random.default_rng(seed)
    m = (r.random((B, T)) < p).astype(np.float32)
    if force0:
        m[:, 0] = 1
    return m


@pytest.mark.parametrize("B,T,p", [(1, 1, 0.5), (3, 7, 0.4), (5, 64, 0.15), (4, 130, 0.3), (6, 9, 0.0), (2, 5, 1.0)])
@pytest.mark.parametrize("rule", ["gt_half", "nonzero"])
def test_index_matches_scalar_loop(B, T, p, rule):
    m = _mask(B, T, p, seed=B * 100 + T)
    m[m == 0] = np.random.default_rng(1).choice([0.0, 0.3, 1e-8], size=(m == 0).sum())
    a, b = ev.event_index(m, rule), ev.event_index_scalar(m, rule)
    for k in ("counts", "offsets", "indices", "rows", "slot_of"):
        np.testing.assert_array_equal(a[k], b[k], err_msg=k)
    assert a["total"] == b["total"] and a["kmax"] == b["kmax"]


def test_index_invariants_and_nan_rule():
    m = _mask(16, 50, 0.3, seed=3)
    m[2, 7] = np.nan
    m[3, 9] = 0.5          # not > 0.5
    m[4, 1] = 0.5000001
    i = ev.event_index(m, "gt_half")
    np.testing.assert_array_equal(i["counts"], (m > 0.5).sum(1))
    np.testing.assert_array_equal(i["offsets"], np.concatenate([[0], np.cumsum((m > 0.5).sum(1))]))
    for b in range(16):
        seg = i["indices"][i["offsets"][b]:i["offsets"][b + 1]]
        assert np.all(np.diff(seg) > 0)
        for k, t in enumerate(seg):
            assert i["slot_of"][b, t] == k
    assert i["slot_of"][2, 7] == -1                        # NaN is not > 0.5
    assert ev.event_index(m, "nonzero")["slot_of"][2, 7] >= 0  # but it is nonzero
    assert i["slot_of"][3, 9] == -1 and i["slot_of"][4, 1] >= 0


def test_gather_scatter_roundtrip():
    r = np.random.default_rng(4)
    m = _mask(4, 20, 0.3, seed=5)
    states = r.standard_normal((4, 20, 3, 5))
    base = r.standard_normal((4, 20, 3, 5))
    i = ev.event_index(m)
    K = i["kmax"]
    g = ev.gather_padded(states, i, K)
    assert np.all(g[ev.pad_mask(i, K) == 0] == 0)
    out = ev.scatter(base, g, i)
    sel = (m > 0.5)[..., None, None]
    np.testing.assert_array_equal(out, np.where(sel, states, base))
    np.testing.assert_array_equal(ev.scatter_packed(base, ev.gather_packed(states, i), i), out)


def test_reference_sparse_event_tests_on_oracle():
    """tests/test_kernels.py:182-232, run against the oracle restatement."""
    r = np.random.default_rng(6)
    states = r.standard_normal((2, 16, 8, 32))
    mask = np.zeros((2, 16))
    mask[0, [2, 5, 10]] = 1
    mask[1, [1, 7]] = 1
    out = ev.naive_sparse_event_attention(states, mask, lambda x: x * 2.0)
    np.testing.assert_array_equal(out[0, 0], states[0, 0])
    np.testing.assert_array_equal(out[0, 3], states[0, 3])
    np.testing.assert_allclose(out[0, 2], states[0, 2] * 2.0)
    np.testing.assert_allclose(out[0, 5], states[0, 5] * 2.0)
    s2 = r.standard_normal((2, 8, 4, 16))
    np.testing.assert_array_equal(ev.naive_sparse_event_attention(s2, np.zeros((2, 8)), lambda x: x), s2)
    np.testing.assert_array_equal(ev.naive_sparse_event_attention(s2, np.ones((2, 8)), lambda x: x * 0), 0 * s2)


def test_track_causal_attention_matches_sdpa():
    r = np.random.default_rng(7)
    nb, T, H, dh = 5, 24, 3, 16
    q, k, v = (r.standard_normal((nb, T, H, dh)) for _ in range(3))
    m = _mask(nb, T, 0.3, seed=8, force0=True)
    i = ev.event_index(m)
    out = ev.track_causal_attention(q, k, v, i)
    for b in range(nb):
        o, c = i["offsets"][b], i["counts"][b]
        ts = i["indices"][o:o + c]
        tq = torch.tensor(q[b, ts]).permute(1, 0, 2)   # (H, c, dh)
        tk = torch.tensor(k[b, ts]).permute(1, 0, 2)
        tv = torch.tensor(v[b, ts]).permute(1, 0, 2)
        ref = F.scaled_dot_product_attention(tq, tk, tv, is_causal=True).permute(1, 0, 2).numpy()
        np.testing.assert_allclose(out[o:o + c], ref, rtol=1e-10, atol=1e-12)
    # segment of length one: output is v
    m1 = np.zeros((1, T), np.float32)
    m1[0, 5] = 1
    i1 = ev.event_index(m1)
    np.testing.assert_allclose(ev.track_causal_attention(q[:1], k[:1], v[:1], i1)[0], v[0, 5], rtol=1e-12)


def test_slots_attention_matches_multihead_attention():
    r = np.random.default_rng(9)
    P, N, H, dh = 4, 7, 2, 8
    x = r.standard_normal((P, N, H * dh))
    pad = r.random((P, N)) < 0.3
    pad[:, 0] = False
    mha = torch.nn.MultiheadAttention(H * dh, H, batch_first=True, bias=False)
    with torch.no_grad():
        mha.in_proj_weight.copy_(torch.cat([torch.eye(H * dh)] * 3, 0))
        mha.out_proj.weight.copy_(torch.eye(H * dh))
    xt = torch.tensor(x, dtype=torch.float64)
    mha = mha.double()
    ref, _ = mha(xt, xt, xt, key_padding_mask=torch.tensor(pad))
    q = x.reshape(P, N, H, dh)
    got = ev.slots_attention(q, q, q, key_pad=pad).reshape(P, N, H * dh)
    np.testing.assert_allclose(got, ref.detach().numpy(), rtol=1e-10, atol=1e-12)
    allpad = np.ones((1, N), bool)
    assert np.isnan(ev.slots_attention(q[:1], q[:1], q[:1], key_pad=allpad)).all()
