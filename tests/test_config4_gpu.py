"""GPU parity at benchmark config 4 (the base-preset long-horizon chain) at its full shapes.

  * Four chained selective scans at (1024 sequences, T=1024, d=768), d_state 16, bf16 I/O, raw mode
    with the skip term, each fed the previous scan's output (the reference's unclamped GPU recurrence,
    hclsm/kernels/ssm_scan_kernel.py:227-290).  Each scan is checked against the float64 oracle on 64
    sequences (the first 16, the last 16, and every 31st between), fed the bf16 input the GPU scan saw; every
    output is checked finite; the first scan is checked for exact linearity in x (y(2x) == 2 y(x) bit for bit:
    doubling is exact in floating point, and the kernel's arithmetic is the same for both) and exact causality
    (changing x at t >= 512 leaves y at t < 512 bit-identical).
  * The event index of the p=0.05 mask (t=0 forced) bit-exact against the oracle's, and the causal
    event attention over it, 12 heads x 64, on every one of the ~53K events, against the float64 oracle
    fed the same bf16 rows (the per-track causal attention of the benchmark configuration, reached in
    the reference through sparse_event_attn.py:153-188).

Tolerances (normwise relative, max|got-ref|/max|ref|): bf16 inputs with fp32 accumulation 2e-2.
The inputs are the bench's config-4 draw (hclsm_amd.workloads.chain_config).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import events as ev
from oracle.ssm_scan import normwise_rel_err, ssm_scan_ref

pytestmark = pytest.mark.gpu

LOWP_TOL = 2e-2
SEL = sorted(set(range(16)) | set(range(16, 1008, 31)) | set(range(1008, 1024)))   # 64 sequences across the batch


@pytest.fixture(scope="module")
def cfg4():
    from hclsm_amd.workloads import chain_config
    print("config 4: drawing inputs on cuda:0", flush=True)
    d = chain_config("cuda")
    torch.cuda.synchronize()
    yield d
    del d
    torch.cuda.empty_cache()


def _scan(d, x):
    from hclsm_amd.kernels import fused_ssm_scan_hip
    return fused_ssm_scan_hip(x, d["dt"], d["A_log"], d["B"], d["C"], D=d["D"], clamp_mode="raw")


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def test_config4_chained_scans(cfg4):
    d = cfg4
    sel = torch.tensor(SEL, device="cuda")
    fixed = [_np(d[k][sel]) for k in ("dt", "B", "C")]
    A_log, Dv = _np(d["A_log"]), _np(d["D"])
    x = d["x"]
    for i in range(4):
        print(f"config 4: scan {i}", flush=True)
        y = _scan(d, x)
        torch.cuda.synchronize()
        assert y.shape == (1024, 1024, 768) and y.dtype == torch.bfloat16
        assert bool(torch.isfinite(y).all())
        ref = ssm_scan_ref(_np(x[sel]), fixed[0], A_log, fixed[1], fixed[2], D=Dv, clamp_mode="raw")
        err = normwise_rel_err(_np(y[sel]), ref)
        assert err <= LOWP_TOL, f"config 4 scan {i}: normwise err {err:.3e}"
        if i > 0:
            del x
        x = y


def test_config4_scan_linearity_and_causality(cfg4):
    d = cfg4
    print("config 4: linearity and causality of the first scan", flush=True)
    y1 = _scan(d, d["x"])
    x2 = d["x"] * 2                       # exact in bf16
    y2 = _scan(d, x2)
    torch.cuda.synchronize()
    assert torch.equal(y2, y1 * 2)
    del x2, y2
    xc = d["x"].clone()
    xc[:, 512:] = torch.randn(xc[:, 512:].shape, device="cuda").to(torch.bfloat16)
    yc = _scan(d, xc)
    torch.cuda.synchronize()
    assert torch.equal(yc[:, :512], y1[:, :512])
    assert not torch.equal(yc[:, 512:], y1[:, 512:])


def test_config4_event_attention(cfg4):
    from hclsm_amd.kernels.event_attention import event_attention
    from hclsm_amd.kernels.sparse_event_attn import build_event_index
    d = cfg4
    print("config 4: event index + 12-head causal event attention", flush=True)
    idx = build_event_index(d["mask"])
    ref_i = ev.event_index(d["mask"].cpu().numpy())
    for name in ("counts", "offsets", "slot_of"):
        np.testing.assert_array_equal(getattr(idx, name).cpu().numpy(), ref_i[name])
    total = idx.total()
    assert total == ref_i["total"] and 50_000 < total < 57_000
    np.testing.assert_array_equal(idx.indices[:total].cpu().numpy(), ref_i["indices"])
    np.testing.assert_array_equal(idx.rows[:total].cpu().numpy(), ref_i["rows"])
    out = event_attention(d["q"], d["k"], d["v"], idx, capacity=total)
    torch.cuda.synchronize()
    assert out.shape == (total, 12, 64) and out.dtype == torch.bfloat16
    rows = torch.from_numpy(ref_i["rows"].astype(np.int64)).cuda()
    ts = torch.from_numpy(ref_i["indices"].astype(np.int64)).cuda()
    packed = [_np(d[k][rows, ts]) for k in ("q", "k", "v")]
    ref = ev.track_causal_attention_packed(*packed, ref_i["offsets"])
    err = normwise_rel_err(_np(out), ref)
    assert err <= LOWP_TOL, f"config 4 event attention: normwise err {err:.3e}"
    # a track's first event attends only to itself: its output is its own v row
    first = torch.from_numpy(ref_i["offsets"][:-1].astype(np.int64)).cuda()
    assert torch.equal(out[first], d["v"][:, 0])
