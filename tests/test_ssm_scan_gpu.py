"""GPU parity of the HIP selective scan against the numpy oracle.

Tolerances (normwise relative, max|got-ref|/max|ref|):
  fp32 I/O: 1e-5;  bf16 / fp16 I/O with fp32 state: 2e-2 (oracle fed the rounded inputs).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.ssm_scan import normwise_rel_err, ssm_scan_ref

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
LOWP_TOL = 2e-2


def _inputs(N, T, Dn, S, dtype=torch.float32, seed=0, A_hi=math.log(16.0), dt_kind="softplus"):
    from hclsm_amd.workloads import scan_inputs
    d = scan_inputs(N, T, Dn, S, dtype=dtype, seed=seed)
    if dt_kind == "ref_test":   # tests/test_kernels.py:125 distribution
        g = torch.Generator().manual_seed(seed + 7)
        d["dt"] = (torch.rand(N, T, Dn, generator=g).abs() + 0.01).to(dtype)
        d["A_log"] = torch.randn(Dn, S, generator=g)
    else:
        d["A_log"] = d["A_log"] * (A_hi / math.log(16.0))
    return d


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _run(d, mode, with_D, dev="cuda", want_h=False):
    from hclsm_amd.kernels import fused_ssm_scan_hip
    args = [d[k].to(dev) for k in ("x", "dt", "A_log", "B", "C")]
    return fused_ssm_scan_hip(*args, D=d["D"].to(dev) if with_D else None, clamp_mode=mode,
                              return_h_final=want_h)


@pytest.mark.parametrize("mode", ["raw", "model"])
@pytest.mark.parametrize("with_D", [False, True])
def test_config0_fp32(mode, with_D):
    from hclsm_amd.workloads import scan_config
    d = scan_config(0)
    y = _run(d, mode, with_D)
    torch.cuda.synchronize()
    ref = ssm_scan_ref(_np(d["x"]), _np(d["dt"]), _np(d["A_log"]), _np(d["B"]), _np(d["C"]),
                       D=_np(d["D"]) if with_D else None, clamp_mode=mode)
    assert y.dtype == torch.float32
    err = normwise_rel_err(_np(y), ref)
    assert err <= FP32_TOL, f"cfg0 {mode} D={with_D}: normwise err {err:.3e}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_lowp_io(dtype):
    d = _inputs(64, 40, 192, 16, dtype=dtype, seed=3)
    y = _run(d, "raw", True)
    ref = ssm_scan_ref(_np(d["x"]), _np(d["dt"]), _np(d["A_log"]), _np(d["B"]), _np(d["C"]),
                       D=_np(d["D"]), clamp_mode="raw")
    assert y.dtype == dtype
    err = normwise_rel_err(_np(y), ref)
    assert err <= LOWP_TOL, f"{dtype}: normwise err {err:.3e}"


@pytest.mark.parametrize("N,T,Dn,S", [
    (1, 1, 1, 1),        # smallest
    (3, 7, 5, 3),        # ragged everything, T < chunk
    (2, 9, 70, 5),       # T = chunk + 1, D not a multiple of 64
    (2, 17, 130, 17),    # S just over a power of two
    (2, 16, 64, 32),
    (1, 24, 128, 33),
    (1, 8, 64, 64),      # maximum d_state
    (4, 33, 384, 8),
])
@pytest.mark.parametrize("mode", ["raw", "model"])
def test_shapes_fp32(N, T, Dn, S, mode):
    d = _inputs(N, T, Dn, S, seed=N * 1000 + T * 10 + S, dt_kind="ref_test")
    y, h = _run(d, mode, True, want_h=True)
    ref, href = ssm_scan_ref(_np(d["x"]), _np(d["dt"]), _np(d["A_log"]), _np(d["B"]), _np(d["C"]),
                             D=_np(d["D"]), clamp_mode=mode, return_h_final=True)
    assert normwise_rel_err(_np(y), ref) <= FP32_TOL
    assert normwise_rel_err(_np(h), href) <= FP32_TOL


def test_reference_test_distribution_modes_differ():
    """On the reference test's own inputs (tests/test_kernels.py:120-128) raw and model
    semantics disagree, as the reference's parallel-vs-sequential test would show."""
    d = _inputs(2, 16, 32, 8, seed=11, dt_kind="ref_test")
    y_raw = _run(d, "raw", False)
    y_mod = _run(d, "model", False)
    ref_raw = ssm_scan_ref(_np(d["x"]), _np(d["dt"]), _np(d["A_log"]), _np(d["B"]), _np(d["C"]), clamp_mode="raw")
    ref_mod = ssm_scan_ref(_np(d["x"]), _np(d["dt"]), _np(d["A_log"]), _np(d["B"]), _np(d["C"]), clamp_mode="model")
    assert normwise_rel_err(_np(y_raw), ref_raw) <= FP32_TOL
    assert normwise_rel_err(_np(y_mod), ref_mod) <= FP32_TOL
    assert normwise_rel_err(ref_raw, ref_mod) > 1e-2


def test_config1_bf16_full_and_properties():
    """Full config-1 launch (1024, 64, 384) bf16 against the oracle on every sequence (in blocks of 256, each
    block and the whole output at the bf16 bar), plus linearity on the whole output."""
    from hclsm_amd.workloads import scan_config
    d = scan_config(1)
    y = _run(d, "raw", True)
    torch.cuda.synchronize()
    assert y.shape == (1024, 64, 384) and y.dtype == torch.bfloat16
    assert torch.isfinite(y).all()
    yn = _np(y)
    dmax = rmax = 0.0
    for s0 in range(0, 1024, 256):
        sel = slice(s0, s0 + 256)
        ref = ssm_scan_ref(_np(d["x"][sel]), _np(d["dt"][sel]), _np(d["A_log"]), _np(d["B"][sel]), _np(d["C"][sel]),
                           D=_np(d["D"]), clamp_mode="raw")
        err = normwise_rel_err(yn[sel], ref)
        assert err <= LOWP_TOL, f"cfg1 sequences {s0}..{s0 + 255}: normwise err {err:.3e}"
        dmax = max(dmax, float(np.abs(yn[sel] - ref).max()))
        rmax = max(rmax, float(np.abs(ref).max()))
    assert dmax / rmax <= LOWP_TOL, f"cfg1 all sequences: normwise err {dmax / rmax:.3e}"
    # linearity in x (dt fixed): y(2x) - D*2x == 2 (y(x) - D*x) up to bf16 rounding
    d2 = dict(d)
    d2["x"] = (d["x"].float() * 2).to(torch.bfloat16)   # exact in bf16
    y2 = _run(d2, "raw", False)
    y1 = _run(d, "raw", False)
    err_lin = normwise_rel_err(_np(y2), 2 * _np(y1))
    assert err_lin <= 1e-2, f"linearity err {err_lin:.3e}"


def test_causality_and_zero_B():
    d = _inputs(4, 20, 96, 16, seed=5)
    y = _run(d, "raw", False)
    d2 = {k: v.clone() for k, v in d.items()}
    d2["x"][:, 12:] = torch.randn_like(d2["x"][:, 12:])
    d2["dt"][:, 12:] = 0.3
    y2 = _run(d2, "raw", False)
    assert torch.equal(y[:, :12], y2[:, :12])  # outputs before t=12 ignore later inputs
    d3 = {k: v.clone() for k, v in d.items()}
    d3["B"].zero_()
    y3 = _run(d3, "raw", True)
    assert torch.allclose(y3, d3["x"].cuda() * d3["D"].cuda(), rtol=1e-6, atol=1e-6)


def test_empty_and_errors():
    from hclsm_amd.kernels import ssm_scan_fn
    x = torch.zeros(0, 5, 8, device="cuda")
    y = ssm_scan_fn(x, x, torch.zeros(8, 4, device="cuda"), torch.zeros(0, 5, 4, device="cuda"),
                    torch.zeros(0, 5, 4, device="cuda"))
    assert y.shape == (0, 5, 8)
    xc = torch.zeros(2, 3, 8)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ssm_scan_fn(xc, xc, torch.zeros(8, 4), torch.zeros(2, 3, 4), torch.zeros(2, 3, 4))
    from hclsm_amd._lib import HipKernelError
    xg = torch.zeros(1, 2, 8, device="cuda")
    with pytest.raises(HipKernelError, match="not supported"):
        ssm_scan_fn(xg, xg, torch.zeros(8, 129, device="cuda"), torch.zeros(1, 2, 129, device="cuda"),
                    torch.zeros(1, 2, 129, device="cuda"))


def test_backend_semantics():
    """Backend strings map to the reference's semantics (ssm_scan_kernel.py:412-421)."""
    from hclsm_amd.kernels import ssm_scan_fn
    d = _inputs(2, 16, 32, 8, seed=21, dt_kind="ref_test")
    args = [d[k].cuda() for k in ("x", "dt", "A_log", "B", "C")]
    raw = ssm_scan_ref(*[_np(d[k]) for k in ("x", "dt", "A_log", "B", "C")], clamp_mode="raw")
    mod = ssm_scan_ref(*[_np(d[k]) for k in ("x", "dt", "A_log", "B", "C")], clamp_mode="model")
    for be in ("auto", "triton", "hip", "parallel"):
        assert normwise_rel_err(_np(ssm_scan_fn(*args, backend=be)), raw) <= FP32_TOL
    for be in ("sequential", "no-such-backend"):
        assert normwise_rel_err(_np(ssm_scan_fn(*args, backend=be)), mod) <= FP32_TOL


@pytest.mark.parametrize("N,T,Dn", [
    (1, 1, 2),           # one step, one lane pair
    (3, 7, 5),           # odd channels (one channel per lane), T < chunk
    (2, 9, 70),          # T = chunk + 1, partial wave
    (2, 17, 130),        # second channel group holds a single active lane pair
    (1, 33, 129),        # odd channels, several chunks plus a tail
    (2, 64, 384),        # config-1 slice
])
@pytest.mark.parametrize("mode", ["raw", "model"])
def test_shapes_bf16_state16(N, T, Dn, mode):
    """bf16 I/O with d_state 16 runs the matrix-core kernel (rank-1 input term split into two
    exact bf16 halves).  The fp32 final state must match the oracle at the fp32 bar: the
    only rounding that the bf16 path adds is the bf16 output."""
    d = _inputs(N, T, Dn, 16, dtype=torch.bfloat16, seed=N * 100 + T + Dn,
                dt_kind="ref_test" if mode == "model" else "softplus")
    y, h = _run(d, mode, True, want_h=True)
    ref, href = ssm_scan_ref(_np(d["x"]), _np(d["dt"]), _np(d["A_log"]), _np(d["B"]), _np(d["C"]),
                             D=_np(d["D"]), clamp_mode=mode, return_h_final=True)
    assert y.dtype == torch.bfloat16
    assert normwise_rel_err(_np(h), href) <= FP32_TOL, "final state"
    assert normwise_rel_err(_np(y), ref) <= 5e-3, "bf16 output: one rounding, at most 2^-8 relative"


def test_bf16_state16_misaligned_pointer():
    """x starting at an odd element: the pair-load kernel does not apply and the one-channel
    form runs; results equal the aligned call bit for bit."""
    from hclsm_amd import _lib
    d = _inputs(2, 12, 64, 16, dtype=torch.bfloat16, seed=5)
    dev = "cuda"
    x, dt, A, B, C, D = (d[k].to(dev) for k in ("x", "dt", "A_log", "B", "C", "D"))
    y0 = torch.empty_like(x)
    y1 = torch.empty_like(x)
    buf = torch.empty(x.numel() + 1, dtype=torch.bfloat16, device=dev)
    buf[1:] = x.reshape(-1)
    L = _lib.lib()
    st = torch.cuda.current_stream().cuda_stream
    for xp, yp in ((x.data_ptr(), y0), (buf.data_ptr() + 2, y1)):
        _lib.check(L.hclsm_ssm_scan_fwd(xp, dt.data_ptr(), A.data_ptr(), B.data_ptr(), C.data_ptr(), D.data_ptr(),
                                        yp.data_ptr(), None, 2, 12, 64, 16, _lib.BF16, _lib.SCAN_RAW, st),
                   "hclsm_ssm_scan_fwd")
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)
    ref = ssm_scan_ref(_np(d["x"]), _np(d["dt"]), _np(d["A_log"]), _np(d["B"]), _np(d["C"]), D=_np(d["D"]),
                       clamp_mode="raw")
    assert normwise_rel_err(_np(y0), ref) <= 5e-3


def test_launch_on_current_side_stream():
    """Launches go to torch's current stream: on a side stream the result is ordered by that stream."""
    from hclsm_amd import _lib
    from hclsm_amd.kernels import ssm_scan_fn
    d = _inputs(4, 16, 64, 16, dtype=torch.bfloat16, seed=21)
    side = torch.cuda.Stream()
    args = [d[k].cuda() for k in ("x", "dt", "A_log", "B", "C")]
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        assert _lib.stream_of(args[0]) == side.cuda_stream
        y = ssm_scan_fn(*args, backend="hip")
    side.synchronize()
    ref = ssm_scan_ref(*(_np(d[k]) for k in ("x", "dt", "A_log", "B", "C")), clamp_mode="raw")
    assert normwise_rel_err(_np(y), ref) <= 5e-3


@pytest.mark.parametrize("N,T,Dn,S,dtype,tol", [
    (3, 20, 64, 16, torch.float32, FP32_TOL),    # fp32 SGPR kernel
    (2, 9, 70, 8, torch.float32, FP32_TOL),      # fp32 SGPR, one channel per lane
    (2, 33, 48, 48, torch.float32, FP32_TOL),    # generic kernel (d_state 48, the small preset's)
    (4, 64, 384, 16, torch.bfloat16, LOWP_TOL),  # bf16 matrix-core kernel, two channels per lane
    (2, 17, 129, 16, torch.bfloat16, LOWP_TOL),  # bf16 matrix-core kernel, one channel per lane
    (2, 12, 40, 8, torch.float16, LOWP_TOL),     # fp16 generic kernel
])
def test_block_scan_fused_epilogues(N, T, Dn, S, dtype, tol):
    """hclsm_ssm_block_scan_fwd: softplus / clamp of dt, the clamped scan and silu(gate) in one kernel,
    against the oracle (oracle.modules.block_scan_ref)."""
    from oracle.modules import block_scan_ref
    from hclsm_amd.kernels import ssm_block_scan
    g = torch.Generator().manual_seed(N * 1000 + T + S)
    z = torch.randn(N, T, Dn, generator=g).to(dtype)
    dt_in = (torch.randn(N, T, Dn, generator=g) * 2 - 1).to(dtype)     # softplus spans both clamps
    dt_in[0, 0, :4] = torch.tensor([30.0, -9.0, 0.5, 25.0]).to(dtype)   # threshold and lower-clamp branches
    A_log = -torch.rand(Dn, S, generator=g) * 0.5
    Bm = (torch.randn(N, T, S, generator=g) / 4).to(dtype)
    Cm = (torch.randn(N, T, S, generator=g) / 4).to(dtype)
    gate = torch.randn(N, T, Dn, generator=g).to(dtype)
    y = ssm_block_scan(*(t.cuda() for t in (z, dt_in, A_log, Bm, Cm, gate)))
    ref = block_scan_ref(*(_np(t) for t in (z, dt_in, A_log, Bm, Cm, gate)))
    assert y.dtype == dtype
    assert normwise_rel_err(_np(y), ref) <= tol


def test_block_scan_gradients_match_float64_autograd():
    """Backward of the fused block scan (HIP reverse scan + chain rule through softplus / clamp / silu)
    against float64 torch autograd of the same math on the CPU."""
    import torch.nn.functional as F
    from hclsm_amd.kernels import ssm_block_scan
    g = torch.Generator().manual_seed(77)
    N, T, Dn, S = 2, 24, 32, 16
    z, dt_in, gate = (torch.randn(N, T, Dn, generator=g, dtype=torch.float64) for _ in range(3))
    dt_in = dt_in * 2 - 1
    A_log = -torch.rand(Dn, S, generator=g, dtype=torch.float64) * 0.5
    Bm, Cm = (torch.randn(N, T, S, generator=g, dtype=torch.float64) / 4 for _ in range(2))
    w = torch.randn(N, T, Dn, generator=g, dtype=torch.float64)
    ins = [t.float().cuda().requires_grad_() for t in (z, dt_in, A_log, Bm, Cm, gate)]
    (ssm_block_scan(*ins) * w.float().cuda()).sum().backward()
    r = [t.clone().requires_grad_() for t in (z, dt_in, A_log, Bm, Cm, gate)]
    dt = F.softplus(r[1]).clamp(1e-3, 1.0)
    A = -torch.exp(r[2]).clamp(1e-6, 1.0)
    h = torch.zeros(N, Dn, S, dtype=torch.float64)
    ys = []
    for t in range(T):
        h = torch.exp((dt[:, t, :, None] * A).clamp(-20.0, 0.0)) * h + (dt[:, t] * r[0][:, t])[:, :, None] * r[3][:, t, None, :]
        ys.append((h * r[4][:, t, None, :]).sum(-1))
    ((torch.stack(ys, 1) * F.silu(r[5])) * w).sum().backward()
    for got, ref, name in zip(ins, r, ("z", "dt_in", "A_log", "B", "C", "gate")):
        assert normwise_rel_err(_np(got.grad), _np(ref.grad)) <= 1e-5, name


def test_block_scan_bf16_gradient_at_the_lower_dt_clamp():
    """bf16 dt_in = -6.90625 gives softplus = 1.0006e-3 in fp32: inside the clamp's closed interval
    [1e-3, 1], so dt_in receives gradient (dt = softplus), although the value rounded to bf16
    (0.000999451) would sit below it.  The backward recomputes clamp(softplus(dt_in)) in fp32 as the
    forward does; the float64 reference of the same math on the bf16 inputs must agree."""
    import torch.nn.functional as F
    from hclsm_amd.kernels import ssm_block_scan
    g = torch.Generator().manual_seed(78)
    N, T, Dn, S = 2, 16, 64, 16
    bf = torch.bfloat16
    z, gate = (torch.randn(N, T, Dn, generator=g).to(bf) for _ in range(2))
    dt_in = torch.full((N, T, Dn), -6.90625).to(bf)
    dt_in[:, :, ::2] = torch.tensor(-7.5).to(bf)          # below the clamp: no gradient there
    A_log = -torch.rand(Dn, S, generator=g) * 0.5
    Bm, Cm = ((torch.randn(N, T, S, generator=g) / 4).to(bf) for _ in range(2))
    w = torch.randn(N, T, Dn, generator=g)
    ins = [t.cuda().requires_grad_() for t in (z, dt_in, A_log, Bm, Cm, gate)]
    (ssm_block_scan(*ins).float() * w.cuda()).sum().backward()
    r = [t.double().clone().requires_grad_() for t in (z, dt_in, A_log, Bm, Cm, gate)]
    sp = F.softplus(r[1])
    assert bool(((sp[:, :, 1::2] >= 1e-3) & (sp[:, :, 1::2] < 1.0034e-3)).all())
    dt = sp.clamp(1e-3, 1.0)
    A = -torch.exp(r[2]).clamp(1e-6, 1.0)
    h = torch.zeros(N, Dn, S, dtype=torch.float64)
    ys = []
    for t in range(T):
        h = torch.exp(dt[:, t, :, None] * A) * h + (dt[:, t] * r[0][:, t])[:, :, None] * r[3][:, t, None, :]
        ys.append((h * r[4][:, t, None, :]).sum(-1))
    ((torch.stack(ys, 1) * F.silu(r[5])) * w.double()).sum().backward()
    gd = ins[1].grad.float().cpu()
    assert bool((gd[:, :, 1::2] != 0).all()) and bool((gd[:, :, ::2] == 0).all())
    for got, ref, name in zip(ins, r, ("z", "dt_in", "A_log", "B", "C", "gate")):
        assert normwise_rel_err(_np(got.grad), _np(ref.grad)) <= LOWP_TOL, name


@pytest.mark.parametrize("S", [96, 128])
@pytest.mark.parametrize("dtype,tol", [(torch.float32, FP32_TOL), (torch.bfloat16, LOWP_TOL)])
def test_large_d_state_forward(S, dtype, tol):
    """d_state up to 128 (the large preset uses 96): the generic kernel splits a channel's states over
    adjacent lanes."""
    for mode in ("raw", "model"):
        d = _inputs(3, 21, 70, S, dtype=dtype, seed=S + 1, dt_kind="ref_test" if mode == "model" else "softplus")
        y, h = _run(d, mode, True, want_h=True)
        ref, href = ssm_scan_ref(_np(d["x"]), _np(d["dt"]), _np(d["A_log"]), _np(d["B"]), _np(d["C"]),
                                 D=_np(d["D"]), clamp_mode=mode, return_h_final=True)
        assert normwise_rel_err(_np(y), ref) <= tol, mode
        assert normwise_rel_err(_np(h), href) <= max(tol, 1e-5), mode


def test_large_preset_level0_block_runs():
    """The large preset's SimplifiedSSMBlock shape (d_state 96, the split-lane instantiation): the block output
    matches the oracle, and all six gradients of the fused block scan (dt recomputed in the kernel as
    clamp(softplus(dt_in), 1e-3, 1)) match float64 autograd of the same math at the fp32 bar."""
    import torch.nn.functional as F
    from oracle.modules import block_scan_ref
    from hclsm_amd.kernels import ssm_block_scan
    g = torch.Generator().manual_seed(96)
    N, T, Dn, S = 2, 12, 96, 96
    z, gate = (torch.randn(N, T, Dn, generator=g) for _ in range(2))
    dt_in = torch.randn(N, T, Dn, generator=g) * 2 - 1
    A_log = -torch.rand(Dn, S, generator=g) * 0.5
    Bm, Cm = (torch.randn(N, T, S, generator=g) / 4 for _ in range(2))
    w = torch.randn(N, T, Dn, generator=g)
    ins = [t.cuda().requires_grad_() for t in (z, dt_in, A_log, Bm, Cm, gate)]
    y = ssm_block_scan(*ins)
    ref = block_scan_ref(*(_np(t) for t in (z, dt_in, A_log, Bm, Cm, gate)))
    assert normwise_rel_err(_np(y), ref) <= FP32_TOL
    (y * w.cuda()).sum().backward()
    r = [t.double().clone().requires_grad_() for t in (z, dt_in, A_log, Bm, Cm, gate)]
    dt = F.softplus(r[1]).clamp(1e-3, 1.0)
    A = -torch.exp(r[2]).clamp(1e-6, 1.0)
    h = torch.zeros(N, Dn, S, dtype=torch.float64)
    ys = []
    for t in range(T):
        h = torch.exp(dt[:, t, :, None] * A) * h + (dt[:, t] * r[0][:, t])[:, :, None] * r[3][:, t, None, :]
        ys.append((h * r[4][:, t, None, :]).sum(-1))
    ((torch.stack(ys, 1) * F.silu(r[5])) * w.double()).sum().backward()
    for got, want, name in zip(ins, r, ("z", "dt_in", "A_log", "B", "C", "gate")):
        assert normwise_rel_err(_np(got.grad), _np(want.grad)) <= FP32_TOL, name
