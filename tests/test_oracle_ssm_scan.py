"""CPU pins of the scan oracle (oracle/ssm_scan.py).

The oracle is checked against what the mathematics fixes, chosen so that a plausible
mistake (dropped term, wrong sign, clamp applied in the wrong mode, transposed
operand, off-by-one in time) fails at least one test:
  * an independent brute-force scalar implementation (tiny shapes),
  * the closed form of a constant-gate recurrence,
  * T = 1, linearity in x, causality, zero-B,
  * the Blelloch restatement of the reference's parallel scan (raw mode),
  * clamp-mode identities (model == raw where clamps are inactive; A -> -1 where
    exp(A_log) >= 1), and the reference's own test distribution where they differ,
  * central finite differences for the backward oracle.
There are no golden vectors in the reference (tests/test_kernels.py only compares
implementations on unseeded inputs), so these properties are the pins.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle.ssm_scan import (
    blelloch_scan_ref,
    normwise_rel_err,
    parallel_scan_ref,
    ssm_scan_bwd_ref,
    ssm_scan_ref,
    ssm_scan_scalar_ref,
)


def _inputs(N, T, Dn, S, seed, kind="config"):
    r = np.random.default_rng(seed)
    x = r.standard_normal((N, T, Dn))
    if kind == "config":
        dt = np.log1p(np.exp(-2 + 0.5 * r.standard_normal((N, T, Dn))))
        A_log = r.uniform(0, math.log(16), (Dn, S))
    elif kind == "ref_test":  # tests/test_kernels.py:120-128
        dt = np.abs(r.random((N, T, Dn))) + 0.01
        A_log = r.standard_normal((Dn, S))
    else:  # clamps inactive: exp(A_log) in (0.6, 1], dt in [0.01, 0.9]
        dt = r.uniform(0.01, 0.9, (N, T, Dn))
        A_log = -r.random((Dn, S)) * 0.5
    B = r.standard_normal((N, T, S)) / math.sqrt(S)
    C = r.standard_normal((N, T, S)) / math.sqrt(S)
    D = r.standard_normal(Dn)
    return x, dt, A_log, B, C, D


@pytest.mark.parametrize("mode", ["raw", "model"])
@pytest.mark.parametrize("kind", ["config", "ref_test"])
def test_vectorised_equals_scalar_bruteforce(mode, kind):
    x, dt, A_log, B, C, D = _inputs(2, 5, 3, 4, seed=1, kind=kind)
    got = ssm_scan_ref(x, dt, A_log, B, C, D=D, clamp_mode=mode)
    ref = ssm_scan_scalar_ref(x, dt, A_log, B, C, D=D, clamp_mode=mode)
    assert np.abs(got - ref).max() <= 1e-12 * max(1.0, np.abs(ref).max())


def test_constant_gate_closed_form():
    # dt, A, B, x constant over time => h_t = b (1 - a^(t+1)) / (1 - a), a = e^{dt A}, b = dt B x
    N, T, Dn, S = 1, 12, 2, 3
    dtv, xv = 0.3, 1.7
    A_log = np.log(np.array([[0.5, 1.0, 2.0], [3.0, 0.25, 1.5]]))
    Bv = np.array([0.4, -1.1, 0.8])
    x = np.full((N, T, Dn), xv)
    dt = np.full((N, T, Dn), dtv)
    B = np.broadcast_to(Bv, (N, T, S)).copy()
    C = np.ones((N, T, S))
    y = ssm_scan_ref(x, dt, A_log, B, C, clamp_mode="raw")
    A = -np.exp(A_log)
    a = np.exp(dtv * A)                       # (Dn, S)
    b = dtv * Bv[None, :] * xv                # (Dn, S)
    for t in range(T):
        h = b * (1 - a ** (t + 1)) / (1 - a)
        np.testing.assert_allclose(y[0, t], h.sum(-1), rtol=1e-12)


def test_T1_and_zero_B_and_skip():
    x, dt, A_log, B, C, D = _inputs(3, 1, 4, 5, seed=2)
    y = ssm_scan_ref(x, dt, A_log, B, C, D=D)
    expect = (C[:, 0, None, :] * dt[:, 0, :, None] * B[:, 0, None, :] * x[:, 0, :, None]).sum(-1) + D * x[:, 0]
    np.testing.assert_allclose(y[:, 0], expect, rtol=1e-12)
    y0 = ssm_scan_ref(x, dt, A_log, np.zeros_like(B), C, D=D)
    np.testing.assert_allclose(y0, D * x, rtol=1e-12)


def test_linearity_and_causality():
    x, dt, A_log, B, C, _ = _inputs(2, 9, 6, 4, seed=3)
    x2 = np.random.default_rng(9).standard_normal(x.shape)
    ya = ssm_scan_ref(2.5 * x - 0.5 * x2, dt, A_log, B, C)
    yb = 2.5 * ssm_scan_ref(x, dt, A_log, B, C) - 0.5 * ssm_scan_ref(x2, dt, A_log, B, C)
    np.testing.assert_allclose(ya, yb, rtol=1e-10, atol=1e-12)
    xp, dtp, Bp = x.copy(), dt.copy(), B.copy()
    xp[:, 5:] += 1.0
    dtp[:, 5:] *= 2.0
    Bp[:, 5:] -= 0.3
    y1 = ssm_scan_ref(x, dt, A_log, B, C)
    y2 = ssm_scan_ref(xp, dtp, A_log, Bp, C)
    np.testing.assert_array_equal(y1[:, :5], y2[:, :5])
    assert np.abs(y1[:, 5:] - y2[:, 5:]).max() > 1e-3


@pytest.mark.parametrize("T", [1, 2, 5, 8, 13, 16])
def test_blelloch_restatement_matches_sequential_raw(T):
    x, dt, A_log, B, C, _ = _inputs(2, T, 5, 3, seed=T)
    np.testing.assert_allclose(parallel_scan_ref(x, dt, A_log, B, C),
                               ssm_scan_ref(x, dt, A_log, B, C, clamp_mode="raw"), rtol=1e-10, atol=1e-12)
    g = np.random.default_rng(0).random((3, T, 4))
    b = np.random.default_rng(1).standard_normal((3, T, 4))
    h = np.zeros((3, 4))
    for t in range(T):
        h = g[:, t] * h + b[:, t]
        np.testing.assert_allclose(blelloch_scan_ref(g, b)[:, t], h, rtol=1e-12, atol=1e-14)


def test_model_equals_raw_when_clamps_inactive():
    x, dt, A_log, B, C, D = _inputs(3, 10, 7, 6, seed=4, kind="inactive")
    np.testing.assert_allclose(ssm_scan_ref(x, dt, A_log, B, C, D=D, clamp_mode="model"),
                               ssm_scan_ref(x, dt, A_log, B, C, D=D, clamp_mode="raw"), rtol=1e-12)


def test_model_clamps_A_to_minus_one_and_dt_range():
    x, dt, A_log, B, C, _ = _inputs(2, 6, 3, 4, seed=5, kind="config")   # exp(A_log) in [1, 16]
    dt_in = np.clip(dt, 1e-3, 1.0)
    y_model = ssm_scan_ref(x, dt, A_log, B, C, clamp_mode="model")
    y_raw_A1 = ssm_scan_ref(x, dt_in, np.zeros_like(A_log), B, C, clamp_mode="raw")
    np.testing.assert_allclose(y_model, y_raw_A1, rtol=1e-12)
    dt_big = dt + 2.0                                                       # clamp dt to 1
    np.testing.assert_allclose(ssm_scan_ref(x, dt_big, A_log, B, C, clamp_mode="model"),
                               ssm_scan_ref(x, np.ones_like(dt), np.zeros_like(A_log), B, C, clamp_mode="raw"),
                               rtol=1e-12)


def test_reference_test_distribution_raw_vs_model_differ():
    """The reference's test_parallel_matches_sequential (test_kernels.py:135-140) compares
    the clamped sequential scan with the unclamped parallel scan on A_log = randn; the
    two semantics genuinely disagree there, so that reference test cannot pass as written."""
    x, dt, A_log, B, C, _ = _inputs(2, 16, 32, 8, seed=6, kind="ref_test")
    e = normwise_rel_err(ssm_scan_ref(x, dt, A_log, B, C, clamp_mode="raw"),
                         ssm_scan_ref(x, dt, A_log, B, C, clamp_mode="model"))
    assert e > 1e-2


def _fd_grad(f, arr, eps=1e-6):
    g = np.zeros_like(arr)
    it = np.nditer(arr, flags=["multi_index"])
    for _ in it:
        i = it.multi_index
        old = arr[i]
        arr[i] = old + eps
        fp = f()
        arr[i] = old - eps
        fm = f()
        arr[i] = old
        g[i] = (fp - fm) / (2 * eps)
    return g


@pytest.mark.parametrize("mode", ["raw", "model"])
def test_backward_oracle_matches_finite_differences(mode):
    N, T, Dn, S = 2, 4, 3, 2
    r = np.random.default_rng(7)
    x = r.standard_normal((N, T, Dn))
    # keep every clamp input away from its boundary so the function is smooth there
    dt = r.uniform(0.05, 0.9, (N, T, Dn)) if mode == "raw" else r.choice([0.2, 0.5, 1.6], (N, T, Dn)) + r.uniform(0, 0.1, (N, T, Dn))
    A_log = r.uniform(-1.0, 1.0, (Dn, S))
    A_log[np.abs(A_log) < 0.05] = 0.3
    B = r.standard_normal((N, T, S))
    C = r.standard_normal((N, T, S))
    D = r.standard_normal(Dn)
    gy = r.standard_normal((N, T, Dn))
    grads = ssm_scan_bwd_ref(x, dt, A_log, B, C, gy, D=D, clamp_mode=mode)
    arrays = {"x": x, "dt": dt, "A_log": A_log, "B": B, "C": C, "D": D}
    loss = lambda: float((gy * ssm_scan_ref(x, dt, A_log, B, C, D=D, clamp_mode=mode)).sum())
    for name, arr in arrays.items():
        fd = _fd_grad(loss, arr)
        np.testing.assert_allclose(grads[name], fd, rtol=1e-5, atol=1e-7, err_msg=name)


def test_reference_fixture_shapes():
    """Shapes of tests/test_kernels.py:120-133 (B, T, d_inner, d_state)."""
    for (Bn, T, Dn, S) in [(2, 16, 32, 8), (1, 8, 64, 16), (4, 32, 16, 4)]:
        x, dt, A_log, B, C, _ = _inputs(Bn, T, Dn, S, seed=8, kind="ref_test")
        y = ssm_scan_ref(x, dt, A_log, B, C, clamp_mode="model")
        assert y.shape == x.shape and np.isfinite(y).all()
