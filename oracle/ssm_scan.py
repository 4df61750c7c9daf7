"""Oracle: selective SSM scan (forward and backward).  TEST INFRASTRUCTURE ONLY.

Restates the recurrence of the reference's ``hclsm/kernels/ssm_scan_kernel.py``:

    h_t[d,s] = exp(dt_t[d] * A[d,s]) * h_{t-1}[d,s] + dt_t[d] * B_t[s] * x_t[d]
    y_t[d]   = sum_s h_t[d,s] * C_t[s]          (+ Dskip[d] * x_t[d] if given)

in two semantic modes that the reference mixes:

  * ``clamp_mode="raw"``   -- ``parallel_ssm_scan_pytorch`` (ssm_scan_kernel.py:168-218,
    ``A = -exp(A_log)`` at :191) and the Triton kernel ``_ssm_scan_fwd_kernel``
    (:227-290, ``A_neg = -exp(A)`` at :255, no clamps).
  * ``clamp_mode="model"`` -- ``sequential_ssm_scan`` (:42-86) and the inline scan of
    ``SimplifiedSSMBlock.forward`` (dynamics/level0_ssm.py:82-101):
    ``A = -clamp(exp(A_log), 1e-6, 1)`` (:63), ``dt = clamp(dt, 1e-3, 1)`` (:68),
    ``dA = exp(clamp(dt*A, -20, 0))`` (:77).

The skip term ``Dskip`` exists in no reference path; the benchmark configurations add
it (y_t += D * x_t) and it defaults to absent.

All arithmetic is float64 unless ``dtype`` says otherwise; inputs are upcast first.
Shapes follow the reference: x, dt (N, T, D); A_log (D, S); B, C (N, T, S).
"""

from __future__ import annotations

import numpy as np

_A_MIN, _A_MAX = 1e-6, 1.0       # ssm_scan_kernel.py:63
_DT_MIN, _DT_MAX = 1e-3, 1.0     # ssm_scan_kernel.py:68
_ARG_MIN, _ARG_MAX = -20.0, 0.0  # ssm_scan_kernel.py:77


def _prep(x, dt, A_log, B, C, clamp_mode, dtype):
    x = np.asarray(x, dtype=dtype)
    dt = np.asarray(dt, dtype=dtype)
    A_log = np.asarray(A_log, dtype=dtype)
    B = np.asarray(B, dtype=dtype)
    C = np.asarray(C, dtype=dtype)
    if clamp_mode == "raw":
        A = -np.exp(A_log)                                   # :191 / :255
        dtc = dt
    elif clamp_mode == "model":
        A = -np.clip(np.exp(A_log), _A_MIN, _A_MAX)          # :63
        dtc = np.clip(dt, _DT_MIN, _DT_MAX)                  # :68
    else:
        raise ValueError(f"clamp_mode must be 'raw' or 'model', got {clamp_mode!r}")
    return x, dtc, A_log, A, B, C


def _gate(dtc_t, A, clamp_mode):
    arg = dtc_t[:, :, None] * A[None, :, :]                  # (N, D, S)
    if clamp_mode == "model":
        arg = np.clip(arg, _ARG_MIN, _ARG_MAX)               # :77
    return np.exp(arg)


def ssm_scan_ref(x, dt, A_log, B, C, D=None, clamp_mode="raw", dtype=np.float64,
                 return_h_final=False):
    """Sequential scan over T, vectorised over (N, D, S).

    Follows ``sequential_ssm_scan`` (ssm_scan_kernel.py:42-86) step for step; with
    ``clamp_mode="raw"`` the clamps are dropped as in :191 and :255-283.
    Returns y (N, T, D) in ``dtype`` (and h_final (N, D, S) as the Triton kernel
    stores at :289-290 when ``return_h_final``).
    """
    x, dtc, _, A, B, C = _prep(x, dt, A_log, B, C, clamp_mode, dtype)
    N, T, Dn = x.shape
    S = B.shape[-1]
    h = np.zeros((N, Dn, S), dtype=dtype)                    # :73
    y = np.empty((N, T, Dn), dtype=dtype)
    for t in range(T):                                       # :75
        dA = _gate(dtc[:, t], A, clamp_mode)                 # :77
        dB = dtc[:, t, :, None] * B[:, t, None, :]           # :78
        h = dA * h + dB * x[:, t, :, None]                   # :80
        y[:, t] = (h * C[:, t, None, :]).sum(axis=-1)        # :81
    if D is not None:
        y += np.asarray(D, dtype=dtype)[None, None, :] * x
    if return_h_final:
        return y, h
    return y


def ssm_scan_scalar_ref(x, dt, A_log, B, C, D=None, clamp_mode="raw"):
    """Brute-force scalar loops in pure Python float arithmetic (tiny inputs only).

    An implementation independent of ``ssm_scan_ref``'s vectorisation, used to pin it.
    """
    import math
    x = np.asarray(x, dtype=np.float64)
    dt = np.asarray(dt, dtype=np.float64)
    A_log = np.asarray(A_log, dtype=np.float64)
    B = np.asarray(B, dtype=np.float64)
    C = np.asarray(C, dtype=np.float64)
    N, T, Dn = x.shape
    S = B.shape[-1]
    y = np.zeros((N, T, Dn))
    for n in range(N):
        for d in range(Dn):
            h = [0.0] * S
            for t in range(T):
                dtv = float(dt[n, t, d])
                if clamp_mode == "model":
                    dtv = min(max(dtv, _DT_MIN), _DT_MAX)
                acc = 0.0
                for s in range(S):
                    e = math.exp(float(A_log[d, s]))
                    if clamp_mode == "model":
                        e = min(max(e, _A_MIN), _A_MAX)
                    arg = dtv * (-e)
                    if clamp_mode == "model":
                        arg = min(max(arg, _ARG_MIN), _ARG_MAX)
                    h[s] = math.exp(arg) * h[s] + dtv * float(B[n, t, s]) * float(x[n, t, d])
                    acc += h[s] * float(C[n, t, s])
                if D is not None:
                    acc += float(D[d]) * float(x[n, t, d])
                y[n, t, d] = acc
    return y


def blelloch_scan_ref(gates, tokens):
    """Work-efficient (Brent-Kung up-sweep / down-sweep) scan of h_t = g_t*h_{t-1} + b_t.

    Restates ``_parallel_associative_scan`` (ssm_scan_kernel.py:93-165): pad T to a
    power of two with gate 1 / token 0 (:114-120), up-sweep (:126-141), down-sweep
    (:154-163).  gates, tokens: (N, T, ...).  Returns h (N, T, ...).
    """
    g = np.array(gates, dtype=np.float64, copy=True)
    b = np.array(tokens, dtype=np.float64, copy=True)
    N, T = g.shape[:2]
    if T == 1:
        return b
    Tp = 1
    while Tp < T:
        Tp *= 2
    if Tp != T:
        pad = [(0, 0), (0, Tp - T)] + [(0, 0)] * (g.ndim - 2)
        g = np.pad(g, pad, constant_values=1.0)
        b = np.pad(b, pad, constant_values=0.0)
    levels = Tp.bit_length() - 1
    for lv in range(levels):                                  # up-sweep
        stride = 2 ** (lv + 1)
        idx = np.arange(stride - 1, Tp, stride)
        src = idx - stride // 2
        b_new = b.copy()
        g_new = g.copy()
        b_new[:, idx] = g[:, idx] * b[:, src] + b[:, idx]
        g_new[:, idx] = g[:, idx] * g[:, src]
        b, g = b_new, g_new
    for lv in range(levels - 2, -1, -1):                      # down-sweep
        stride = 2 ** (lv + 1)
        half = stride // 2
        idx = np.arange(stride + half - 1, Tp, stride)
        src = idx - half
        if len(idx):
            b_new = b.copy()
            b_new[:, idx] = g[:, idx] * b[:, src] + b[:, idx]
            b = b_new
    return b[:, :T]


def parallel_scan_ref(x, dt, A_log, B, C):
    """Raw-mode scan through the Blelloch restatement (ssm_scan_kernel.py:168-218)."""
    x = np.asarray(x, np.float64)
    dt = np.asarray(dt, np.float64)
    A = -np.exp(np.asarray(A_log, np.float64))
    B = np.asarray(B, np.float64)
    C = np.asarray(C, np.float64)
    N, T, Dn = x.shape
    S = B.shape[-1]
    dA = np.exp(dt[..., None] * A[None, None])                # :201
    dBx = (dt[..., None] * B[:, :, None, :]) * x[..., None]   # :203
    h = blelloch_scan_ref(dA.reshape(N, T, -1), dBx.reshape(N, T, -1)).reshape(N, T, Dn, S)
    return (h * C[:, :, None, :]).sum(-1)                     # :214


def ssm_scan_bwd_ref(x, dt, A_log, B, C, gy, D=None, clamp_mode="raw"):
    """Reverse scan: gradients of sum(gy * y) w.r.t. (x, dt, A_log, B, C, D).

    Raw mode follows ``_TritonSSMScan.backward`` (ssm_scan_kernel.py:321-377): recompute
    all h (:336-338), then walk t backwards accumulating grad_h (:348-373) and finish
    with the chain rule through A = -exp(A_log) (:375).  Model mode is the autograd of
    ``sequential_ssm_scan``: every clamp passes gradient only where its input lies in
    the closed clamp interval (torch's clamp backward).
    Returns a dict of float64 arrays (``D`` only if D was given).
    """
    x, dtc, A_log64, A, B, C = _prep(x, dt, A_log, B, C, clamp_mode, np.float64)
    gy = np.asarray(gy, np.float64)
    dt64 = np.asarray(dt, np.float64)
    N, T, Dn = x.shape
    S = B.shape[-1]
    hs = np.zeros((T + 1, N, Dn, S))
    gates = np.empty((T, N, Dn, S))
    for t in range(T):
        gates[t] = _gate(dtc[:, t], A, clamp_mode)
        hs[t + 1] = gates[t] * hs[t] + dtc[:, t, :, None] * B[:, t, None, :] * x[:, t, :, None]
    gh = np.zeros((N, Dn, S))
    gx = np.zeros_like(x)
    gdtc = np.zeros_like(x)
    gB = np.zeros_like(B)
    gC = np.zeros_like(C)
    gA = np.zeros((Dn, S))
    for t in range(T - 1, -1, -1):
        gh = gh + gy[:, t, :, None] * C[:, t, None, :]
        gC[:, t] = (gy[:, t, :, None] * hs[t + 1]).sum(axis=1)
        g_gate = gh * hs[t]
        g_arg = g_gate * gates[t]
        if clamp_mode == "model":
            arg = dtc[:, t, :, None] * A[None]
            g_arg = g_arg * ((arg >= _ARG_MIN) & (arg <= _ARG_MAX))
        gdtc[:, t] = (g_arg * A[None]).sum(-1) + (gh * B[:, t, None, :]).sum(-1) * x[:, t]
        gA += (g_arg * dtc[:, t, :, None]).sum(0)
        gx[:, t] = (gh * B[:, t, None, :]).sum(-1) * dtc[:, t]
        gB[:, t] = (gh * (dtc[:, t] * x[:, t])[:, :, None]).sum(1)
        gh = gh * gates[t]
    e = np.exp(A_log64)
    if clamp_mode == "model":
        gA_log = gA * (-e) * ((e >= _A_MIN) & (e <= _A_MAX))
        gdt = gdtc * ((dt64 >= _DT_MIN) & (dt64 <= _DT_MAX))
    else:
        gA_log = gA * (-e)
        gdt = gdtc
    out = {"x": gx, "dt": gdt, "A_log": gA_log, "B": gB, "C": gC}
    if D is not None:
        Dv = np.asarray(D, np.float64)
        out["x"] = gx + gy * Dv[None, None, :]
        out["D"] = (gy * x).sum(axis=(0, 1))
    return out


def normwise_rel_err(got, ref):
    """max|got - ref| / max|ref| -- the tolerance measure used for float parity."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.abs(ref).max() if ref.size else 0.0
    num = np.abs(got - ref).max() if ref.size else 0.0
    return float(num / den) if den > 0 else float(num)
