"""Seeded synthetic inputs for the benchmark configurations of the hot path.

Each generator draws on the CPU from ``torch.Generator().manual_seed(1000 + cfg)``
in a fixed order, rounds to the I/O dtype, and returns CPU tensors; callers copy
the same tensors to the GPU, and checkers upcast the rounded values.

  cfg 0: scan fp32  (128, 16, 256), d_state 16, raw mode, skip D
  cfg 1: scan bf16  (1024, 64, 384), d_state 16, raw mode, skip D  (bandwidth test)
  cfg 2: fused slot attention, B=32, M=196, K=32, D=384, 3 iterations, MLP 768
  cfg 3: sparse event attention, 1024 tracks, T=64, 6 heads x 64, p=0.15, t=0 forced
  cfg 4: scan chain (1024, 1024, 768) bf16 x4 + event attention 12 x 64, p=0.05
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

SCAN_SHAPES = {
    0: dict(batch=128, T=16, d_inner=256, d_state=16, dtype=torch.float32),
    1: dict(batch=1024, T=64, d_inner=384, d_state=16, dtype=torch.bfloat16),
    4: dict(batch=1024, T=1024, d_inner=768, d_state=16, dtype=torch.bfloat16),
}


def scan_inputs(batch, T, d_inner, d_state, dtype=torch.float32, seed=1000):
    """x ~ N(0,1); dt = softplus(-2 + 0.5 N(0,1)); A_log ~ U(0, ln 16) so A in [-16,-1];
    B, C ~ N(0,1)/sqrt(d_state); D ~ N(0,1).  Returns dict of CPU tensors."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, T, d_inner, generator=g)
    dt = F.softplus(-2.0 + 0.5 * torch.randn(batch, T, d_inner, generator=g))
    A_log = torch.rand(d_inner, d_state, generator=g) * math.log(16.0)
    B = torch.randn(batch, T, d_state, generator=g) / math.sqrt(d_state)
    C = torch.randn(batch, T, d_state, generator=g) / math.sqrt(d_state)
    D = torch.randn(d_inner, generator=g)
    return dict(x=x.to(dtype), dt=dt.to(dtype), A_log=A_log, B=B.to(dtype), C=C.to(dtype), D=D)


def scan_config(cfg: int):
    s = SCAN_SHAPES[cfg]
    return scan_inputs(s["batch"], s["T"], s["d_inner"], s["d_state"], s["dtype"], seed=1000 + cfg)


def scan_algorithmic_bytes(batch, T, d_inner, d_state, io_bytes, with_D=True):
    """HBM bytes one scan must move: read x, dt, B, C, A_log (+D); write y."""
    b = 3 * batch * T * d_inner * io_bytes + 2 * batch * T * d_state * io_bytes + d_inner * d_state * 4
    if with_D:
        b += d_inner * 4
    return b


def xavier_uniform(shape, generator):
    fan_out, fan_in = shape
    bound = math.sqrt(6.0 / (fan_in + fan_out))
    return (torch.rand(shape, generator=generator) * 2 - 1) * bound


def slot_config(B=32, M=196, N=32, d=384, hidden=768, seed=1002, wdtype=torch.bfloat16):
    """benchmark config 2: tokens = LayerNorm(randn(B, M, d)) (no affine); mu ~ 0.1 N(0,1);
    slots0 = mu + 0.5 N(0,1); Xavier-uniform W_q, W_k, W_v (d x d), GRU W_ih, W_hh (3d x d),
    MLP d -> hidden -> d; biases 0, LayerNorm weight 1 / bias 0; matrices rounded to ``wdtype``.
    Returns (inputs, slots0, weights) as CPU tensors (weights already rounded, stored fp32)."""
    g = torch.Generator().manual_seed(seed)
    tokens = F.layer_norm(torch.randn(B, M, d, generator=g), (d,))
    mu = 0.1 * torch.randn(d, generator=g)
    slots0 = mu + 0.5 * torch.randn(B, N, d, generator=g)
    rnd = lambda t: t.to(wdtype).float()
    w = dict(w_q=rnd(xavier_uniform((d, d), g)), w_k=rnd(xavier_uniform((d, d), g)),
             w_v=rnd(xavier_uniform((d, d), g)), w_ih=rnd(xavier_uniform((3 * d, d), g)),
             w_hh=rnd(xavier_uniform((3 * d, d), g)), w1=rnd(xavier_uniform((hidden, d), g)),
             w2=rnd(xavier_uniform((d, hidden), g)))
    z = lambda n: torch.zeros(n)
    o = lambda n: torch.ones(n)
    w.update(b_ih=z(3 * d), b_hh=z(3 * d), b1=z(hidden), b2=z(d), ln_pre_w=o(d), ln_pre_b=z(d),
             ln_mlp_w=o(d), ln_mlp_b=z(d), ln_in_w=o(d), ln_in_b=z(d))
    return tokens, slots0, w


def slot_flops(B=32, M=196, N=32, d=384, hidden=768, n_iter=3):
    """Algorithmic FLOPs of config 2 (k/v projections once + n_iter iterations)."""
    kv = 2 * B * M * d * d * 2
    it = (2 * B * N * d * d            # q
          + 2 * B * N * M * d * 2       # logits + attn @ v
          + 2 * B * N * d * 3 * d * 2   # GRU W_ih, W_hh
          + 2 * B * N * d * hidden * 2)  # MLP
    return kv + n_iter * it


def chain_config(device, seed=1004, H=12, dh=64, p_event=0.05):
    """benchmark config 4, drawn on ``device`` (3.2 G values; a CPU draw of this size takes minutes) from
    ``torch.Generator(device).manual_seed(1004)`` in this order: x0 = N(0,1) (1024, 1024, 768);
    dt = softplus(-2 + 0.5 N(0,1)); A_log ~ U(0, ln 16) (768, 16); B, C = N(0,1)/4 (1024, 1024, 16);
    D = N(0,1) (768); event mask = U(0,1) < p_event with t=0 forced, (1024, 1024) fp32; q, k, v = N(0,1)
    (1024, 1024, H, dh).  Scan tensors and q, k, v in bf16; A_log, D and the mask fp32."""
    N, T, Dn, S = 1024, 1024, 768, 16
    g = torch.Generator(device=device).manual_seed(seed)
    bf = torch.bfloat16
    out = dict(x=torch.randn(N, T, Dn, generator=g, device=device).to(bf))
    out["dt"] = F.softplus(-2 + 0.5 * torch.randn(N, T, Dn, generator=g, device=device)).to(bf)
    out["A_log"] = torch.rand(Dn, S, generator=g, device=device) * math.log(16.0)
    out["B"] = (torch.randn(N, T, S, generator=g, device=device) / 4).to(bf)
    out["C"] = (torch.randn(N, T, S, generator=g, device=device) / 4).to(bf)
    out["D"] = torch.randn(Dn, generator=g, device=device)
    m = (torch.rand(N, T, generator=g, device=device) < p_event).float()
    m[:, 0] = 1
    out["mask"] = m
    for name in ("q", "k", "v"):
        out[name] = torch.randn(N, T, H, dh, generator=g, device=device).to(bf)
    return out
