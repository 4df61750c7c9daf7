"""GPU parity of the slot-attention kernels (hclsm_slot_attn_core, hclsm_layer_norm, hclsm_linear,
hclsm_gru_cell) and the full iteration against oracle/slot_attention.py.

Tolerances (normwise relative): fp32 1e-5; bf16 operands with fp32 accumulation 2e-2."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import slot_attention as sa
from oracle.ssm_scan import normwise_rel_err

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("B,N,M,D", [(2, 16, 64, 128), (1, 8, 32, 64), (4, 32, 196, 256), (3, 32, 196, 384),
                                     (48, 32, 196, 384)])   # the last fills the device: the wide-grid kernels
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_core_matches_oracle(B, N, M, D, dtype, tol):
    from hclsm_amd.kernels import naive_slot_attention, slot_attention_fn
    g = torch.Generator().manual_seed(B + N + M)
    Q, K, V = (torch.randn(s, generator=g).to(dtype) for s in ((B, N, D), (B, M, D), (B, M, D)))
    out, attn = naive_slot_attention(Q.cuda(), K.cuda(), V.cuda())
    ref_o, ref_a = sa.slot_attention_core(_np(Q), _np(K), _np(V))
    assert out.shape == (B, N, D) and attn.shape == (B, N, M) and out.dtype == dtype
    assert normwise_rel_err(_np(out), ref_o) <= tol
    assert normwise_rel_err(_np(attn), ref_a) <= tol
    out2, attn2 = slot_attention_fn(Q.cuda(), K.cuda(), V.cuda())     # Triton semantics: +1e-8
    ref_o2, _ = sa.slot_attention_core(_np(Q), _np(K), _np(V), denom_eps=1e-8)
    assert normwise_rel_err(_np(out2), ref_o2) <= tol


def test_reference_column_sums_and_dispatch():
    """tests/test_kernels.py:66-77 and :88-97 on the HIP path."""
    from hclsm_amd.kernels import naive_slot_attention, slot_attention_fn
    torch.manual_seed(0)
    for (B, N, M, D) in [(2, 16, 64, 128), (1, 8, 32, 64), (4, 32, 196, 256)]:
        Q, K, V = torch.randn(B, N, D, device="cuda"), torch.randn(B, M, D, device="cuda"), torch.randn(B, M, D, device="cuda")
        _, attn = naive_slot_attention(Q, K, V)
        cs = attn.sum(dim=1)
        assert torch.allclose(cs, torch.ones_like(cs), atol=1e-5)
        a, _ = naive_slot_attention(Q, K, V)
        b, _ = slot_attention_fn(Q, K, V, backend="naive")
        assert torch.allclose(a, b, atol=1e-5)
        _, attn_auto = slot_attention_fn(Q, K, V)
        assert torch.allclose(attn_auto.sum(1), torch.ones_like(cs), atol=1e-4)


def test_core_backward_matches_torch_autograd():
    from hclsm_amd.kernels import naive_slot_attention
    g = torch.Generator().manual_seed(7)
    Q, K, V = (torch.randn(s, generator=g, dtype=torch.float64) for s in ((2, 8, 32), (2, 20, 32), (2, 20, 32)))
    w = torch.randn(2, 8, 32, generator=g, dtype=torch.float64)
    qc, kc, vc = (t.float().cuda().requires_grad_() for t in (Q, K, V))
    out, attn = naive_slot_attention(qc, kc, vc)
    ((out * w.float().cuda()).sum() + attn.sum() * 0.5).backward()
    q64, k64, v64 = (t.clone().requires_grad_() for t in (Q, K, V))
    a64 = torch.softmax(torch.bmm(q64, k64.transpose(1, 2)) * 32 ** -0.5, dim=1)
    ((torch.bmm(a64, v64) * w).sum() + a64.sum() * 0.5).backward()
    for got, ref in ((qc.grad, q64.grad), (kc.grad, k64.grad), (vc.grad, v64.grad)):
        assert normwise_rel_err(_np(got), ref.numpy()) <= 1e-5


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_building_blocks(dtype, tol):
    from hclsm_amd.kernels import slot_iteration as si
    g = torch.Generator().manual_seed(9)
    M, K, N = 100, 96, 72
    x = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g) / 8
    b = torch.randn(N, generator=g)
    r = torch.randn(M, N, generator=g)
    xd, wd = x.to(dtype), w.to(dtype)
    st = torch.cuda.current_stream().cuda_stream
    y = si._linear(xd.cuda(), wd.cuda(), bias=b.cuda(), resid=r.cuda(), relu=True, clamp=1.5,
                   out_dtype=torch.float32, stream=st)
    ref = np.clip(np.maximum(_np(xd) @ _np(wd).T + _np(b), 0) + _np(r), -1.5, 1.5)
    assert normwise_rel_err(_np(y), ref) <= tol
    # LayerNorm prologue from fp32 rows with a large common offset (the shifted statistics matter)
    lw0, lb0 = torch.rand(K, generator=g) + 0.5, torch.randn(K, generator=g)
    xo = x * 0.5 + 40.0
    y_ln = si._linear(xo.cuda(), wd.cuda(), ln=True, ln_w=lw0.cuda(), ln_b=lb0.cuda(), out_dtype=torch.float32,
                      stream=st)
    xn = sa.layer_norm(_np(xo), _np(lw0), _np(lb0))
    if dtype != torch.float32:
        xn = _np(torch.from_numpy(xn).to(dtype))
    assert normwise_rel_err(_np(y_ln), xn @ _np(wd).T) <= tol
    lw, lb = torch.rand(K, generator=g) + 0.5, torch.randn(K, generator=g)
    ln = si._ln(x.cuda(), K, M, K, lw.cuda(), lb.cuda(), dtype, st)
    assert normwise_rel_err(_np(ln), sa.layer_norm(_np(x), _np(lw), _np(lb))) <= (1e-5 if dtype == torch.float32 else 8e-3)
    H = 64
    cell = torch.nn.GRUCell(K, H)
    xin = torch.randn(M, K, generator=g).to(dtype)
    h = torch.randn(M, H, generator=g)
    W = si.SlotWeights(dtype, H, 0, {"w_ih": cell.weight_ih.detach().to(dtype).cuda(), "w_hh": cell.weight_hh.detach().to(dtype).cuda(),
                                      "b_ih": cell.bias_ih.detach().cuda(), "b_hh": cell.bias_hh.detach().cuda()})
    hb = h.to(dtype)
    out = si._gru(xin.cuda(), hb.cuda(), h.cuda(), W, st)
    # gate products see h rounded to the operand dtype; the blend uses the fp32 h
    H_ = H
    gi = _np(xin) @ _np(W.t["w_ih"]).T + _np(cell.bias_ih)
    gh = _np(hb) @ _np(W.t["w_hh"]).T + _np(cell.bias_hh)
    rg = sa.sigmoid(gi[:, :H_] + gh[:, :H_])
    zg = sa.sigmoid(gi[:, H_:2 * H_] + gh[:, H_:2 * H_])
    ng = np.tanh(gi[:, 2 * H_:] + rg * gh[:, 2 * H_:])
    ref = (1 - zg) * ng + zg * _np(h)
    assert normwise_rel_err(_np(out), ref) <= tol


def _weights(d, hidden, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    from hclsm_amd.workloads import xavier_uniform
    w = dict(w_q=xavier_uniform((d, d), g), w_ih=xavier_uniform((3 * d, d), g) * scale,
             w_hh=xavier_uniform((3 * d, d), g) * scale, w1=xavier_uniform((hidden, d), g),
             w2=xavier_uniform((d, hidden), g), b_ih=torch.randn(3 * d, generator=g) * 0.1,
             b_hh=torch.randn(3 * d, generator=g) * 0.1, b1=torch.randn(hidden, generator=g) * 0.1,
             b2=torch.randn(d, generator=g) * 0.1, ln_pre_w=torch.rand(d, generator=g) + 0.5,
             ln_pre_b=torch.randn(d, generator=g) * 0.1, ln_mlp_w=torch.rand(d, generator=g) + 0.5,
             ln_mlp_b=torch.randn(d, generator=g) * 0.1)
    return w


@pytest.mark.parametrize("mode_name,dtype,tol", [("reference", torch.float32, 1e-5), ("config2", torch.bfloat16, 2e-2),
                                                 ("reference", torch.bfloat16, 2e-2)])
def test_iteration_matches_oracle(mode_name, dtype, tol):
    from hclsm_amd.kernels import slot_iteration as si
    d, hidden, B, N, M = 128, 512 if mode_name == "reference" else 256, 3, 16, 49
    w = _weights(d, hidden, seed=11)
    w = {n: t.to(dtype).float() if n in si._WEIGHT_KEYS else t for n, t in w.items()}
    W = si.SlotWeights.from_dict(w, dtype)
    g = torch.Generator().manual_seed(12)
    slots = torch.randn(B, N, d, generator=g)
    k = torch.randn(B, M, d, generator=g).to(dtype)
    v = torch.randn(B, M, d, generator=g).to(dtype)
    mode = si.REFERENCE_MODE if mode_name == "reference" else si.CONFIG2_MODE
    out = si.slot_attention_iteration(slots.cuda(), k.cuda(), v.cuda(), W, mode)
    kw = dict(logit_clamp=mode.logit_clamp, renorm_eps=mode.renorm_eps, slot_clamp=mode.slot_clamp)
    ref = sa.slot_iteration(_np(slots), _np(k), _np(v), {n: _np(t) for n, t in w.items()}, **kw)
    err = normwise_rel_err(_np(out), ref)
    assert err <= tol, f"{mode_name} {dtype}: {err:.3e}"


def test_config2_forward_bf16():
    """benchmark config 2: 32 frames x 196 tokens x 384, 32 slots, 3 iterations, MLP 768, bf16 weights."""
    from hclsm_amd.kernels import slot_iteration as si
    from hclsm_amd.workloads import slot_config
    tokens, slots0, w = slot_config()
    W = si.SlotWeights.from_dict(w, torch.bfloat16)
    out = si.slot_attention_forward(tokens.cuda(), slots0.cuda(), W, 3, si.CONFIG2_MODE)
    torch.cuda.synchronize()
    ref = sa.slot_attention_forward(tokens.numpy(), slots0.numpy(), {n: t.numpy() for n, t in w.items()}, 3,
                                    logit_clamp=None, renorm_eps=1e-8, slot_clamp=None)
    err = normwise_rel_err(_np(out), ref)
    assert err <= 2e-2, f"config 2 normwise err {err:.3e}"


@pytest.mark.parametrize("mode_name,dtype,B,N,M,d,d_in,hidden", [
    ("reference", torch.bfloat16, 3, 7, 50, 128, 96, 512),     # partial slot tile, logit / slot clamps
    ("config2", torch.bfloat16, 2, 64, 197, 256, 128, 256),    # 64 slots (four row tiles), M not a multiple of 32
    ("reference", torch.float16, 2, 16, 33, 64, 64, 256),
    ("config2", torch.float16, 4, 32, 196, 128, 160, 384),
])
def test_forward_iteration_matches_oracle(mode_name, dtype, B, N, M, d, d_in, hidden):
    """hclsm_slot_attention_forward with 16-bit operands (per iteration: the attention core, the GRU, the MLP;
    the q projection is folded into k Wq where the fused core takes the shape, and kept otherwise), partial tiles
    and ragged token counts; result against the oracle."""
    from hclsm_amd.kernels import slot_iteration as si
    from hclsm_amd.workloads import xavier_uniform
    g = torch.Generator().manual_seed(B * 100 + N + M)
    w = _weights(d, hidden, seed=B + N)
    w["w_k"] = xavier_uniform((d, d_in), g)
    w["w_v"] = xavier_uniform((d, d_in), g)
    w["ln_in_w"] = torch.rand(d_in, generator=g) + 0.5
    w["ln_in_b"] = torch.randn(d_in, generator=g) * 0.1
    w = {n: t.to(dtype).float() if n in si._WEIGHT_KEYS else t for n, t in w.items()}
    W = si.SlotWeights.from_dict(w, dtype)
    tokens = torch.randn(B, M, d_in, generator=g)
    slots0 = torch.randn(B, N, d, generator=g) * 0.5
    mode = si.REFERENCE_MODE if mode_name == "reference" else si.CONFIG2_MODE
    out = si.slot_attention_forward(tokens.cuda(), slots0.cuda(), W, 3, mode)
    ref = sa.slot_attention_forward(tokens.numpy(), slots0.numpy(), {n: _np(t) for n, t in w.items()}, 3,
                                    logit_clamp=mode.logit_clamp, renorm_eps=mode.renorm_eps, slot_clamp=mode.slot_clamp)
    err = normwise_rel_err(_np(out), ref)
    assert err <= 2e-2, f"{mode_name} {dtype}: {err:.3e}"


@pytest.mark.parametrize("mode_name,dtype,tol,B,N,M,d,hidden", [
    ("config2", torch.bfloat16, 2e-2, 4, 32, 196, 384, 768),   # the 16-bit forward with the LayerNorm in the core
    ("reference", torch.float32, 1e-5, 2, 8, 40, 128, 256),    # fp32: LayerNorm launches and the q projection
])
def test_forward_without_layernorm_affine(mode_name, dtype, tol, B, N, M, d, hidden):
    """hclsm_slot_attention_forward with every LayerNorm weight and bias pointer NULL (the C ABI's "no affine"):
    the result of the oracle with weights 1 and biases 0."""
    from hclsm_amd.kernels import slot_iteration as si
    from hclsm_amd.workloads import xavier_uniform
    g = torch.Generator().manual_seed(B * 10 + d)
    w = _weights(d, hidden, seed=d + N)
    w["w_k"] = xavier_uniform((d, d), g)
    w["w_v"] = xavier_uniform((d, d), g)
    w = {n: t.to(dtype).float() if n in si._WEIGHT_KEYS else t for n, t in w.items()}
    ln_keys = ("ln_pre_w", "ln_pre_b", "ln_mlp_w", "ln_mlp_b", "ln_in_w", "ln_in_b")
    W = si.SlotWeights.from_dict({n: (None if n in ln_keys else t) for n, t in w.items()}, dtype)
    assert not any(n in W.t for n in ln_keys)
    ref_w = {n: _np(t) for n, t in w.items() if n not in ln_keys}
    for n in ln_keys:
        ref_w[n] = np.ones(d) if n.endswith("_w") else np.zeros(d)
    tokens = torch.randn(B, M, d, generator=g)
    slots0 = torch.randn(B, N, d, generator=g) * 0.5
    mode = si.REFERENCE_MODE if mode_name == "reference" else si.CONFIG2_MODE
    out = si.slot_attention_forward(tokens.cuda(), slots0.cuda(), W, 2, mode)
    ref = sa.slot_attention_forward(tokens.numpy(), slots0.numpy(), ref_w, 2, logit_clamp=mode.logit_clamp,
                                    renorm_eps=mode.renorm_eps, slot_clamp=mode.slot_clamp)
    err = normwise_rel_err(_np(out), ref)
    assert err <= tol, f"{mode_name} {dtype}: {err:.3e}"


@pytest.mark.parametrize("mode_name,dtype,B,N,M,d", [
    ("config2", torch.bfloat16, 3, 32, 196, 384),    # config 2's per-frame shape: 8 column blocks of 48, GRU hidden side in the core
    ("reference", torch.bfloat16, 2, 5, 1, 384),     # one token, a partial slot tile (one 16-slot tile, hidden side in the core)
    ("config2", torch.float16, 2, 16, 256, 256),     # the longest token count the fused core takes
    ("config2", torch.float16, 2, 32, 100, 384),     # fp16 operands with the hidden side in the core
    ("reference", torch.bfloat16, 4, 17, 31, 192),   # one column block, two slot tiles, ragged tokens
    ("config2", torch.bfloat16, 2, 32, 257, 128),    # past the fused core's token limit: the two-launch core
])
def test_fused_attention_core_shapes(mode_name, dtype, B, N, M, d):
    """The iteration's attention core (one launch per iteration for 16-bit operands, N <= 32, M <= 256,
    d in {128, 192, 256, 384}: the slot LayerNorm formed in the core against k Wq, and at d = 384 the GRU's
    hidden-side products too) inside the forward, against the oracle."""
    from hclsm_amd.kernels import slot_iteration as si
    from hclsm_amd.workloads import xavier_uniform
    g = torch.Generator().manual_seed(B * 1000 + N * 10 + M)
    w = _weights(d, 2 * d, seed=N + d)
    w["w_k"] = xavier_uniform((d, d), g)
    w["w_v"] = xavier_uniform((d, d), g)
    w["ln_in_w"] = torch.ones(d)
    w["ln_in_b"] = torch.zeros(d)
    w = {n: t.to(dtype).float() if n in si._WEIGHT_KEYS else t for n, t in w.items()}
    W = si.SlotWeights.from_dict(w, dtype)
    tokens = torch.randn(B, M, d, generator=g)
    slots0 = torch.randn(B, N, d, generator=g) * 0.5
    mode = si.REFERENCE_MODE if mode_name == "reference" else si.CONFIG2_MODE
    out = si.slot_attention_forward(tokens.cuda(), slots0.cuda(), W, 2, mode)
    ref = sa.slot_attention_forward(tokens.numpy(), slots0.numpy(), {n: _np(t) for n, t in w.items()}, 2,
                                    logit_clamp=mode.logit_clamp, renorm_eps=mode.renorm_eps, slot_clamp=mode.slot_clamp)
    err = normwise_rel_err(_np(out), ref)
    assert err <= 2e-2, f"{mode_name} {dtype} N={N} M={M} d={d}: {err:.3e}"


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2e-2), (torch.float16, 2e-2)])
def test_large_linear_lds_tiles(dtype, tol):
    """hclsm_linear at a size that takes the LDS-staged 64x64-tile kernel (>= 2048 32x32 tiles), with
    bias, ReLU, residual and clamp, ragged M and N, and K not a multiple of the 128-wide chunk."""
    from hclsm_amd.kernels import slot_iteration as si
    g = torch.Generator().manual_seed(31)
    M, N, K = 2085, 1040, 416
    x = torch.randn(M, K, generator=g).to(dtype)
    w = (torch.randn(N, K, generator=g) / 16).to(dtype)
    b = torch.randn(N, generator=g)
    r = torch.randn(M, N, generator=g)
    st = torch.cuda.current_stream().cuda_stream
    y = si._linear(x.cuda(), w.cuda(), bias=b.cuda(), resid=r.cuda(), relu=True, clamp=2.0, out_dtype=torch.float32,
                   stream=st)
    ref = np.clip(np.maximum(_np(x) @ _np(w).T + _np(b), 0) + _np(r), -2.0, 2.0)
    assert normwise_rel_err(_np(y), ref) <= tol


@pytest.mark.parametrize("dtype,tol,M,N,K", [
    (torch.bfloat16, 2e-2, 8200, 1040, 416),    # 128x128 LDS tiles: N >= 768, >= 512 tiles; ragged M, N; K tail
    (torch.float16, 2e-2, 8200, 1040, 416),
    (torch.float32, 1e-5, 2085, 1040, 420),     # fp32 LDS-staged tiles (float4 operands), K tail of 4
    (torch.bfloat16, 2e-2, 8200, 1040, 448),    # 128x128 tiles, K a whole number of 64-wide chunks; ragged M, N
    (torch.float16, 2e-2, 8200, 272, 1536),     # 64x64 tiles, long K (12 chunks), a partial column tile
])
def test_large_linear_wide_tiles(dtype, tol, M, N, K):
    """hclsm_linear at sizes that take the 128x128-tile 16-bit kernel and the fp32 LDS kernel, with bias,
    ReLU, residual and clamp."""
    from hclsm_amd.kernels import slot_iteration as si
    g = torch.Generator().manual_seed(32)
    x = torch.randn(M, K, generator=g).to(dtype)
    w = (torch.randn(N, K, generator=g) / 16).to(dtype)
    b = torch.randn(N, generator=g)
    r = torch.randn(M, N, generator=g)
    st = torch.cuda.current_stream().cuda_stream
    y = si._linear(x.cuda(), w.cuda(), bias=b.cuda(), resid=r.cuda(), relu=True, clamp=2.0, out_dtype=torch.float32,
                   stream=st)
    ref = np.clip(np.maximum(_np(x) @ _np(w).T + _np(b), 0) + _np(r), -2.0, 2.0)
    assert normwise_rel_err(_np(y), ref) <= tol


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_large_linear_wide_tiles_16bit_out(dtype):
    """The 128x128-tile kernel with fp32 output plus the 16-bit shadow copy (Y2), and with 16-bit output: each
    equals the oracle's product (rounded once for the 16-bit copies), and the copies agree bit for bit."""
    from hclsm_amd.kernels import slot_iteration as si
    g = torch.Generator().manual_seed(33)
    M, N, K = 4100, 1152, 384
    x = torch.randn(M, K, generator=g).to(dtype)
    w = (torch.randn(N, K, generator=g) / 16).to(dtype)
    b = torch.randn(N, generator=g)
    st = torch.cuda.current_stream().cuda_stream
    y, y2 = si._linear(x.cuda(), w.cuda(), bias=b.cuda(), out_dtype=torch.float32, shadow=True, stream=st)
    ref = _np(x) @ _np(w).T + _np(b)
    assert normwise_rel_err(_np(y), ref) <= 1e-5 * 10
    assert normwise_rel_err(_np(y2.float()), ref) <= 2e-2
    assert torch.equal(y.to(dtype), y2)
    yb = si._linear(x.cuda(), w.cuda(), bias=b.cuda(), out_dtype=dtype, stream=st)
    assert torch.equal(yb, y2)


@pytest.mark.parametrize("D,pad", [(96, 0), (384, 0), (384, 4), (1000, 0), (1024, 0), (97, 0), (384, 1), (1030, 0),
                                   (4, 0), (256, 0), (512, 0)])
@pytest.mark.parametrize("io", [(torch.float32, torch.float32), (torch.float32, torch.bfloat16),
                                (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16)])
@pytest.mark.parametrize("M", [37, 8203])
def test_layer_norm_rows(D, pad, io, M):
    """hclsm_layer_norm over row widths taking the vector kernel (D % 4 == 0, D <= 1024, aligned rows: one to four
    4-element units per lane, a wave per row, or with more than 8192 rows and D <= 512 a half-wave per row, the
    last wave half empty at an odd row count) and the scalar one (odd widths, unaligned row strides, D > 1024),
    rows with a large common offset (20; 2 at 8203 rows, whose lowest-variance 4-wide rows lose more than 1e-5 to
    the fp32 rounding of a mean near 20 in any fp32 LayerNorm), against the float64 LayerNorm."""
    from hclsm_amd.kernels import slot_iteration as si
    din, dout = io
    g = torch.Generator().manual_seed(D + pad + M)
    ldx = D + pad
    x = (torch.randn(M, ldx, generator=g) * 0.5 + (20.0 if M < 1000 else 2.0)).to(din)
    w, b = torch.rand(D, generator=g) + 0.5, torch.randn(D, generator=g)
    print(f"layer_norm M={M} D={D} pad={pad} io={io}", flush=True)
    y = si._ln(x.cuda(), ldx, M, D, w.cuda(), b.cuda(), dout, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    want = sa.layer_norm(_np(x[:, :D]), _np(w), _np(b))
    tol = 1e-5 if dout == torch.float32 and din == torch.float32 else 8e-3
    assert normwise_rel_err(_np(y), want) <= tol


@pytest.mark.parametrize("name", ["w_hh", "w_qkv", "w1_n"])
def test_forward_rejects_misaligned_weights_before_any_launch(name):
    """16-bit weights are read with 16-byte loads; a weight pointer off that alignment (W_hh, or the optional
    [W_q^T W_k; W_v] or W1 diag(gamma), moved by one element through the C ABI) is rejected with HCLSM_ERR_UNSUPPORTED before any
    launch: the output buffer keeps its contents."""
    import ctypes
    from hclsm_amd import _lib
    from hclsm_amd.kernels import slot_iteration as si
    from hclsm_amd.workloads import slot_config
    tokens, slots0, w = slot_config(B=2, M=24, N=8)
    W = si.SlotWeights.from_dict(w, torch.bfloat16)
    d = W.d
    wt = W.t[name]
    shifted = torch.empty(wt.numel() + 8, dtype=torch.bfloat16, device="cuda")
    shifted[1:1 + wt.numel()].copy_(wt.reshape(-1))
    st = si._struct(W)
    setattr(st, name, shifted.data_ptr() + 2)                     # 2 bytes past a 16-byte boundary
    L = _lib.lib()
    x, s0 = tokens.cuda().contiguous(), slots0.cuda().contiguous()
    out = torch.full_like(s0, 7.0)
    B, M, d_in = x.shape
    nbytes = L.hclsm_slot_attention_workspace(B, s0.shape[1], M, d_in, d, W.hidden, _lib.BF16)
    ws = torch.empty(int(nbytes), dtype=torch.uint8, device="cuda")
    rc = L.hclsm_slot_attention_forward(ctypes.byref(st), x.data_ptr(), d_in, s0.data_ptr(), out.data_ptr(), B,
                                        s0.shape[1], M, d, W.hidden, 3, d ** -0.5, 0.0, 1e-8, 0.0, _lib.BF16,
                                        ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == -4, _lib.strerror(rc)
    assert bool((out == 7.0).all())


def test_forward_keys_with_no_slots():
    """slot_attention_forward(..., return_k=True) with no slots (N = 0) still forms the keys: they equal those of
    a call with slots, bit for bit (k = LN_in(inputs) W_k^T does not depend on the slots)."""
    from hclsm_amd.kernels import slot_iteration as si
    from hclsm_amd.workloads import slot_config
    tokens, slots0, w = slot_config(B=3, M=40, N=8)
    W = si.SlotWeights.from_dict(w, torch.bfloat16)
    x = tokens.cuda()
    _, k_ref = si.slot_attention_forward(x, slots0.cuda(), W, 3, return_k=True)
    out0, k0 = si.slot_attention_forward(x, slots0[:, :0].cuda(), W, 3, return_k=True)
    torch.cuda.synchronize()
    assert out0.shape == (3, 0, W.d) and k0.shape == k_ref.shape
    assert torch.equal(k0, k_ref)


@pytest.mark.parametrize("B,M,N,d,d_in", [(6, 196, 32, 384, 384), (3, 70, 16, 128, 96)])
def test_forward_kq_projection(B, M, N, d, d_in):
    """With the weight set's [W_q^T W_k; W_v] (w_qkv) the 16-bit forward projects the inputs straight to
    kq = k W_q and v, with no kq GEMM per call and no k.  The slots are checked against the oracle and against
    the forward without w_qkv (k projected, then k W_q); kq from both against LN_in(x) W_k^T W_q in float64."""
    from hclsm_amd.kernels import slot_iteration as si
    from hclsm_amd.workloads import slot_config, xavier_uniform
    tokens, slots0, w = slot_config(B=B, M=M, N=N, d=d, hidden=2 * d, seed=B + M)
    g = torch.Generator().manual_seed(M)
    w["w_k"] = xavier_uniform((d, d_in), g).to(torch.bfloat16).float()
    w["w_v"] = xavier_uniform((d, d_in), g).to(torch.bfloat16).float()
    w["ln_in_w"] = torch.rand(d_in, generator=g) + 0.5
    w["ln_in_b"] = torch.randn(d_in, generator=g) * 0.1
    tokens = torch.randn(B, M, d_in, generator=g) + 0.3
    W = si.SlotWeights.from_dict(w, torch.bfloat16)
    assert "w_qkv" in W.t and si.forms_kq(B, N, M, d_in, W)
    W_plain = si.SlotWeights(W.dtype, W.d, W.hidden, {n: t for n, t in W.t.items() if n != "w_qkv"})
    x, s0 = tokens.cuda(), slots0.cuda()
    out, kq = si.slot_attention_forward(x, s0, W, 3, si.CONFIG2_MODE, return_kq=True)
    out_p, kq_p = si.slot_attention_forward(x, s0, W_plain, 3, si.CONFIG2_MODE, return_kq=True)
    torch.cuda.synchronize()
    ref = sa.slot_attention_forward(tokens.numpy(), slots0.numpy(), {n: _np(t) for n, t in w.items()}, 3,
                                    logit_clamp=None, renorm_eps=1e-8, slot_clamp=None)
    assert normwise_rel_err(_np(out), ref) <= 2e-2
    assert normwise_rel_err(_np(out_p), ref) <= 2e-2
    assert normwise_rel_err(_np(out), _np(out_p)) <= 1e-2
    xn = sa.layer_norm(_np(tokens), _np(w["ln_in_w"]), _np(w["ln_in_b"]))
    kq64 = (xn @ _np(w["w_k"]).T) @ _np(w["w_q"])
    assert kq.shape == (B, M, d) and kq.dtype == torch.bfloat16
    assert normwise_rel_err(_np(kq), kq64) <= 1e-2
    assert normwise_rel_err(_np(kq_p), kq64) <= 1e-2


@pytest.mark.parametrize("B,M,N,d,hidden,dtype", [(6, 196, 32, 384, 768, torch.bfloat16),
                                                   (3, 70, 16, 128, 256, torch.float16),
                                                   (2, 40, 8, 64, 128, torch.bfloat16)])
def test_forward_norm_slots_folded_into_w1(B, M, N, d, hidden, dtype):
    """With the weight set's W1 diag(gamma), its row sums and W1 beta + b1 (w1_n, w1_n_sum, w1_n_bias), a 16-bit
    iteration takes norm_slots into the W1 launch (statistics of the slot rows formed there, no LayerNorm launch).
    gamma, beta and b1 are non-trivial and the slot rows carry a mean offset.  The slots match the oracle and the
    forward without the folded weights, and one iteration through hclsm_slot_attention_iteration matches the
    oracle's iteration."""
    from hclsm_amd.kernels import slot_iteration as si
    from hclsm_amd.workloads import slot_config
    tokens, slots0, w = slot_config(B=B, M=M, N=N, d=d, hidden=hidden, seed=B * M + d)
    g = torch.Generator().manual_seed(d + hidden)
    w["ln_mlp_w"] = torch.rand(d, generator=g) + 0.5
    w["ln_mlp_b"] = torch.randn(d, generator=g) * 0.2
    w["b1"] = torch.randn(hidden, generator=g) * 0.1
    slots0 = slots0 + 1.5
    W = si.SlotWeights.from_dict(w, dtype)
    assert "w1_n" in W.t
    W_plain = si.SlotWeights(W.dtype, W.d, W.hidden, {n: t for n, t in W.t.items() if not n.startswith("w1_n")})
    x, s0 = tokens.cuda(), slots0.cuda()
    print(f"norm fold B={B} M={M} N={N} d={d} hidden={hidden} {dtype}", flush=True)
    out = si.slot_attention_forward(x, s0, W, 3, si.CONFIG2_MODE)
    out_p = si.slot_attention_forward(x, s0, W_plain, 3, si.CONFIG2_MODE)
    torch.cuda.synchronize()
    wn = {n: _np(t) for n, t in w.items()}
    ref = sa.slot_attention_forward(tokens.numpy(), slots0.numpy(), wn, 3, logit_clamp=None, renorm_eps=1e-8,
                                    slot_clamp=None)
    assert normwise_rel_err(_np(out), ref) <= 2e-2
    assert normwise_rel_err(_np(out), _np(out_p)) <= 1e-2
    # one iteration on given keys and values
    k = torch.randn(B, M, d, generator=g).to(dtype)
    v = torch.randn(B, M, d, generator=g).to(dtype)
    it = si.slot_attention_iteration(s0, k.cuda(), v.cuda(), W, si.CONFIG2_MODE)
    torch.cuda.synchronize()
    ref_it = sa.slot_iteration(slots0.numpy(), _np(k), _np(v), wn, logit_clamp=None, renorm_eps=1e-8,
                               slot_clamp=None)
    assert normwise_rel_err(_np(it), ref_it) <= 2e-2


def test_kq_offset_only_for_fused_core_shapes():
    """hclsm_slot_attention_kq_offset is valid for 16-bit fused-core shapes only: fp32, no slots, and a slot
    width the fused core does not take give HCLSM_ERR_UNSUPPORTED, and return_kq raises there; return_k still
    gives the keys (projected through [W_k; W_v]) where w_qkv is present."""
    from hclsm_amd import _lib
    from hclsm_amd.kernels import slot_iteration as si
    from hclsm_amd.workloads import slot_config
    L = _lib.lib()
    assert L.hclsm_slot_attention_kq_offset(2, 8, 40, 384, 384, 768, _lib.BF16) >= 0
    assert L.hclsm_slot_attention_kq_offset(2, 8, 40, 384, 384, 768, _lib.F32) == -4
    assert L.hclsm_slot_attention_kq_offset(2, 0, 40, 384, 384, 768, _lib.BF16) == -4
    assert L.hclsm_slot_attention_kq_offset(2, 8, 40, 64, 64, 256, _lib.BF16) == -4
    tokens, slots0, w = slot_config(B=2, M=40, N=8)
    W32 = si.SlotWeights.from_dict(w, torch.float32)
    with pytest.raises(ValueError):
        si.slot_attention_forward(tokens.cuda(), slots0.cuda(), W32, 3, return_kq=True)
    W = si.SlotWeights.from_dict(w, torch.bfloat16)
    _, k = si.slot_attention_forward(tokens.cuda(), slots0.cuda(), W, 3, return_k=True)
    xn = sa.layer_norm(_np(tokens))
    assert normwise_rel_err(_np(k), xn @ _np(w["w_k"]).T) <= 1e-2
