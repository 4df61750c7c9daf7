"""The allocation-free slot-attention forward (hclsm_slot_attention_forward_noalloc) against
hclsm_slot_attention_forward, both called through the C ABI.

Both run the same kernels on the same inputs, so the outputs must be bitwise equal.  Two calls in a
row, the second on a smaller input (fewer frames, fewer tokens), check that nothing depends on the
state the static scratch array keeps from the previous call.  A third shape with more workspace than
the array holds must be rejected with HCLSM_ERR_SCRATCH before any launch.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

HCLSM_ERR_SCRATCH = -6
SCRATCH_BYTES = 64 << 20


def _weights(d, hidden, seed, dtype):
    from hclsm_amd.kernels import slot_iteration as si
    from hclsm_amd.workloads import slot_config
    _, _, w = slot_config(B=1, M=8, N=4, d=d, hidden=hidden, seed=seed)
    return si.SlotWeights.from_dict(w, dtype)


def _inputs(B, M, N, d, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.nn.functional.layer_norm(torch.randn(B, M, d, generator=g), (d,))
    s0 = 0.1 * torch.randn(d, generator=g) + 0.5 * torch.randn(B, N, d, generator=g)
    return x.cuda().contiguous(), s0.cuda().contiguous()


def _call(noalloc, W, x, s0, n_iter, renorm_eps):
    from hclsm_amd import _lib
    from hclsm_amd.kernels import slot_iteration as si
    L = _lib.lib()
    B, M, d_in = x.shape
    N, d = s0.shape[1], W.d
    out = torch.full_like(s0, float("nan"))
    st = si._struct(W)
    code = _lib.dtype_code(W.dtype)
    stream = torch.cuda.current_stream().cuda_stream
    common = (ctypes.byref(st), x.data_ptr(), d_in, s0.data_ptr(), out.data_ptr(), B, N, M, d, W.hidden, n_iter,
              d ** -0.5, 0.0, renorm_eps, 0.0, code)
    if noalloc:
        rc = L.hclsm_slot_attention_forward_noalloc(*common, stream)
    else:
        nbytes = L.hclsm_slot_attention_workspace(B, N, M, d_in, d, W.hidden, code)
        ws = torch.empty(int(nbytes), dtype=torch.uint8, device="cuda")
        rc = L.hclsm_slot_attention_forward(*common, ws.data_ptr(), ws.numel(), stream)
    torch.cuda.synchronize()
    assert rc == 0, _lib.strerror(rc)
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_forward_equals_workspace_forward(dtype):
    d, hidden = 384, 768
    W = _weights(d, hidden, 1002, dtype)
    # config 2, then a smaller call: fewer frames and a token count that is not a multiple of 32
    for (B, M, N, seed) in [(32, 196, 32, 11), (5, 45, 16, 12)]:
        print(f"noalloc forward dtype={dtype} B={B} M={M} N={N}", flush=True)
        x, s0 = _inputs(B, M, N, d, seed)
        ref = _call(False, W, x, s0, 3, 1e-8)
        got = _call(True, W, x, s0, 3, 1e-8)
        assert torch.isfinite(ref).all()
        assert torch.equal(got, ref)


def test_noalloc_rejects_oversized_workspace():
    from hclsm_amd import _lib
    L = _lib.lib()
    W = _weights(384, 768, 1002, torch.bfloat16)
    B, M, N, d = 512, 196, 32, 384
    need = L.hclsm_slot_attention_workspace(B, N, M, d, d, W.hidden, _lib.BF16)
    assert need > SCRATCH_BYTES
    x = torch.empty(B, M, d, device="cuda")
    s0 = torch.empty(B, N, d, device="cuda")
    st = __import__("hclsm_amd.kernels.slot_iteration", fromlist=["_struct"])._struct(W)
    rc = L.hclsm_slot_attention_forward_noalloc(ctypes.byref(st), x.data_ptr(), d, s0.data_ptr(), s0.data_ptr(), B, N,
                                                M, d, W.hidden, 3, d ** -0.5, 0.0, 1e-8, 0.0, _lib.BF16,
                                                torch.cuda.current_stream().cuda_stream)
    assert rc == HCLSM_ERR_SCRATCH
    assert "scratch" in _lib.strerror(rc)


def test_noalloc_forward_replays_under_graph_capture():
    """The allocation-free forward captured once in a graph (after a warm call, which sets up the scratch address
    and the per-device launch tables) and replayed on new inputs copied into the captured buffers: every replay,
    with eager work and synchronisations between them, equals the eager allocation-free call on the same inputs
    bit for bit.  The forward records no memset or allocation, only kernel launches and stream-ordered copies."""
    from hclsm_amd import _lib
    from hclsm_amd.kernels import slot_iteration as si
    L = _lib.lib()
    d, hidden, B, M, N = 384, 768, 8, 196, 32
    W = _weights(d, hidden, 1002, torch.bfloat16)
    x, s0 = _inputs(B, M, N, d, 21)
    out = torch.zeros_like(s0)
    st = si._struct(W)

    def launch(stream):
        return L.hclsm_slot_attention_forward_noalloc(ctypes.byref(st), x.data_ptr(), d, s0.data_ptr(), out.data_ptr(),
                                                      B, N, M, d, W.hidden, 3, d ** -0.5, 0.0, 1e-8, 0.0, _lib.BF16,
                                                      stream)
    assert launch(torch.cuda.current_stream().cuda_stream) == 0   # warm call
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    codes = []
    with torch.cuda.graph(graph):
        codes.append(launch(torch.cuda.current_stream().cuda_stream))
    assert codes == [0]
    torch.cuda.synchronize()
    for seed in (22, 23, 24):
        print(f"graph replay seed={seed}", flush=True)
        xn, sn = _inputs(B, M, N, d, seed)
        x.copy_(xn)
        s0.copy_(sn)
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        ref = _call(True, W, x, s0, 3, 1e-8)
        assert torch.isfinite(ref).all()
        assert torch.equal(got, ref)
    del graph
