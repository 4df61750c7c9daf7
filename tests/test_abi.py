"""The C-ABI library loads without a GPU and exports every entry point of include/hclsm_amd.h.

No compute calls here (there is no GPU in the CPU test environment); argument
validation that happens before any launch is exercised with NULL device pointers.
"""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "hclsm_amd.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hclsm_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from hclsm_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("libhclsm_amd.so not built (run python -m hclsm_amd.build)")
    return _lib.lib()


def test_header_declares_entry_points():
    names = _declared()
    assert "hclsm_ssm_scan_fwd" in names and "hclsm_abi_version" in names


def test_every_declared_symbol_is_exported(lib):
    from hclsm_amd import _lib
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (hclsm_[a-z0-9_]+)$", out, flags=re.M))
    missing = [n for n in _declared() if n not in exported]
    assert not missing, f"declared in the header but not exported: {missing}"
    for n in _declared():
        assert hasattr(lib, n)
    # the Python binding declares argtypes for exactly the header's entry points
    assert sorted(_lib.exported_symbols()) == _declared()


def test_version_and_strerror(lib):
    from hclsm_amd import _lib
    assert lib.hclsm_abi_version() == _lib.ABI_VERSION == 3
    for code in (0, -1, -2, -3, -4, -5, -6):
        assert _lib.strerror(code)
    assert "unknown" in _lib.strerror(-999)


def test_argument_errors_before_launch(lib):
    f = lib.hclsm_ssm_scan_fwd
    # negative size, bad dtype, bad mode, oversized d_state, NULL pointer: all rejected on the host
    assert f(None, None, None, None, None, None, None, None, -1, 4, 4, 4, 0, 0, None) == -2
    assert f(None, None, None, None, None, None, None, None, 1, 4, 4, 4, 7, 0, None) == -3
    assert f(None, None, None, None, None, None, None, None, 1, 4, 4, 4, 0, 9, None) == -5
    assert f(None, None, None, None, None, None, None, None, 1, 4, 4, 129, 0, 0, None) == -4
    assert f(None, None, None, None, None, None, None, None, 1, 4, 4, 4, 0, 0, None) == -1
    # empty problem: nothing to launch, success
    assert f(None, None, None, None, None, None, None, None, 0, 4, 4, 4, 0, 0, None) == 0


def test_scan_backward_argument_errors_before_launch(lib):
    f = lib.hclsm_ssm_scan_bwd
    null13 = [None] * 13
    # bad mode, oversized d_state, a per-sequence slab past 32-bit buffer offsets, NULL pointers
    assert f(*null13, 1, 4, 4, 4, 1, 7, None, 0, None) == -5
    assert f(*null13, 1, 4, 4, 4, 1, 2, None, 0, None) == -1   # block mode is accepted
    assert f(*null13, 1, 4, 4, 129, 1, 0, None, 0, None) == -4
    assert f(*null13, 1, 1 << 20, 1 << 10, 16, 1, 0, None, 0, None) == -4   # 2^30 bf16 elements = 2 GiB
    assert f(*null13, 1, 4, 4, 4, 1, 0, None, 0, None) == -1


def test_level1_forward_argument_errors_before_launch(lib):
    f = lib.hclsm_level1_forward
    ws = lib.hclsm_level1_forward_workspace
    assert ws(-1, 4, 64, 256, 1) == -2
    assert ws(4, 4, 64, 256, 9) == -3
    assert ws(0, 4, 64, 256, 1) >= 0
    args = dict(ev=None, evd=0, out=None, outd=0, n=None, cap=4, N=8, rows=None, om=None, ds=64, dm=64, H=4,
                hid=256, L=1, params=None, fold=None, eps=1e-5, dt=1, ws=None, wsb=0, st=None)

    def call(**kw):
        a = {**args, **kw}
        return f(a["ev"], a["evd"], a["out"], a["outd"], a["n"], a["cap"], a["N"], a["rows"], a["om"], a["ds"], a["dm"],
                 a["H"], a["hid"], a["L"], a["params"], a["fold"], a["eps"], a["dt"], a["ws"], a["wsb"], a["st"])
    assert call(dm=60, H=4) == -4            # head dim 15: unsupported
    assert call(dm=64, H=3) == -2            # d_model not a multiple of n_heads
    assert call(dt=7) == -3                  # compute dtype
    assert call(evd=2) == -3                 # ev dtype neither F32 nor the compute dtype
    assert call(ds=48) == -4                 # d_slot not a multiple of 32 for 16-bit operands
    assert call() == -1                      # NULL pointers
    assert call(cap=0) == 0                  # nothing to do


def test_slot_tracker_argument_errors_before_launch(lib):
    assert lib.hclsm_slot_track_cost_workspace(-1, 32, 192, 1) == -2
    assert lib.hclsm_slot_track_cost_workspace(2, 32, 96, 1) == -4       # d_slot not a multiple of 64
    assert lib.hclsm_slot_track_cost_workspace(2, 32, 448, 0) == -4      # d_slot above 384
    assert lib.hclsm_slot_track_cost_workspace(2, 32, 192, 9) == -3
    assert lib.hclsm_slot_track_cost_workspace(2, 200, 192, 1) > 0        # the pair MLP has no slot limit
    assert lib.hclsm_slot_track_sequence_workspace(2, 8, 129, 192, 0, 1) == -4   # Sinkhorn: N <= 128
    assert lib.hclsm_slot_track_sequence_workspace(2, 8, 128, 192, 1, 1) > \
        lib.hclsm_slot_track_sequence_workspace(2, 8, 128, 192, 0, 1)              # room for the GRU carry
    f = lib.hclsm_slot_track_cost
    assert f(None, None, None, None, None, 2, 32, 192, None, 1, None, 0, None) == -1
    assert f(None, None, None, None, None, 0, 32, 192, None, 1, None, 0, None) == 0
    assert f(None, None, None, None, None, 2, 32, 100, None, 1, None, 0, None) == -4
    m = lib.hclsm_slot_track_match
    assert m(None, None, None, None, None, None, 2, 129, 20, 0.05, None) == -4
    assert m(None, None, None, None, None, None, 2, 32, -1, 0.05, None) == -2
    assert m(None, None, None, None, None, None, 2, 32, 20, 0.05, None) == -1
    assert m(None, None, None, None, None, None, 0, 32, 20, 0.05, None) == 0
    s = lib.hclsm_slot_track_sequence
    assert s(*[None] * 7, 2, 8, 32, 192, 20, 0.05, None, 1, None, 0, None) == -1
    assert s(*[None] * 7, 2, 8, 32, 192, -1, 0.05, None, 1, None, 0, None) == -2
    assert s(*[None] * 7, 2, 0, 32, 192, 20, 0.05, None, 1, None, 0, None) == 0
    r = lib.hclsm_slot_track_reorder_update
    assert r(*[None] * 6, 2, 32, 192, None, 1, None, 0, None) == -1
    assert r(*[None] * 6, 2, 32, 64, None, 5, None, 0, None) == -3


def test_top_down_argument_errors_before_launch(lib):
    assert lib.hclsm_event_top_down_workspace(-1, 192) == -2
    assert lib.hclsm_event_top_down_workspace(32, 192) == 2 * 32 * 192 * 4
    f = lib.hclsm_event_top_down
    P = 256   # stand-in address: every call below returns before anything is launched

    def call(B=2, T=8, N=32, D=192, dtype=1, ev=P, kpad=0, offs=P, ctx=None, S2=4, DL2=512, wx=P, ldw=192,
             ws=P, ws_bytes=1 << 20):
        return f(P, ev, offs, P, kpad, ctx, S2, DL2, P, P, None, wx, ldw, None, P, B, T, N, D, dtype, ws,
                 ws_bytes, None)
    assert call(B=-1) == -2
    assert call(kpad=-1) == -2
    assert call(dtype=9) == -3
    assert call(D=100) == -4                              # d_slot not a multiple of 32
    assert call(D=416) == -4                              # d_slot above 384
    assert call(B=0) == 0                                 # nothing to do
    assert call(ev=None) == -1
    assert call(offs=None) == -1                          # packed rows need the offsets
    assert call(ctx=P, S2=0) == -2
    assert call(ctx=P, DL2=16385) == -4                   # the mean context exceeds 64 KB of LDS
    assert call(ctx=P, wx=None) == -1
    assert call(ctx=P, ldw=100) == -2
    assert call(ctx=P, ws_bytes=16) == -2
    assert call(ctx=P, wx=P + 2) == -4                    # operand rows must be 16-byte aligned


def test_noalloc_forward_rejects_oversized_shapes_before_launch(lib):
    """hclsm_slot_attention_forward_noalloc: a shape whose workspace exceeds the static scratch array
    (64 MiB) returns HCLSM_ERR_SCRATCH (-6) on the host; negative sizes return HCLSM_ERR_SHAPE."""
    f = lib.hclsm_slot_attention_forward_noalloc
    need = lib.hclsm_slot_attention_workspace(512, 32, 196, 384, 384, 768, 1)
    assert need > (64 << 20)
    assert f(None, None, 384, None, None, 512, 32, 196, 384, 768, 3, 0.05, 0.0, 1e-8, 0.0, 1, None) == -6
    assert f(None, None, 384, None, None, -1, 32, 196, 384, 768, 3, 0.05, 0.0, 1e-8, 0.0, 1, None) == -2


def test_slot_keys_offsets(lib):
    """hclsm_slot_attention_k_offset / _kq_offset (host arithmetic, no launch): kq is formed only by 16-bit
    forwards whose iterations take the fused core (slot widths 128, 192, 256, 384, up to 32 slots), elsewhere
    HCLSM_ERR_UNSUPPORTED; both offsets sit inside the workspace and apart from each other; bad shapes and dtypes
    are rejected."""
    from hclsm_amd import _lib
    args = (32, 32, 196, 384, 384, 768)
    ws = lib.hclsm_slot_attention_workspace(*args, _lib.BF16)
    k_off = lib.hclsm_slot_attention_k_offset(*args, _lib.BF16)
    kq_off = lib.hclsm_slot_attention_kq_offset(*args, _lib.BF16)
    nb = 32 * 196 * 384 * 2
    assert 0 <= k_off and 0 <= kq_off and max(k_off, kq_off) + nb <= ws and abs(kq_off - k_off) >= nb
    assert lib.hclsm_slot_attention_kq_offset(*args, _lib.F16) >= 0
    assert lib.hclsm_slot_attention_kq_offset(*args, _lib.F32) == -4           # fp32 keeps the q projection
    assert lib.hclsm_slot_attention_kq_offset(32, 0, 196, 384, 384, 768, _lib.BF16) == -4   # no slots
    assert lib.hclsm_slot_attention_kq_offset(32, 33, 196, 384, 384, 768, _lib.BF16) == -4  # > 32 slots
    assert lib.hclsm_slot_attention_kq_offset(2, 8, 40, 64, 64, 256, _lib.BF16) == -4       # width 64
    assert lib.hclsm_slot_attention_kq_offset(-1, 8, 40, 384, 384, 768, _lib.BF16) == -2
    assert lib.hclsm_slot_attention_kq_offset(2, 8, 40, 384, 384, 768, 9) == -3


def test_scan_checkpoint_pair_argument_errors_before_launch(lib):
    """The training pair's entry points reject what they do not take on the host: modes, shapes, dtypes other
    than bf16 with d_state 16, missing or short workspaces; empty problems behave as the plain pair's."""
    fwd, blk, bwd = lib.hclsm_ssm_scan_fwd_ckpt, lib.hclsm_ssm_block_scan_fwd_ckpt, lib.hclsm_ssm_scan_bwd_ckpt
    n8, n9, n13 = [None] * 8, [None] * 9, [None] * 13
    ws_need = lib.hclsm_ssm_scan_bwd_workspace(2, 16, 64, 16)
    assert ws_need > 0
    assert fwd(*n8, 2, 16, 64, 16, 1, 2, None, 0, None) == -5        # BLOCK is the block entry's mode
    assert fwd(*n8, -1, 16, 64, 16, 1, 0, None, 0, None) == -2
    assert fwd(*n8, 2, 16, 64, 8, 1, 0, None, 0, None) == -4          # d_state 8
    assert fwd(*n8, 2, 16, 64, 16, 0, 0, None, 0, None) == -4         # fp32 I/O
    assert fwd(*n8, 2, 16, 64, 16, 1, 0, None, 0, None) == -1         # no workspace
    assert fwd(*n8, 2, 16, 64, 16, 1, 0, ctypes.c_void_p(256), ws_need - 1, None) == -2   # workspace too small
    assert fwd(*n8, 0, 16, 64, 16, 1, 0, None, 0, None) == 0          # nothing to scan
    assert blk(*n9, 2, 16, 64, 16, 1, None, 0, None) == -1
    assert blk(*n9, 2, 16, 64, 32, 1, None, 0, None) == -4
    assert blk(*n9, 0, 16, 64, 16, 1, None, 0, None) == 0
    assert bwd(*n13, 2, 16, 64, 16, 1, 0, None, 0, None) == -1
    assert bwd(*n13, 2, 16, 64, 16, 2, 0, None, 0, None) == -4        # fp16
    assert bwd(*n13, 2, 16, 64, 16, 1, 7, None, 0, None) == -5
