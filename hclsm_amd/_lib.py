"""ctypes binding of libhclsm_amd.so (the C ABI declared in include/hclsm_amd.h).

torch is imported first on purpose: torch's ROCm wheel ships its own
``libamdhip64.so`` (SONAME ``libamdhip64.so.7``), and loading it before our library
makes the dynamic linker resolve our library's HIP dependency to that same
runtime, so device pointers and ``hipStream_t`` handles from torch are valid here.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libhclsm_amd.so"

F32, BF16, F16, U8 = 0, 1, 2, 3
ABI_VERSION = 3   # HCLSM_ABI_VERSION of include/hclsm_amd.h that these bindings (struct layouts) follow
SCAN_RAW, SCAN_MODEL, SCAN_BLOCK = 0, 1, 2
ERR_UNSUPPORTED = -4   # HCLSM_ERR_UNSUPPORTED: valid arguments the entry point does not implement
EVENT_GT_HALF, EVENT_NONZERO = 0, 1
ATTN_TRACK_CAUSAL, ATTN_SLOTS = 0, 1

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float

# name -> argtypes, in header order
_SIGNATURES: dict[str, list] = {
    "hclsm_abi_version": [],
    "hclsm_strerror": [_int],
    "hclsm_ssm_scan_fwd": [_c_void_p] * 8 + [_i64] * 4 + [_int, _int, _c_void_p],
    "hclsm_ssm_block_scan_fwd": [_c_void_p] * 9 + [_i64] * 4 + [_int, _c_void_p],
    "hclsm_ssm_scan_bwd_workspace": [_i64, _i64, _i64, _i64],
    "hclsm_ssm_scan_bwd": [_c_void_p] * 13 + [_i64] * 4 + [_int, _int, _c_void_p, _i64, _c_void_p],
    "hclsm_ssm_scan_fwd_ckpt": [_c_void_p] * 8 + [_i64] * 4 + [_int, _int, _c_void_p, _i64, _c_void_p],
    "hclsm_ssm_block_scan_fwd_ckpt": [_c_void_p] * 9 + [_i64] * 4 + [_int, _c_void_p, _i64, _c_void_p],
    "hclsm_ssm_scan_bwd_ckpt": [_c_void_p] * 13 + [_i64] * 4 + [_int, _int, _c_void_p, _i64, _c_void_p],
    "hclsm_event_index": [_c_void_p, _int, _i64, _i64, _int] + [_c_void_p] * 6 + [_c_void_p],
    "hclsm_event_gather": [_c_void_p, _c_void_p, _i64, _i64, _i64, _i64] + [_c_void_p] * 3 + [_c_void_p],
    "hclsm_event_gather_packed": [_c_void_p, _c_void_p, _i64, _i64, _i64, _i64] + [_c_void_p] * 3 + [_c_void_p],
    "hclsm_event_scatter": [_c_void_p] * 3 + [_i64] * 4 + [_c_void_p, _c_void_p],
    "hclsm_event_scatter_packed": [_c_void_p] * 3 + [_i64] * 3 + [_c_void_p, _c_void_p, _c_void_p],
    "hclsm_event_top_down_workspace": [_i64, _i64],
    "hclsm_event_top_down": [_c_void_p] * 4 + [_i64, _c_void_p, _i64, _i64] + [_c_void_p] * 4 + [_i64] +
                            [_c_void_p] * 2 + [_i64] * 4 + [_int, _c_void_p, _i64, _c_void_p],
    "hclsm_event_attention": [_c_void_p] * 8 + [_i64] * 5 + [_f32, _int, _int, _c_void_p],
    "hclsm_track_causal_attention": [_c_void_p, _int, _int] + [_c_void_p] * 4 + [_i64] * 5 + [_f32, _int, _c_void_p, _c_void_p],
    "hclsm_layer_norm": [_c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _f32, _int, _int,
                         _c_void_p],
    "hclsm_linear": [_c_void_p, _i64, _int, _c_void_p, _i64, _c_void_p, _c_void_p, _i64, _c_void_p, _i64, _int,
                     _c_void_p, _i64, _i64, _i64, _i64, _int, _f32, _int, _c_void_p, _c_void_p, _f32, _int,
                     _c_void_p],
    "hclsm_gru_cell": [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p,
                       _c_void_p, _c_void_p, _i64, _c_void_p, _i64, _i64, _i64, _i64, _int, _c_void_p],
    "hclsm_slot_attn_core_workspace": [_i64, _i64, _i64, _int],
    "hclsm_slot_attn_core": [_c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p,
                             _i64, _i64, _c_void_p, _int, _i64, _i64, _i64, _i64, _f32, _f32, _f32, _f32,
                             _int, _c_void_p, _i64, _c_void_p],
    "hclsm_slot_attention_workspace": [_i64, _i64, _i64, _i64, _i64, _i64, _int],
    "hclsm_slot_attention_k_offset": [_i64, _i64, _i64, _i64, _i64, _i64, _int],
    "hclsm_slot_attention_kq_offset": [_i64, _i64, _i64, _i64, _i64, _i64, _int],
    "hclsm_slot_attention_iteration": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _c_void_p,
                                       _i64, _i64, _i64, _i64, _i64, _f32, _f32, _f32, _f32, _int, _c_void_p,
                                       _i64, _c_void_p],
    "hclsm_slot_attention_forward": [_c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64,
                                     _i64, _i64, _f32, _f32, _f32, _f32, _int, _c_void_p, _i64, _c_void_p],
    "hclsm_slot_attention_forward_noalloc": [_c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i64, _i64,
                                             _i64, _i64, _i64, _f32, _f32, _f32, _f32, _int, _c_void_p],
    "hclsm_level1_forward_workspace": [_i64, _i64, _i64, _i64, _int],
    "hclsm_relation_graph_workspace": [_i64, _i64, _i64, _i64, _int],
    "hclsm_relation_graph_forward": [_c_void_p] * 4 + [_i64] * 5 + [_int, _c_void_p, _f32, _int, _c_void_p, _i64,
                                                                    _c_void_p],
    "hclsm_level1_forward": [_c_void_p, _int, _c_void_p, _int, _c_void_p, _i64, _i64, _c_void_p, _c_void_p,
                             _i64, _i64, _i64, _i64, _i64, _c_void_p, _c_void_p, _f32, _int, _c_void_p, _i64,
                             _c_void_p],
    "hclsm_gnn_message_pass_workspace": [_i64, _i64, _i64, _i64, _int],
    "hclsm_gnn_message_pass": [_c_void_p] * 4 + [_i64] * 7 + [_c_void_p, _int, _c_void_p, _i64, _c_void_p],
    "hclsm_slot_track_cost_workspace": [_i64, _i64, _i64, _int],
    "hclsm_slot_track_cost": [_c_void_p] * 5 + [_i64] * 3 + [_c_void_p, _int, _c_void_p, _i64, _c_void_p],
    "hclsm_slot_track_match": [_c_void_p] * 6 + [_i64] * 3 + [_f32, _c_void_p],
    "hclsm_slot_track_reorder_update_workspace": [_i64, _i64, _i64, _int],
    "hclsm_slot_track_reorder_update": [_c_void_p] * 6 + [_i64] * 3 + [_c_void_p, _int, _c_void_p, _i64, _c_void_p],
    "hclsm_slot_track_sequence_workspace": [_i64, _i64, _i64, _i64, _int, _int],
    "hclsm_slot_track_sequence": [_c_void_p] * 7 + [_i64] * 5 + [_f32, _c_void_p, _int, _c_void_p, _i64, _c_void_p],
    "hclsm_issue_probe": [_int, _i64, _int, _c_void_p, _c_void_p],
}
_RESTYPES = {"hclsm_strerror": ctypes.c_char_p, "hclsm_slot_attn_core_workspace": ctypes.c_int64,
             "hclsm_ssm_scan_bwd_workspace": ctypes.c_int64,
             "hclsm_slot_attention_workspace": ctypes.c_int64, "hclsm_slot_attention_k_offset": ctypes.c_int64,
             "hclsm_slot_attention_kq_offset": ctypes.c_int64, "hclsm_level1_forward_workspace": ctypes.c_int64,
             "hclsm_relation_graph_workspace": ctypes.c_int64, "hclsm_slot_track_cost_workspace": ctypes.c_int64,
             "hclsm_slot_track_reorder_update_workspace": ctypes.c_int64,
             "hclsm_slot_track_sequence_workspace": ctypes.c_int64,
             "hclsm_event_top_down_workspace": ctypes.c_int64, "hclsm_gnn_message_pass_workspace": ctypes.c_int64}


class HclsmSlotWeights(ctypes.Structure):
    """Mirror of the C struct HclsmSlotWeights (include/hclsm_amd.h)."""
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "w_q", "w_kv", "w_ih", "w_hh", "w1", "w2", "b_ih", "b_hh", "b1", "b2",
        "ln_in_w", "ln_in_b", "ln_pre_w", "ln_pre_b", "ln_mlp_w", "ln_mlp_b", "w_qt", "w_qkv",
        "w1_n", "w1_n_sum", "w1_n_bias")]

_lib = None


class HipKernelError(RuntimeError):
    """An hclsm_amd entry point returned a non-zero code."""


def lib() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP kernels first "
                "(python -m hclsm_amd.build, or __graft_entry__.build())")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, _int)
        got = handle.hclsm_abi_version()
        if got != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI version {got}, these bindings expect {ABI_VERSION}: rebuild it "
                               "(python -m hclsm_amd.build)")
        _lib = handle
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def strerror(code: int) -> str:
    return lib().hclsm_strerror(int(code)).decode()


def check(code: int, what: str) -> None:
    if code != 0:
        raise HipKernelError(f"{what} failed: {strerror(code)} (code {code})")


def ptr(t: "torch.Tensor | None") -> int | None:
    return None if t is None else t.data_ptr()


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return F32
    if dt == torch.bfloat16:
        return BF16
    if dt == torch.float16:
        return F16
    raise TypeError(f"hclsm_amd kernels take float32/bfloat16/float16 tensors, got {dt}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of_device(device_index: int) -> int:
    """hipStream_t of torch's current stream on a device given by index."""
    if _raw_stream is not None:
        return _raw_stream(device_index)
    return torch.cuda.current_stream(device_index).cuda_stream


def stream_of(t: torch.Tensor) -> int:
    """hipStream_t of torch's current stream on t's device."""
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream
