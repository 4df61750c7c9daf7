"""Drop-in counterpart of the reference's ``hclsm/kernels/__init__.py`` (:9-61).

Every public name runs on libhclsm_amd.so (gfx950 HIP).  ``TRITON_AVAILABLE`` is kept
for callers that test it and is always False: there is no Triton path here.
``HIP_AVAILABLE`` says whether the library is loadable and a ROCm GPU is visible.
"""

from __future__ import annotations

import torch

from hclsm_amd.kernels.ssm_scan_kernel import (
    ssm_scan_fn,
    ssm_block_scan,
    sequential_ssm_scan,
    parallel_ssm_scan_pytorch,
    fused_ssm_scan_triton,
    fused_ssm_scan_hip,
)

from hclsm_amd.kernels.sparse_event_attn import (
    sparse_event_attn_fn,
    naive_sparse_event_attention,
    sparse_event_attention,
    EventIndex,
    build_event_index,
    gather_events_padded,
    scatter_events_padded,
    gather_packed,
    scatter_packed,
    gather_events_packed,
    scatter_events_packed,
)

from hclsm_amd.kernels.level1_packed import Level1Weights, level1_forward_packed

from hclsm_amd.kernels.event_attention import (
    TrackCausalPlan,
    event_attention,
    track_causal_event_attention,
    slots_attention,
)

from hclsm_amd.kernels.slot_attention_kernel import (
    slot_attention_core,
    slot_attention_fn,
    naive_slot_attention,
    compiled_slot_attention,
    fused_slot_attention_triton,
    TRITON_AVAILABLE,
)
from hclsm_amd.kernels.gnn_message_pass import (
    gnn_message_pass_fn,
    naive_gnn_message_pass,
    optimized_gnn_message_pass,
    chunked_gnn_message_pass,
)
from hclsm_amd.kernels.hierarchical_state import (
    hierarchical_state_fn,
    hierarchical_state_naive,
    hierarchical_state_fused,
    hierarchical_state_streamed,
)
from hclsm_amd.kernels._common import HipFallbackWarning
from hclsm_amd.kernels.slot_iteration import (
    SlotMode,
    SlotWeights,
    REFERENCE_MODE,
    CONFIG2_MODE,
    slot_attention_iteration,
    slot_attention_forward,
)



def _hip_available() -> bool:
    try:
        from hclsm_amd import _lib
        _lib.lib()
    except Exception:
        return False
    return torch.cuda.is_available()


HIP_AVAILABLE = _hip_available()

from hclsm_amd.kernels import ops  # noqa: E402  registers the hclsm_hip:: torch.library ops

__all__ = [
    "slot_attention_core",
    "slot_attention_fn",
    "naive_slot_attention",
    "compiled_slot_attention",
    "fused_slot_attention_triton",
    "SlotMode",
    "SlotWeights",
    "REFERENCE_MODE",
    "CONFIG2_MODE",
    "slot_attention_iteration",
    "slot_attention_forward",
    "ssm_scan_fn",
    "ssm_block_scan",
    "sequential_ssm_scan",
    "parallel_ssm_scan_pytorch",
    "fused_ssm_scan_triton",
    "fused_ssm_scan_hip",
    "sparse_event_attn_fn",
    "naive_sparse_event_attention",
    "sparse_event_attention",
    "EventIndex",
    "build_event_index",
    "gather_events_padded",
    "scatter_events_padded",
    "gather_packed",
    "scatter_packed",
    "gather_events_packed",
    "scatter_events_packed",
    "Level1Weights",
    "level1_forward_packed",
    "event_attention",
    "track_causal_event_attention",
    "TrackCausalPlan",
    "slots_attention",
    "gnn_message_pass_fn",
    "naive_gnn_message_pass",
    "optimized_gnn_message_pass",
    "chunked_gnn_message_pass",
    "hierarchical_state_fn",
    "hierarchical_state_naive",
    "hierarchical_state_fused",
    "hierarchical_state_streamed",
    "HipFallbackWarning",
    "TRITON_AVAILABLE",
    "HIP_AVAILABLE",
    "ops",
]
