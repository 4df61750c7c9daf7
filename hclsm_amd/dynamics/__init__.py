"""Counterparts of the reference's hclsm/dynamics modules on the hot path, routed through
hclsm_amd.kernels (the reference modules inline their own PyTorch versions instead)."""

from hclsm_amd.dynamics.level0_ssm import Level0SSM, SimplifiedSSMBlock
from hclsm_amd.dynamics.level1_event import EventTransformerBlock, Level1EventDynamics, SwiGLUFFN
from hclsm_amd.dynamics.hierarchy_manager import HierarchyManager, level1_events_packed
from hclsm_amd.dynamics.event_detector import event_mask_rule

__all__ = ["Level0SSM", "SimplifiedSSMBlock", "EventTransformerBlock", "Level1EventDynamics", "SwiGLUFFN",
           "HierarchyManager", "level1_events_packed", "event_mask_rule"]
