"""Counterparts of the reference's hclsm/objects modules on the hot path (slot attention) and next to it
(relation graph)."""

from hclsm_amd.objects.dynamic_slots import DynamicSlotAttention
from hclsm_amd.objects.relation_graph import RelationGraph

__all__ = ["DynamicSlotAttention", "RelationGraph"]
