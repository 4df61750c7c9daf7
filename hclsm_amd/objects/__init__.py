"""Counterparts of the reference's hclsm/objects modules on the hot path (slot attention) and next to it
(slot tracker, relation graph)."""

from hclsm_amd.objects.dynamic_slots import DynamicSlotAttention
from hclsm_amd.objects.relation_graph import RelationGraph
from hclsm_amd.objects.slot_tracker import SlotTracker, sinkhorn_matching

__all__ = ["DynamicSlotAttention", "RelationGraph", "SlotTracker", "sinkhorn_matching"]
