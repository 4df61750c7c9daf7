"""Counterpart of the reference's hclsm/objects/dynamic_slots.py on the hot path."""

from hclsm_amd.objects.dynamic_slots import DynamicSlotAttention

__all__ = ["DynamicSlotAttention"]
