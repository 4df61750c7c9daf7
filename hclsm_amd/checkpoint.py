"""Reference training checkpoints into the hot-path modules.

The reference trainer saves ``step_N.pt`` as ``{"model": state_dict, "optimizer": ..., "scheduler": ...,
"scaler": ..., "global_step": int, "is_fsdp": bool}`` with ``torch.save``
(hclsm/training/distributed.py:295-304; FSDP saves the full, unwrapped state dict).  The modules here keep
the reference's module trees and parameter names, so their slices of that state dict load unchanged:

    slot_attention.*, target_slot_attention.*  -> hclsm_amd.objects.DynamicSlotAttention (model.py:72, :123)
    slot_tracker.*                             -> hclsm_amd.objects.SlotTracker           (model.py:74)
    relation_graph.*                           -> hclsm_amd.objects.RelationGraph         (model.py:75)
    level0_ssm.*                               -> hclsm_amd.dynamics.Level0SSM            (model.py:82)
    level1_event.*                             -> hclsm_amd.dynamics.Level1EventDynamics  (model.py:89)
    hierarchy_manager.*                        -> hclsm_amd.dynamics.HierarchyManager     (model.py:91-93)

Files are read with ``torch.load(weights_only=True)``: nothing stored in them is executed.  A checkpoint
that the safe loader refuses (for instance a scheduler state holding a pickled callable) is reported, not
loaded another way; ``read_model_state`` also accepts an already-loaded state dict.
"""

from __future__ import annotations

from pathlib import Path
from types import SimpleNamespace

import torch

# Hot-path fields of the reference presets (hclsm/config.py:193-290 and the dataclass defaults :31-83).
PRESETS = {
    "tiny": dict(d_world=256, d_slot=128, n_max_slots=16, n_iterations=3, d_edge=64, gnn_rounds=1, d_state=32,
                 n_blocks=2, l1=(256, 2, 4), l2_d_model=384),
    "small": dict(d_world=384, d_slot=192, n_max_slots=32, n_iterations=5, d_edge=96, gnn_rounds=2, d_state=48,
                  n_blocks=3, l1=(384, 3, 6), l2_d_model=512),
    "base": dict(d_world=768, d_slot=256, n_max_slots=64, n_iterations=7, d_edge=128, gnn_rounds=2, d_state=64,
                 n_blocks=4, l1=(512, 4, 8), l2_d_model=768),
    "large": dict(d_world=1024, d_slot=384, n_max_slots=128, n_iterations=7, d_edge=192, gnn_rounds=3, d_state=96,
                  n_blocks=6, l1=(768, 6, 12), l2_d_model=1024),
}

_WRAPPER_PREFIXES = ("module.", "_orig_mod.", "_fsdp_wrapped_module.")


def preset_config(name: str) -> SimpleNamespace:
    """An HCLSMConfig-shaped namespace with the hot-path fields of a reference preset."""
    p = PRESETS[name]
    d_model, n_layers, n_heads = p["l1"]
    return SimpleNamespace(
        d_world=p["d_world"],
        objects=SimpleNamespace(d_slot=p["d_slot"], n_max_slots=p["n_max_slots"], n_iterations=p["n_iterations"],
                                existence_threshold=0.5, birth_threshold=0.7, d_edge=p["d_edge"],
                                gnn_rounds=p["gnn_rounds"]),
        dynamics=SimpleNamespace(
            level0=SimpleNamespace(d_state=p["d_state"], n_blocks=p["n_blocks"], expand_ratio=2),
            level1=SimpleNamespace(d_model=d_model, n_layers=n_layers, n_heads=n_heads),
            level2=SimpleNamespace(d_model=p["l2_d_model"])))


def _strip(key: str) -> str:
    changed = True
    while changed:
        changed = False
        for pre in _WRAPPER_PREFIXES:
            if key.startswith(pre):
                key, changed = key[len(pre):], True
        key = key.replace("._fsdp_wrapped_module.", ".").replace("._checkpoint_wrapped_module.", ".")
    return key


def read_model_state(source) -> dict:
    """The model state dict of a reference checkpoint: a path to ``step_N.pt`` (loaded with
    weights_only=True), the loaded checkpoint dict, or a bare state dict.  Wrapper prefixes (DDP
    ``module.``, torch.compile ``_orig_mod.``, FSDP ``_fsdp_wrapped_module.``) are removed."""
    if isinstance(source, (str, Path)):
        try:
            ckpt = torch.load(str(source), map_location="cpu", weights_only=True)
        except Exception as e:   # the safe loader refused the file: report it, do not fall back
            raise RuntimeError(f"{source}: torch.load(weights_only=True) refused the checkpoint ({e}); "
                               "it is not loaded any other way") from e
    else:
        ckpt = source
    state = ckpt["model"] if isinstance(ckpt, dict) and isinstance(ckpt.get("model"), dict) else ckpt
    if not isinstance(state, dict):
        raise ValueError("no model state dict in the checkpoint")
    return {_strip(k): v for k, v in state.items()}


def module_state(state: dict, prefix: str) -> dict:
    """The entries of one submodule (``prefix.``) with the prefix removed."""
    pre = prefix + "."
    return {k[len(pre):]: v for k, v in state.items() if k.startswith(pre)}


def build_hot_path(source, config, device="cuda", with_target: bool = False) -> dict:
    """Construct the hot-path modules for ``config`` (HCLSMConfig-shaped: ``d_world``, ``objects``,
    ``dynamics.level0/level1/level2``) and load their weights from a reference checkpoint (strict: every
    parameter of each module must be present with the reference's name and shape).  Returns a dict
    keyed by the reference's attribute names."""
    from hclsm_amd.dynamics import HierarchyManager, Level0SSM, Level1EventDynamics
    from hclsm_amd.objects import DynamicSlotAttention, RelationGraph, SlotTracker
    state = read_model_state(source)
    d_slot = config.objects.d_slot
    mods = {
        "slot_attention": DynamicSlotAttention(config.objects, config.d_world),
        "slot_tracker": SlotTracker(config.objects),
        "relation_graph": RelationGraph(config.objects),
        "level0_ssm": Level0SSM(config.dynamics.level0, d_slot),
        "level1_event": Level1EventDynamics(config.dynamics.level1, d_slot),
        "hierarchy_manager": HierarchyManager(d_slot, config.dynamics.level2.d_model),
    }
    if with_target:
        mods["target_slot_attention"] = DynamicSlotAttention(config.objects, config.d_world)
    for name, m in mods.items():
        sub = module_state(state, name)
        if not sub:
            raise KeyError(f"checkpoint has no '{name}.' entries")
        m.load_state_dict(sub, strict=True)
        m.to(device).eval()
    return mods
