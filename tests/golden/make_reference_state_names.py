"""Writes reference_state_names.json: for each reference preset (hclsm/config.py:193-290), the hot-path
fields of its config and the state-dict keys and shapes of the reference's hot-path modules, as
hclsm/model.py:73-93 builds them (DynamicSlotAttention, SlotTracker, RelationGraph, Level0SSM,
Level1EventDynamics, HierarchyManager).  The module classes are imported from /root/reference and only
constructed (no forward runs); run in the build container, where /root/reference exists:
    python tests/golden/make_reference_state_names.py"""

from __future__ import annotations

import json
import sys
from pathlib import Path

OUT = Path(__file__).resolve().parent / "reference_state_names.json"


def main() -> None:
    sys.path.insert(0, "/root/reference")
    import torch
    from hclsm.config import HCLSMConfig
    from hclsm.dynamics.hierarchy_manager import HierarchyManager
    from hclsm.dynamics.level0_ssm import Level0SSM
    from hclsm.dynamics.level1_event import Level1EventDynamics
    from hclsm.objects.dynamic_slots import DynamicSlotAttention
    from hclsm.objects.relation_graph import RelationGraph
    from hclsm.objects.slot_tracker import SlotTracker

    torch.manual_seed(0)
    out = {}
    for preset in ("tiny", "small", "base", "large"):
        cfg = getattr(HCLSMConfig, preset)()
        ob, dy = cfg.objects, cfg.dynamics
        d_slot = ob.d_slot
        mods = {"slot_attention": DynamicSlotAttention(ob, cfg.d_world), "slot_tracker": SlotTracker(ob),
                "relation_graph": RelationGraph(ob), "level0_ssm": Level0SSM(dy.level0, d_slot),
                "level1_event": Level1EventDynamics(dy.level1, d_slot),
                "hierarchy_manager": HierarchyManager(d_slot, dy.level2.d_model)}
        out[preset] = {
            "config": dict(d_world=cfg.d_world, d_slot=d_slot, n_max_slots=ob.n_max_slots,
                           n_iterations=ob.n_iterations, d_edge=ob.d_edge, gnn_rounds=ob.gnn_rounds,
                           d_state=dy.level0.d_state, n_blocks=dy.level0.n_blocks,
                           expand_ratio=dy.level0.expand_ratio,
                           l1=[dy.level1.d_model, dy.level1.n_layers, dy.level1.n_heads],
                           l2_d_model=dy.level2.d_model),
            "modules": {name: {k: list(v.shape) for k, v in m.state_dict().items()} for name, m in mods.items()},
        }
    OUT.write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
