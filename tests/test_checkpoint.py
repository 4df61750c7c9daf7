"""Reference training checkpoints (step_N.pt, hclsm/training/distributed.py:295-304) into the hot-path
modules: safe loading (weights_only), wrapper-prefix stripping, strict name/shape matching.  CPU only:
the modules are constructed and loaded, nothing is launched."""

from __future__ import annotations

import pytest
import torch

from hclsm_amd.checkpoint import build_hot_path, module_state, preset_config, read_model_state


def _reference_shaped_model_state(seed=0):
    """A model state dict with the reference's key layout for the hot-path modules (plus unrelated
    entries that must be ignored), from freshly initialised modules of the tiny preset."""
    from hclsm_amd.dynamics import HierarchyManager, Level0SSM, Level1EventDynamics
    from hclsm_amd.objects import DynamicSlotAttention, RelationGraph, SlotTracker
    torch.manual_seed(seed)
    cfg = preset_config("tiny")
    mods = {"slot_attention": DynamicSlotAttention(cfg.objects, cfg.d_world),
            "target_slot_attention": DynamicSlotAttention(cfg.objects, cfg.d_world),
            "slot_tracker": SlotTracker(cfg.objects),
            "relation_graph": RelationGraph(cfg.objects),
            "level0_ssm": Level0SSM(cfg.dynamics.level0, cfg.objects.d_slot),
            "level1_event": Level1EventDynamics(cfg.dynamics.level1, cfg.objects.d_slot),
            "hierarchy_manager": HierarchyManager(cfg.objects.d_slot, cfg.dynamics.level2.d_model)}
    state = {f"{n}.{k}": v.clone() for n, m in mods.items() for k, v in m.state_dict().items()}
    state["perception.patch_embed.weight"] = torch.randn(8, 8)
    state["position_head.bias"] = torch.randn(3)
    return cfg, state


def _checkpoint(state):
    return {"model": state,
            "optimizer": {"state": {0: {"step": torch.tensor(3.0), "exp_avg": torch.zeros(4)}},
                          "param_groups": [{"lr": 1e-4, "betas": (0.9, 0.95), "params": [0]}]},
            "scheduler": {"last_epoch": 3, "_step_count": 4, "base_lrs": [1e-4]},
            "scaler": None, "global_step": 7, "is_fsdp": False}


def test_build_hot_path_from_reference_checkpoint(tmp_path):
    cfg, state = _reference_shaped_model_state()
    path = tmp_path / "step_7.pt"
    torch.save(_checkpoint(state), path)
    mods = build_hot_path(path, cfg, device="cpu", with_target=True)
    assert set(mods) == {"slot_attention", "target_slot_attention", "slot_tracker", "relation_graph", "level0_ssm",
                         "level1_event", "hierarchy_manager"}
    for name, m in mods.items():
        for k, v in m.state_dict().items():
            assert torch.equal(v, state[f"{name}.{k}"]), f"{name}.{k}"


def test_wrapper_prefixes_are_stripped():
    _, state = _reference_shaped_model_state(1)
    wrapped = {f"module._orig_mod.{k}": v for k, v in state.items()}
    wrapped = {k.replace("level1_event.", "level1_event._fsdp_wrapped_module."): v for k, v in wrapped.items()}
    got = read_model_state({"model": wrapped})
    assert set(got) == set(state)
    assert module_state(got, "level0_ssm").keys() == module_state(state, "level0_ssm").keys()


def test_strict_names_and_shapes(tmp_path):
    cfg, state = _reference_shaped_model_state(2)
    missing = {k: v for k, v in state.items() if not k.startswith("level1_event.")}
    with pytest.raises(KeyError, match="level1_event"):
        build_hot_path(_checkpoint(missing), cfg, device="cpu")
    bad = dict(state)
    bad["level0_ssm.condition_proj.weight"] = torch.zeros(3, 3)
    with pytest.raises(RuntimeError, match="size mismatch"):
        build_hot_path(_checkpoint(bad), cfg, device="cpu")


def _a_scheduler_lambda(step):   # pickled by reference: the safe loader must refuse it
    return 1.0


def test_unsafe_checkpoint_is_refused(tmp_path):
    _, state = _reference_shaped_model_state(3)
    ck = _checkpoint(state)
    ck["scheduler"] = {"lr_lambdas": [_a_scheduler_lambda]}
    path = tmp_path / "step_1.pt"
    torch.save(ck, path)
    with pytest.raises(RuntimeError, match="weights_only"):
        read_model_state(path)


def test_presets_match_reference_configs():
    """hclsm/config.py:193-290: the hot-path fields of the four presets."""
    for name, d_slot, slots, l1 in (("tiny", 128, 16, (256, 2, 4)), ("small", 192, 32, (384, 3, 6)),
                                    ("base", 256, 64, (512, 4, 8)), ("large", 384, 128, (768, 6, 12))):
        c = preset_config(name)
        assert (c.objects.d_slot, c.objects.n_max_slots) == (d_slot, slots)
        assert (c.dynamics.level1.d_model, c.dynamics.level1.n_layers, c.dynamics.level1.n_heads) == l1


@pytest.mark.parametrize("preset", ["tiny", "small", "base", "large"])
def test_module_trees_match_the_reference_modules(preset):
    """State-dict keys and shapes of every hot-path module, and the preset's hot-path config fields, against
    the reference's own modules built from its presets (tests/golden/reference_state_names.json, written by
    tests/golden/make_reference_state_names.py from hclsm/config.py and the reference module classes)."""
    import json
    from pathlib import Path
    from hclsm_amd.checkpoint import PRESETS
    from hclsm_amd.dynamics import HierarchyManager, Level0SSM, Level1EventDynamics
    from hclsm_amd.objects import DynamicSlotAttention, RelationGraph, SlotTracker
    ref = json.loads((Path(__file__).resolve().parent / "golden" / "reference_state_names.json").read_text())[preset]
    p = PRESETS[preset]
    rc = ref["config"]
    assert {k: p[k] for k in ("d_world", "d_slot", "n_max_slots", "n_iterations", "d_edge", "gnn_rounds", "d_state",
                              "n_blocks", "l2_d_model")} == {k: rc[k] for k in ("d_world", "d_slot", "n_max_slots",
                                                                              "n_iterations", "d_edge", "gnn_rounds",
                                                                              "d_state", "n_blocks", "l2_d_model")}
    assert list(p["l1"]) == rc["l1"] and rc["expand_ratio"] == 2
    cfg = preset_config(preset)
    ob, dy = cfg.objects, cfg.dynamics
    mods = {"slot_attention": DynamicSlotAttention(ob, cfg.d_world), "slot_tracker": SlotTracker(ob),
            "relation_graph": RelationGraph(ob), "level0_ssm": Level0SSM(dy.level0, ob.d_slot),
            "level1_event": Level1EventDynamics(dy.level1, ob.d_slot),
            "hierarchy_manager": HierarchyManager(ob.d_slot, dy.level2.d_model)}
    for name, m in mods.items():
        got = {k: list(v.shape) for k, v in m.state_dict().items()}
        assert got == ref["modules"][name], name
