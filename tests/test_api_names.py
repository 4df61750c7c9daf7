"""The drop-in boundary at the Python level: every public name of the reference's hclsm/kernels/__init__.py
(:9-61) is exported by hclsm_amd.kernels, and every name the reference's two callers import from a kernel
submodule (tests/test_kernels.py:13-33, scripts/benchmark_kernels.py:19-33) exists in the submodule of the same
name here, so the sys.modules swap of the integration guide satisfies both callers' imports.  The names come
from tests/golden/kernels_api_names.json, written from the reference's source text by
tests/golden/make_kernels_api_names.py.  CPU only: nothing is launched."""

from __future__ import annotations

import importlib
import inspect
import json
from pathlib import Path

import pytest

FIXTURE = json.loads((Path(__file__).resolve().parent / "golden" / "kernels_api_names.json").read_text())


def test_fixture_is_complete():
    assert len(FIXTURE["all"]) == 17 and set(FIXTURE["all"]) == set(FIXTURE["imported"])
    assert set(FIXTURE["callers"]) == {"tests/test_kernels.py", "scripts/benchmark_kernels.py"}


@pytest.mark.parametrize("name", FIXTURE["all"])
def test_every_reference_name_is_exported(name):
    import hclsm_amd.kernels as hk
    assert hasattr(hk, name), name
    assert name in hk.__all__, name
    sub = importlib.import_module(f"hclsm_amd.kernels.{FIXTURE['imported'][name]}")
    assert hasattr(sub, name), f"{name} not in hclsm_amd.kernels.{FIXTURE['imported'][name]}"


@pytest.mark.parametrize("caller", sorted(FIXTURE["callers"]))
def test_callers_submodule_imports_resolve(caller):
    for sub, names in FIXTURE["callers"][caller].items():
        mod = importlib.import_module(f"hclsm_amd.kernels.{sub}")
        missing = [n for n in names if not hasattr(mod, n)]
        assert not missing, f"{caller}: hclsm_amd.kernels.{sub} lacks {missing}"


def test_signatures_keep_the_reference_positional_parameters():
    """The reference's positional parameters and defaults, in order (extensions are keyword-only)."""
    import hclsm_amd.kernels as hk
    want = {
        "ssm_scan_fn": ["x", "dt", "A_log", "B", "C", "backend"],
        "slot_attention_fn": ["Q", "K", "V", "scale", "backend"],
        "sparse_event_attn_fn": ["states", "event_mask", "attn_fn", "max_events", "backend"],
        "gnn_message_pass_fn": ["nodes", "alive_mask", "edge_mlp", "edge_weight_linear", "msg_mlp", "update_mlp",
                                "n_rounds", "backend", "chunk_size"],
        "chunked_gnn_message_pass": ["nodes", "alive_mask", "edge_mlp", "edge_weight_linear", "msg_mlp",
                                     "update_mlp", "n_rounds", "chunk_size"],
        "hierarchical_state_fn": ["level0_states", "event_scores", "event_threshold", "gather_fn", "level1_fn",
                                  "level2_fn", "scatter_fn", "backend"],
        "hierarchical_state_naive": ["level0_states", "event_scores", "event_threshold", "gather_fn", "level1_fn",
                                     "level2_fn", "scatter_fn"],
    }
    for name, params in want.items():
        sig = inspect.signature(getattr(hk, name))
        pos = [p.name for p in sig.parameters.values()
               if p.kind in (p.POSITIONAL_ONLY, p.POSITIONAL_OR_KEYWORD)]
        assert pos == params, f"{name}: {pos}"
    assert inspect.signature(hk.gnn_message_pass_fn).parameters["backend"].default == "auto"
    assert inspect.signature(hk.chunked_gnn_message_pass).parameters["chunk_size"].default == 16
    assert hk.TRITON_AVAILABLE is False
