"""Writes kernels_api_names.json: every public name of the reference's hclsm/kernels/__init__.py (:9-61), and
the names its two callers import from the kernel submodules (tests/test_kernels.py:13-33,
scripts/benchmark_kernels.py:19-33), read from the files' text with the ast module (the reference is not
imported).  Run in the build container, where /root/reference exists:
    python tests/golden/make_kernels_api_names.py"""

from __future__ import annotations

import ast
import json
from pathlib import Path

REF = Path("/root/reference")
SRC = REF / "hclsm/kernels/__init__.py"
CALLERS = ("tests/test_kernels.py", "scripts/benchmark_kernels.py")
OUT = Path(__file__).resolve().parent / "kernels_api_names.json"


def main() -> None:
    tree = ast.parse(SRC.read_text())
    imported, exported = {}, []
    for node in tree.body:
        if isinstance(node, ast.ImportFrom) and node.module and node.module.startswith("hclsm.kernels."):
            for alias in node.names:
                imported[alias.asname or alias.name] = node.module.rsplit(".", 1)[1]
        elif isinstance(node, ast.Assign) and any(isinstance(t, ast.Name) and t.id == "__all__" for t in node.targets):
            exported = [ast.literal_eval(e) for e in node.value.elts]
    callers = {}
    for rel in CALLERS:
        for node in ast.walk(ast.parse((REF / rel).read_text())):
            if isinstance(node, ast.ImportFrom) and node.module and node.module.startswith("hclsm.kernels"):
                sub = node.module[len("hclsm.kernels"):].lstrip(".") or "__init__"
                callers.setdefault(rel, {}).setdefault(sub, sorted(a.name for a in node.names))
    data = {"source": "hclsm/kernels/__init__.py", "imported": imported, "all": exported, "callers": callers}
    OUT.write_text(json.dumps(data, indent=1, sort_keys=True) + "\n")
    print(f"wrote {OUT}: {len(imported)} imported names, {len(exported)} in __all__")


if __name__ == "__main__":
    main()
