"""Write tests/golden/reference_kernel_imports.json: every name the reference package
imports from its kernel-op modules (maskahead.kernels.ops, maskahead.kernels.splitk),
with the file:line of each import, so that a CPU test can check that maskahead_amd
provides the same names (the drop-in boundary).

The reference's source files are parsed as text with `ast` (nothing of the reference is
imported or run).  Run in a container that has /root/reference:

    python tests/golden/make_import_names.py [/root/reference/src/maskahead]
"""

from __future__ import annotations

import ast
import json
import sys
from pathlib import Path

MODULES = {"kernels.ops": "ops", "kernels.splitk": "splitk"}


def resolve(pkg_parts: list[str], node: ast.ImportFrom) -> str | None:
    """The module an ImportFrom names, relative to the package `maskahead`."""
    if node.level == 0:
        mod = node.module or ""
        return mod[len("maskahead."):] if mod.startswith("maskahead.") else None
    base = pkg_parts[:len(pkg_parts) - (node.level - 1)] if node.level > 1 else pkg_parts
    parts = base + ([node.module] if node.module else [])
    return ".".join(p for p in parts if p)


def main(root: Path) -> dict:
    out: dict = {short: {} for short in MODULES.values()}
    for path in sorted(root.rglob("*.py")):
        rel = path.relative_to(root)
        pkg = list(rel.parts[:-1])                       # package of this file, under maskahead
        tree = ast.parse(path.read_text(), filename=str(path))
        for node in ast.walk(tree):
            if not isinstance(node, ast.ImportFrom):
                continue
            mod = resolve(pkg, node)
            short = MODULES.get(mod or "")
            if short is None:
                continue
            for alias in node.names:
                out[short].setdefault(alias.name, []).append(f"src/maskahead/{rel.as_posix()}:{node.lineno}")
    return {"modules": {f"maskahead.{m}": s for m, s in MODULES.items()},
            "names": {s: dict(sorted(v.items())) for s, v in out.items()}}


if __name__ == "__main__":
    src = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference/src/maskahead")
    data = main(src)
    dst = Path(__file__).resolve().parent / "reference_kernel_imports.json"
    dst.write_text(json.dumps(data, indent=1) + "\n")
    print(f"{dst}: " + ", ".join(f"{s}: {len(v)} names" for s, v in data["names"].items()))
