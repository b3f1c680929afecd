"""Write tests/golden/reference_kernel_imports.json, the drop-in boundary by name:

* "names": every name the reference package imports from the modules this package
  replaces (maskahead.kernels.ops, maskahead.kernels.splitk, maskahead.cache,
  maskahead.eviction), with the file:line of each import;
* "attributes": every attribute the reference's runtime modules (runtime/*.py) read or
  call on a KV-cache object (``self.cache``, a local ``cache``, or a name bound to one)
  or an eviction-state object (``self._eviction`` or a name bound to it), including
  ``getattr(obj, "name", ...)`` reads, with file:line; attributes only ever assigned are
  listed under "assigned".

So a CPU test can check that maskahead_amd provides the same names and members.  The
reference's source files are parsed as text with `ast` (nothing of the reference is
imported or run).  Run in a container that has /root/reference:

    python tests/golden/make_import_names.py [/root/reference/src/maskahead]
"""

from __future__ import annotations

import ast
import json
import sys
from pathlib import Path

MODULES = {"kernels.ops": "ops", "kernels.splitk": "splitk", "cache": "cache", "eviction": "eviction"}
# receivers, by kind: attribute chains on `self` and local names
SELF_ATTRS = {"cache": "cache", "_eviction": "eviction_state"}
LOCAL_NAMES = {"cache": "cache"}
# functions whose local `cache` is not a KV-cache object of this path
NOT_KV_CACHE = {"dynamic_cache_nbytes"}   # runtime/generation_utils.py: a transformers DynamicCache


def resolve(pkg_parts: list[str], node: ast.ImportFrom) -> str | None:
    """The module an ImportFrom names, relative to the package `maskahead`."""
    if node.level == 0:
        mod = node.module or ""
        return mod[len("maskahead."):] if mod.startswith("maskahead.") else None
    base = pkg_parts[:len(pkg_parts) - (node.level - 1)] if node.level > 1 else pkg_parts
    parts = base + ([node.module] if node.module else [])
    return ".".join(p for p in parts if p)


def receiver_kind(node: ast.AST, bound: dict[str, str]) -> str | None:
    """'cache' / 'eviction_state' when `node` is such an object's expression."""
    if isinstance(node, ast.Attribute) and isinstance(node.value, ast.Name) and node.value.id == "self":
        return SELF_ATTRS.get(node.attr)
    if isinstance(node, ast.Name):
        return bound.get(node.id, LOCAL_NAMES.get(node.id))
    return None


def scan_attributes(path: Path, rel: str, reads: dict, writes: dict) -> None:
    tree = ast.parse(path.read_text(), filename=str(path))
    for fn in ast.walk(tree):
        if not isinstance(fn, (ast.FunctionDef, ast.AsyncFunctionDef)) or fn.name in NOT_KV_CACHE:
            continue
        # names bound in this function to a receiver (st = self._eviction)
        bound: dict[str, str] = {}
        for node in ast.walk(fn):
            if isinstance(node, ast.Assign) and len(node.targets) == 1 and isinstance(node.targets[0], ast.Name):
                kind = receiver_kind(node.value, {})
                if kind:
                    bound[node.targets[0].id] = kind
        for node in ast.walk(fn):
            if isinstance(node, ast.Attribute):
                kind = receiver_kind(node.value, bound)
                if kind:
                    dst = writes if isinstance(node.ctx, ast.Store) else reads
                    dst[kind].setdefault(node.attr, []).append(f"src/maskahead/{rel}:{node.lineno}")
            elif isinstance(node, ast.Call) and isinstance(node.func, ast.Name) and node.func.id in ("getattr",
                                                                                                  "hasattr"):
                if len(node.args) >= 2 and isinstance(node.args[1], ast.Constant) and \
                        isinstance(node.args[1].value, str):
                    kind = receiver_kind(node.args[0], bound)
                    if kind:
                        reads[kind].setdefault(node.args[1].value, []).append(f"src/maskahead/{rel}:{node.lineno}")


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
    reads: dict = {"cache": {}, "eviction_state": {}}
    writes: dict = {"cache": {}, "eviction_state": {}}
    for path in sorted((root / "runtime").glob("*.py")):
        scan_attributes(path, path.relative_to(root).as_posix(), reads, writes)
    assigned = {k: {a: w for a, w in v.items() if a not in reads[k]} for k, v in writes.items()}
    return {"modules": {f"maskahead.{m}": s for m, s in MODULES.items()},
            "names": {s: dict(sorted(v.items())) for s, v in out.items()},
            "attributes": {k: dict(sorted(v.items())) for k, v in reads.items()},
            "assigned": {k: dict(sorted(v.items())) for k, v in assigned.items()}}


if __name__ == "__main__":
    src = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference/src/maskahead")
    data = main(src)
    dst = Path(__file__).resolve().parent / "reference_kernel_imports.json"
    dst.write_text(json.dumps(data, indent=1) + "\n")
    print(f"{dst}: " + ", ".join(f"{s}: {len(v)} names" for s, v in data["names"].items()) + "; "
          + ", ".join(f"{k}: {len(v)} attributes" for k, v in data["attributes"].items()))
