"""Write tests/golden/reference_imports.json: every name the reference's callers import from
the hot-path modules, with the file:line of the import and the reference's signature.

The reference is only *parsed* here (``ast``), never imported or run.  For each
``from <module> import <name>`` in the reference's ``wanx/``, ``zimg/``,
``sinkattention/__init__.py`` and ``sinkattention/sparse_attention.py`` whose module is one of

* ``sinkattention``, ``sinkattention.sparse_attention``, ``sinkattention.timing``,
  ``sinkattention.pooling_kernel``  (served by the alias package ``sinkattention`` here),
* ``wanx.runtime.sink_sparse_wan``  (served by ``sinkattn_amd.wan_runtime``),
* ``zimg.runtime.sink_sparse_zimage``  (served by ``sinkattn_amd.zimage_runtime``),

the table records the name, where it is imported, what kind of object the defining module
binds to it (function, class, constant) and, for functions and classes, the parameter list
of the function / ``__init__`` / ``__call__`` as (name, kind, default source text), and a
dataclass's fields with their default source text.

Usage:  python tests/golden/make_import_table.py [/root/reference]
"""
from __future__ import annotations

import ast
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT = HERE / "reference_imports.json"

# reference module -> (defining file relative to the reference root, module serving it here)
MODULES = {
    "sinkattention": ("sinkattention/__init__.py", "sinkattention"),
    "sinkattention.sparse_attention": ("sinkattention/sparse_attention.py", "sinkattention.sparse_attention"),
    "sinkattention.timing": ("sinkattention/timing.py", "sinkattention.timing"),
    "sinkattention.pooling_kernel": ("sinkattention/pooling_kernel.py", "sinkattention.pooling_kernel"),
    "wanx.runtime.sink_sparse_wan": ("wanx/runtime/sink_sparse_wan.py", "sinkattn_amd.wan_runtime"),
    "zimg.runtime.sink_sparse_zimage": ("zimg/runtime/sink_sparse_zimage.py", "sinkattn_amd.zimage_runtime"),
}
CALLER_GLOBS = ("wanx/**/*.py", "zimg/**/*.py", "sinkattention/__init__.py",
                "sinkattention/sparse_attention.py")


def _params(fn: ast.FunctionDef) -> list:
    a = fn.args
    out = []
    pos = list(a.posonlyargs) + list(a.args)
    defaults = [None] * (len(pos) - len(a.defaults)) + list(a.defaults)
    for i, (arg, d) in enumerate(zip(pos, defaults)):
        kind = "POSITIONAL_ONLY" if i < len(a.posonlyargs) else "POSITIONAL_OR_KEYWORD"
        out.append([arg.arg, kind, None if d is None else ast.unparse(d)])
    if a.vararg is not None:
        out.append([a.vararg.arg, "VAR_POSITIONAL", None])
    for arg, d in zip(a.kwonlyargs, a.kw_defaults):
        out.append([arg.arg, "KEYWORD_ONLY", None if d is None else ast.unparse(d)])
    if a.kwarg is not None:
        out.append([a.kwarg.arg, "VAR_KEYWORD", None])
    return out


def _definition(tree: ast.Module, name: str) -> dict:
    for node in tree.body:
        if isinstance(node, (ast.FunctionDef, ast.AsyncFunctionDef)) and node.name == name:
            return {"kind": "function", "params": _params(node)}
        if isinstance(node, ast.ClassDef) and node.name == name:
            methods = {}
            for item in node.body:
                if isinstance(item, ast.FunctionDef) and item.name in ("__init__", "__call__"):
                    methods[item.name] = _params(item)
            out = {"kind": "class", "methods": methods}
            if any(ast.unparse(d).startswith("dataclass") for d in node.decorator_list):
                out["fields"] = [[item.target.id, None if item.value is None else ast.unparse(item.value)]
                                 for item in node.body
                                 if isinstance(item, ast.AnnAssign) and isinstance(item.target, ast.Name)]
            return out
        if isinstance(node, (ast.Assign, ast.AnnAssign)):
            targets = node.targets if isinstance(node, ast.Assign) else [node.target]
            if any(isinstance(t, ast.Name) and t.id == name for t in targets):
                value = node.value
                # `f = SomeFunction.apply`: an autograd Function; callers see forward(ctx, ...)
                if isinstance(value, ast.Attribute) and value.attr == "apply" and isinstance(value.value, ast.Name):
                    for cls in tree.body:
                        if isinstance(cls, ast.ClassDef) and cls.name == value.value.id:
                            for item in cls.body:
                                if isinstance(item, ast.FunctionDef) and item.name == "forward":
                                    return {"kind": "function", "params": _params(item)[1:],
                                            "via": ast.unparse(value)}
                return {"kind": "constant", "value": ast.unparse(value)}
        if isinstance(node, ast.ImportFrom):
            for alias in node.names:
                if (alias.asname or alias.name) == name:
                    return {"kind": "reexport", "from": node.module}
    raise LookupError(name)


def build(root: Path) -> list:
    trees = {m: ast.parse((root / f).read_text()) for m, (f, _) in MODULES.items()}
    rows = {}
    callers = sorted({p for g in CALLER_GLOBS for p in root.glob(g)})
    for path in callers:
        rel = str(path.relative_to(root))
        for node in ast.walk(ast.parse(path.read_text())):
            if not isinstance(node, ast.ImportFrom) or node.module not in MODULES:
                continue
            for alias in node.names:
                key = (node.module, alias.name)
                row = rows.setdefault(key, {
                    "module": node.module,
                    "serving_module": MODULES[node.module][1],
                    "name": alias.name,
                    "imported_at": [],
                    "definition": _definition(trees[node.module], alias.name),
                })
                row["imported_at"].append(f"{rel}:{node.lineno}")
    return [rows[k] for k in sorted(rows)]


def main() -> None:
    root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    table = build(root)
    OUT.write_text(json.dumps(table, indent=1) + "\n")
    print(f"wrote {len(table)} names to {OUT}")


if __name__ == "__main__":
    main()
