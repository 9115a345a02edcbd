"""Writes reference_api.json: the public call surface of the reference's drama3/offload.py and drama3/kernels.py
(module constants with their values, functions and classes with their parameter lists, methods included), read
from the source text with `ast` (nothing is imported or run). tests/test_offload_api.py checks drama3.offload and
drama3.kernels against it.

    python tests/golden/make_api_list.py [/root/reference]
"""
import ast
import json
import operator
import pathlib
import sys

MODULES = ("offload", "kernels")
SKIP = {"kernels": {"SOURCE"}}  # the NVRTC source text: a CUDA program, no part of the Python call surface
_OPS = {ast.Add: operator.add, ast.Sub: operator.sub, ast.Mult: operator.mul, ast.Div: operator.truediv,
        ast.Pow: operator.pow, ast.FloorDiv: operator.floordiv}


def value_of(node):
    """A constant expression's value (numbers, + - * / ** //, tuples), else None."""
    if isinstance(node, ast.Constant) and isinstance(node.value, (int, float)):
        return node.value
    if isinstance(node, ast.BinOp) and type(node.op) in _OPS:
        a, b = value_of(node.left), value_of(node.right)
        return None if a is None or b is None else _OPS[type(node.op)](a, b)
    if isinstance(node, ast.Tuple):
        items = [value_of(e) for e in node.elts]
        return None if any(v is None for v in items) else items
    return None


def params(fn):
    """[[name, kind, default source or null], ...] in inspect.Parameter's kind names."""
    a = fn.args
    out = []
    positional = a.posonlyargs + a.args
    defaults = [None] * (len(positional) - len(a.defaults)) + list(a.defaults)
    for arg, d in zip(positional, defaults):
        kind = "POSITIONAL_ONLY" if arg in a.posonlyargs else "POSITIONAL_OR_KEYWORD"
        out.append([arg.arg, kind, None if d is None else ast.unparse(d)])
    if a.vararg:
        out.append([a.vararg.arg, "VAR_POSITIONAL", None])
    for arg, d in zip(a.kwonlyargs, a.kw_defaults):
        out.append([arg.arg, "KEYWORD_ONLY", None if d is None else ast.unparse(d)])
    if a.kwarg:
        out.append([a.kwarg.arg, "VAR_KEYWORD", None])
    return out


def surface(path, skip):
    tree = ast.parse(pathlib.Path(path).read_text())
    api = {"constants": {}, "functions": {}, "classes": {}}
    for node in tree.body:
        if isinstance(node, ast.Assign):
            names = [t.id for t in node.targets if isinstance(t, ast.Name)]
            names += [e.id for t in node.targets if isinstance(t, ast.Tuple) for e in t.elts if isinstance(e, ast.Name)]
            value = value_of(node.value)
            if len(names) > 1 and isinstance(value, list):
                pairs = zip(names, value)
            else:
                pairs = [(n, value) for n in names]
            for n, v in pairs:
                if not n.startswith("_") and n not in skip:
                    api["constants"][n] = v
        elif isinstance(node, ast.FunctionDef) and not node.name.startswith("_"):
            api["functions"][node.name] = params(node)
        elif isinstance(node, ast.ClassDef) and not node.name.startswith("_"):
            methods = {m.name: params(m) for m in node.body if isinstance(m, ast.FunctionDef)
                       and (not m.name.startswith("_") or m.name == "__init__")}
            api["classes"][node.name] = {"bases": [ast.unparse(b) for b in node.bases], "methods": methods}
    return api


def main():
    root = pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    api = {m: surface(root / "drama3" / f"{m}.py", SKIP.get(m, set())) for m in MODULES}
    out = pathlib.Path(__file__).with_name("reference_api.json")
    out.write_text(json.dumps(api, indent=1, sort_keys=True) + "\n")
    print(f"wrote {out}")


if __name__ == "__main__":
    main()
