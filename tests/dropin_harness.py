"""The reference harness's way of loading and running a drop-in module, restated for the drop-in checks.

benchmarks/ks/auto_bench.py loads a v1 file by path with only its imports, definitions and literal
assignments kept (auto_bench.py:74-98, 143-178), builds Model(*v0 init inputs) and ModelNew(*v1 init inputs)
under the same seed (384-394), copies the v0 state dict into ModelNew (518-521), and runs both on clones of
the v0 inputs under no_grad (530-533, 419-426), comparing floating outputs with allclose and integer
outputs with torch.equal (270-310).  The filter rules and the call order are the interface a drop-in must
survive, so they are kept; the code is this build's own.
"""
from __future__ import annotations

import ast
import importlib.util
import os
import sys
import types

import torch


def _literal(node) -> bool:
    if isinstance(node, ast.Constant):
        return True
    if isinstance(node, (ast.Tuple, ast.List, ast.Set)):
        return all(_literal(e) for e in node.elts)
    if isinstance(node, ast.Dict):
        return all((k is None or _literal(k)) and _literal(v) for k, v in zip(node.keys, node.values))
    if isinstance(node, ast.UnaryOp) and isinstance(node.op, (ast.UAdd, ast.USub)):
        return _literal(node.operand)
    return False


def filtered(tree: ast.Module) -> ast.Module:
    """Keep imports, classes, functions and assignments of literals; drop every other module statement."""
    keep = (ast.Import, ast.ImportFrom, ast.ClassDef, ast.FunctionDef, ast.AsyncFunctionDef)
    tree.body = [n for n in tree.body
                 if isinstance(n, keep)
                 or (isinstance(n, ast.Assign) and _literal(n.value))
                 or (isinstance(n, ast.AnnAssign) and n.value is not None and _literal(n.value))]
    ast.fix_missing_locations(tree)
    return tree


def load(path: str) -> types.ModuleType:
    """Execute the filtered module in a fresh namespace, the file's directory first on sys.path."""
    with open(path, encoding="utf-8") as f:
        tree = ast.parse(f.read(), filename=path)
    name = f"_dropin_{os.path.splitext(os.path.basename(path))[0]}_{abs(hash(os.path.abspath(path)))}"
    mod = types.ModuleType(name)
    mod.__file__ = path
    mod.__package__ = ""
    mod.__spec__ = importlib.util.spec_from_loader(name, loader=None)
    saved = list(sys.path)
    sys.modules[name] = mod
    sys.path.insert(0, os.path.dirname(os.path.abspath(path)))
    try:
        exec(compile(filtered(tree), filename=path, mode="exec"), mod.__dict__)
    finally:
        sys.path[:] = saved
        sys.modules.pop(name, None)
    return mod


def _seed(seed: int) -> None:
    torch.manual_seed(seed)
    if torch.cuda.is_available():
        torch.cuda.manual_seed_all(seed)


def _clone(v):
    if isinstance(v, torch.Tensor):
        return v.detach().clone()
    if isinstance(v, (list, tuple)):
        return type(v)(_clone(x) for x in v)
    return v


def _to(v, device):
    if isinstance(v, torch.Tensor):
        return v.to(device)
    if isinstance(v, (list, tuple)):
        return type(v)(_to(x, device) for x in v)
    return v


def run_case(v0_cls, v0_get_init_inputs, v0_get_inputs, v1_module, device, seed: int = 42):
    """Both models built and run as the harness does; returns (v0 output, v1 output, v0 model, v0 inputs)."""
    _seed(seed)
    v0_init = list(v0_get_init_inputs())
    _seed(seed)
    v1_init = list(v1_module.get_init_inputs())
    model = v0_cls(*v0_init).eval()
    model_new = v1_module.ModelNew(*v1_init).eval()
    _seed(seed)
    v0_inputs = list(v0_get_inputs())
    try:
        model_new.load_state_dict(model.state_dict())
    except Exception:  # the harness ignores a failed copy (auto_bench.py:518-521)
        pass
    model, model_new = model.to(device), model_new.to(device)
    v0_inputs = _to(v0_inputs, device)
    v1_inputs = _clone(v0_inputs)
    with torch.no_grad():
        _seed(seed)
        out0 = model.forward(*_clone(v0_inputs))
        _seed(seed)
        out1 = model_new.forward(*_clone(v1_inputs))
    return out0, out1, model, v0_inputs
