"""CPU checks of the driver entry points in ``__graft_entry__.py`` and
``bench.py``: every attribute they take from the package and the oracle
modules exists, and every named synthetic workload they time resolves.
(``smoke()`` itself needs a GPU; a renamed or removed function would
otherwise surface only on the GPU box.)"""

import ast
import importlib
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


_SCOPES = (ast.FunctionDef, ast.AsyncFunctionDef, ast.ClassDef)


def _scope_nodes(scope):
    """The nodes of one scope, without descending into nested functions or classes."""
    stack = list(ast.iter_child_nodes(scope))
    while stack:
        node = stack.pop()
        yield node
        if not isinstance(node, _SCOPES):
            stack.extend(ast.iter_child_nodes(node))


def _missing_attributes(scope, inherited):
    """``alias.attr`` uses whose alias is a package or oracle module imported in
    this scope or an enclosing one (and not rebound here) but which that
    module does not define."""
    aliases = dict(inherited)
    assigned = set()
    nested = []
    for node in _scope_nodes(scope):
        if isinstance(node, ast.ImportFrom) and node.module in ("akv_amd", "oracle"):
            for a in node.names:
                aliases[a.asname or a.name] = f"{node.module}.{a.name}"
        elif isinstance(node, ast.Name) and isinstance(node.ctx, ast.Store):
            assigned.add(node.id)
        elif isinstance(node, _SCOPES):
            nested.append(node)
    aliases = {k: v for k, v in aliases.items() if k not in assigned}
    missing = []
    for node in _scope_nodes(scope):
        if isinstance(node, ast.Attribute) and isinstance(node.value, ast.Name) and node.value.id in aliases:
            if not hasattr(importlib.import_module(aliases[node.value.id]), node.attr):
                missing.append(f"{node.value.id}.{node.attr} (line {node.lineno})")
    for inner in nested:
        missing += _missing_attributes(inner, aliases)
    return missing


@pytest.mark.parametrize("script", ["__graft_entry__.py", "bench.py"])
def test_referenced_attributes_exist(script):
    missing = _missing_attributes(ast.parse((ROOT / script).read_text()), {})
    assert not missing, f"{script} uses names its modules do not define: {missing}"


def test_bench_workloads_resolve():
    from akv_amd import synth

    tree = ast.parse((ROOT / "bench.py").read_text())
    names = set()
    for node in ast.walk(tree):
        # Pipeline("name", ...) and synth.workload("name")
        if isinstance(node, ast.Call) and node.args and isinstance(node.args[0], ast.Constant) \
                and isinstance(node.args[0].value, str):
            f = node.func
            if (isinstance(f, ast.Name) and f.id == "Pipeline") or \
                    (isinstance(f, ast.Attribute) and f.attr == "workload"):
                names.add(node.args[0].value)
    assert names
    for name in sorted(names):
        synth.workload(name)
