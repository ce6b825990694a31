"""Lint for the test files themselves: a module-level name bound twice in one
test module silently replaces the first binding, so every test that reads it
at run time sees the second value (a shape list once shadowed that way turned
a whole test into a check of other cases).  Fails on any such rebinding of
a constant or function."""
import ast
import glob
import os

import pytest

ROOT = os.path.dirname(os.path.abspath(__file__))


def _module_level_bindings(tree):
    names = []
    for node in tree.body:
        if isinstance(node, (ast.FunctionDef, ast.AsyncFunctionDef, ast.ClassDef)):
            names.append((node.name, node.lineno))
        elif isinstance(node, ast.Assign):
            for t in node.targets:
                if isinstance(t, ast.Name):
                    names.append((t.id, node.lineno))
        elif isinstance(node, ast.AnnAssign) and isinstance(node.target, ast.Name):
            names.append((node.target.id, node.lineno))
    return names


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(ROOT, "*.py"))),
                         ids=os.path.basename)
def test_no_duplicate_module_level_names(path):
    with open(path) as f:
        tree = ast.parse(f.read(), filename=path)
    seen = {}
    dups = []
    for name, line in _module_level_bindings(tree):
        if name in seen and name not in ("__all__",):
            dups.append(f"{name} (lines {seen[name]} and {line})")
        seen.setdefault(name, line)
    assert not dups, f"{os.path.basename(path)} rebinds: " + ", ".join(dups)
