"""Static checks of the GPU-only entry scripts (bench.py, __graft_entry__.py).

Their GPU paths cannot run in a CPU container, so a name used in a branch that
only a GPU run reaches (one bench mode, one config) would surface only on the
box. Every name a function reads must resolve to one of its own scopes, an
enclosing function, the module's top level or the builtins.
"""
import builtins
import os
import symtable

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _module_names(top):
    names = set()
    for sym in top.get_symbols():
        if sym.is_assigned() or sym.is_imported() or sym.is_namespace():
            names.add(sym.get_name())
    return names


def _unresolved(table, module_names, enclosing=()):
    out = []
    for child in table.get_children():
        scope_names = set()
        for sym in child.get_symbols():
            if sym.is_local() or sym.is_parameter() or sym.is_imported() or sym.is_assigned():
                scope_names.add(sym.get_name())
        visible = set().union(*enclosing) if enclosing else set()
        for sym in child.get_symbols():
            name = sym.get_name()
            if not sym.is_referenced() or name in scope_names:
                continue
            if sym.is_free() and name in visible:
                continue
            if name in module_names or hasattr(builtins, name) or name in visible:
                continue
            out.append(f"{child.get_name()}:{child.get_lineno()} reads undefined name {name!r}")
        out += _unresolved(child, module_names, enclosing + (scope_names,))
    return out


@pytest.mark.parametrize("script", ["bench.py", "__graft_entry__.py"])
def test_every_name_resolves(script):
    path = os.path.join(ROOT, script)
    with open(path) as f:
        top = symtable.symtable(f.read(), path, "exec")
    problems = _unresolved(top, _module_names(top))
    assert not problems, "\n".join(problems)


def test_checker_catches_an_undefined_name():
    src = "import os\n\ndef f(a):\n    b = os.sep\n    def g():\n        return a + b\n    return patch_muon(g)\n"
    top = symtable.symtable(src, "<planted>", "exec")
    problems = _unresolved(top, _module_names(top))
    assert problems == ["f:3 reads undefined name 'patch_muon'"]
