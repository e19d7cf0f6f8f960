"""Static checks of bench.py that need no GPU: it compiles, and no function assigns a local that shadows a
module-level constant (such a local makes every earlier use in the function an UnboundLocalError, which the
bench reports only as `configs_error` on the GPU box)."""
import os
import symtable

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _functions(table):
    for child in table.get_children():
        if child.get_type() == "function":
            yield child
        yield from _functions(child)


def test_bench_locals_do_not_shadow_module_constants():
    path = os.path.join(ROOT, "bench.py")
    with open(path) as f:
        src = f.read()
    top = symtable.symtable(src, path, "exec")
    constants = {s.get_name() for s in top.get_symbols() if s.is_assigned() and s.get_name().isupper()}
    bad = []
    for fn in _functions(top):
        for s in fn.get_symbols():
            if s.is_local() and s.is_assigned() and s.get_name() in constants:
                bad.append(f"{fn.get_name()}: {s.get_name()}")
    assert not bad, bad
