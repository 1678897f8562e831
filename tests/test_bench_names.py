"""bench.py, __graft_entry__.py and the package's Python files: every name a function reads is defined
somewhere (a local, an enclosing scope, the module or builtins).  Most of that code runs only on a GPU box,
so a misspelt or missing name would otherwise surface only there; this checks the symbol tables on the CPU."""
import builtins
import pathlib
import symtable

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _undefined(src: str, filename: str):
    top = symtable.symtable(src, filename, "exec")
    module = {s.get_name() for s in top.get_symbols() if s.is_assigned() or s.is_imported() or s.is_namespace()}
    known = module | set(dir(builtins)) | {"__file__", "__name__", "__doc__", "__spec__", "__package__"}
    bad = []

    def walk(table):
        for child in table.get_children():
            for sym in child.get_symbols():
                if sym.is_referenced() and sym.is_global() and sym.get_name() not in known:
                    bad.append("%s: %s" % (child.get_name(), sym.get_name()))
            walk(child)

    walk(top)
    return bad


def test_bench_functions_read_defined_names():
    assert _undefined((ROOT / "bench.py").read_text(), "bench.py") == []


def test_package_functions_read_defined_names():
    files = [ROOT / "__graft_entry__.py"] + sorted((ROOT / "leankv_amd").rglob("*.py"))
    bad = {str(f.relative_to(ROOT)): _undefined(f.read_text(), str(f)) for f in files}
    assert {k: v for k, v in bad.items() if v} == {}


def test_the_check_finds_an_undefined_name():
    src = "import os\ndef f(a):\n    b = a + os.sep\n    return b + missing_name\n"
    assert _undefined(src, "x.py") == ["f: missing_name"]
