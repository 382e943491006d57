"""The CPU oracle (oracle/) is test infrastructure: the product never
imports, links or calls it, and bench.py touches it only in its CPU-baseline
leg (CPU: source and import checks, nothing runs on a GPU).
"""
import ast
import os
import subprocess
import sys

from conftest import PKG, ROOT


def test_package_sources_do_not_reference_the_oracle():
    hits = []
    for d, _, files in os.walk(PKG):
        if "/lib" in d or "__pycache__" in d:
            continue
        for f in files:
            if f.endswith((".py", ".cpp", ".h", ".hip")) or f == "Makefile":
                text = open(os.path.join(d, f), errors="replace").read()
                if "oracle" in text or "pyoracle" in text or "sdref" in text:
                    hits.append(os.path.relpath(os.path.join(d, f), ROOT))
    assert not hits, hits


def test_bench_uses_the_oracle_only_for_the_cpu_baseline():
    tree = ast.parse(open(os.path.join(ROOT, "bench.py")).read())
    users = set()
    for fn in ast.walk(tree):
        if isinstance(fn, ast.FunctionDef):
            for node in ast.walk(fn):
                if isinstance(node, (ast.Import, ast.ImportFrom)) and any(
                        "oracle" in (a.name or "") for a in node.names):
                    users.add(fn.name)
                if isinstance(node, ast.Name) and node.id == "pyoracle":
                    users.add(fn.name)
    top = [n for n in tree.body if isinstance(n, (ast.Import, ast.ImportFrom))
           and any("oracle" in a.name for a in n.names)]
    assert not top, "bench.py imports the oracle at module level"
    assert users == {"cpu_baseline"}, users


def test_importing_the_binding_loads_nothing_from_the_oracle():
    code = ("import sys; sys.path.insert(0, %r); import sdq; sdq.load_library(); "
            "import os; maps = open('/proc/self/maps').read(); "
            "print(any('oracle' in m for m in sys.modules), 'oracle' in maps)") % PKG
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr
    assert out.stdout.split() == ["False", "False"], out.stdout
