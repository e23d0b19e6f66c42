"""Every global name a function of bench.py or the package reads is defined (no GPU needed).

bench.py's extras only run on a GPU box; a name missing from one of their
functions would surface there as a NameError at the end of the benchmark.
"""

import builtins
import symtable
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
FILES = [ROOT / "bench.py", ROOT / "__graft_entry__.py", *sorted((ROOT / "pollux_amd").glob("*.py"))]


@pytest.mark.parametrize("path", FILES, ids=lambda p: p.name)
def test_no_undefined_globals(path):
    top = symtable.symtable(path.read_text(), str(path), "exec")
    defined = {s.get_name() for s in top.get_symbols() if s.is_assigned() or s.is_imported()}
    defined |= set(dir(builtins)) | {"__file__"}
    missing = []

    def walk(t):
        for s in t.get_symbols():
            if s.is_global() and s.is_referenced() and s.get_name() not in defined:
                missing.append(f"{t.get_name()}: {s.get_name()}")
        for c in t.get_children():
            walk(c)

    walk(top)
    assert not missing, missing
