"""The C-ABI library loads and exports every function the headers in include/ declare (CPU
only: nothing is computed)."""
import ctypes
import os
import re

import ggml_mi355x as mx

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    for h in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not h.endswith(".h"):
            continue
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("#"))
        for m in re.finditer(r"MI355X_API\s+[^;{(]*?\b(\w+)\s*\(", text):
            names.append(m.group(1))
    return names


def test_headers_declare_entry_points():
    names = declared_functions()
    assert len(names) >= 30, names
    assert "mi355x_gemm" in names and "ggml_backend_mi355x_graph_compute" in names


def test_library_exports_every_declared_symbol():
    L = mx.lib()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, missing


def test_library_path_is_in_tree():
    assert os.path.dirname(os.path.abspath(mx.LIB_PATH)).startswith(ROOT)
    assert isinstance(mx.lib(), ctypes.CDLL)
