"""The C-ABI library loads and exports every symbol include/larql_hip.h declares
(no compute calls: runs without a GPU)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "larql_hip.h")


def declared_symbols():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(larql_hip_\w+)\s*\(", src)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert len(syms) >= 15
    assert "larql_hip_q4k_matvec" in syms and "larql_hip_q4_matvec" in syms


def test_library_exports_every_declared_symbol():
    import larql_hip

    lib = ctypes.CDLL(larql_hip.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, f"not exported: {missing}"


def test_python_binding_covers_header():
    import larql_hip

    missing = [s for s in declared_symbols() if s not in larql_hip.SIGNATURES]
    assert not missing, f"no ctypes signature for: {missing}"


def test_binding_fails_loudly_without_library(tmp_path, monkeypatch):
    import larql_hip

    monkeypatch.setattr(larql_hip, "_lib", None)
    monkeypatch.setattr(larql_hip, "LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(ImportError):
        larql_hip.load_library()


def test_product_does_not_reference_oracle():
    """Nothing in the shipped package or its sources names the oracle."""
    pkg = os.path.join(ROOT, "encoding-experiment_amd")
    for dirpath, _, files in os.walk(pkg):
        if "_build" in dirpath:
            continue
        for fn in files:
            if fn.endswith((".py", ".hip", ".cpp", ".h", ".hpp")):
                text = open(os.path.join(dirpath, fn), errors="ignore").read()
                assert "import oracle" not in text and "larql_oracle" not in text and "liblarql_oracle" not in text, fn


def test_single_hip_runtime_in_process():
    """The binding must not put a second libamdhip64 next to torch's."""
    import subprocess
    import sys

    code = ("import sys; sys.path[:0] = [%r, %r]; import larql_hip, torch; "
            "maps = [l.split()[-1] for l in open('/proc/self/maps') if 'libamdhip64' in l and 'r-xp' in l]; "
            "print(len(set(maps)))") % (ROOT, os.path.join(ROOT, "encoding-experiment_amd"))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip() == "1", out.stdout
