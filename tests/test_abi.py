"""The C-ABI library loads and exports every entry point include/vastloom_hip.h declares (no
device call is made, so this runs without a GPU)."""

from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

from vastloom_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "vastloom_hip.h"


def declared_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = set()
    for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b(vl_\w+)\s*\(", text, flags=re.M):
        if not re.match(r"\s*typedef", text[m.start():m.end()]):
            names.add(m.group(1))
    return names


def test_header_declares_the_boundary():
    names = declared_functions()
    for core in ("vl_matvec", "vl_moe_layer", "vl_governor_try_reserve", "vl_buffer_alloc",
                 "vl_accel_matvec", "vl_last_error"):
        assert core in names


def test_library_exports_every_declared_symbol():
    handle = C.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in sorted(declared_functions()) if not hasattr(handle, n)]
    assert not missing, f"not exported: {missing}"


def test_python_binding_covers_every_declared_symbol():
    assert declared_functions() <= set(_lib.exported_symbols())
