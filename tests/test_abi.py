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


def _moe_config(routing):
    return _lib.MoeConfig(1, 256, 256, 8, 2, 16, 16, 0, routing, _lib.SCORE_SIGMOID, 0, 1,
                          1.0, 0.0, 0.0)


def test_layer_entries_refuse_missing_router_before_any_launch():
    """Both layer entry points run the same checks before touching a device: a routing that
    needs router weights (or table ids) without them is invalid_argument, not a kernel fault."""
    lib = _lib.lib()
    dummy = C.c_void_p(16)  # never dereferenced: the call must refuse first
    for routing in (_lib.ROUTE_LEARNED, _lib.ROUTE_SOFTMAX, _lib.ROUTE_TABLE):
        cfg = _moe_config(routing)
        inputs = _lib.MoeInputs(dummy.value, 0, 0, 0, 0, 0, dummy.value, dummy.value)
        assert lib.vl_moe_layer(C.byref(cfg), C.byref(inputs), dummy, 1 << 30, None) == 1
        assert b"router" in lib.vl_last_error()
        assert lib.vl_moe_layer_profiled(C.byref(cfg), C.byref(inputs), dummy, 1 << 30, None,
                                         None, 0) == 1
        assert b"router" in lib.vl_last_error()
    cfg = _moe_config(_lib.ROUTE_TABLE)
    inputs = _lib.MoeInputs(dummy.value, dummy.value, 0, 0, 0, 0, dummy.value, dummy.value)
    for fn in (lambda: lib.vl_moe_layer(C.byref(cfg), C.byref(inputs), dummy, 1 << 30, None),
               lambda: lib.vl_moe_layer_profiled(C.byref(cfg), C.byref(inputs), dummy, 1 << 30,
                                                 None, None, 0)):
        assert fn() == 1 and b"table" in lib.vl_last_error()


def test_status_bits_map_to_errors():
    from vastloom_amd.ops import status_error

    assert status_error(0, "x") is None
    cases = {_lib.STATUS_NONFINITE_INPUT: "invalid_argument",
             _lib.STATUS_NONFINITE_OUTPUT: "invalid_format",
             _lib.STATUS_BAD_ROUTE: "invalid_argument",
             _lib.STATUS_INTERNAL: "internal_error"}
    for bit, name in cases.items():
        err = status_error(bit, "layer")
        assert err is not None and err.name == name, (bit, err)
    # A timed-out wait outranks every other bit: the output is not valid at all.
    assert status_error(_lib.STATUS_INTERNAL | _lib.STATUS_BAD_ROUTE, "layer").name == "internal_error"


def test_route_scale_must_be_finite_and_positive():
    """Learned and table routes scale their weights by route_scale; the reference refuses a
    non-finite or non-positive one (route_from_indices, deepseek_v4_reference.cpp:80-90). Softmax
    and given routes do not use it."""
    lib = _lib.lib()
    n = C.c_uint64()
    for routing in (_lib.ROUTE_LEARNED, _lib.ROUTE_TABLE):
        for bad in (0.0, -1.0, float("inf"), float("nan")):
            cfg = _moe_config(routing)
            cfg.route_scale = bad
            assert lib.vl_moe_workspace(C.byref(cfg), C.byref(n)) == 1, (routing, bad)
    cfg = _moe_config(_lib.ROUTE_SOFTMAX)
    cfg.route_scale = 0.0
    rc = lib.vl_moe_workspace(C.byref(cfg), C.byref(n))
    assert rc != 1 or b"configuration" not in lib.vl_last_error()


def test_layer_storage_type_combinations():
    """The layer takes every storage type with a device layout on either side, except a
    GGUF-layout gate/up with a tiled down (the tiled down stage reads h magnitudes that only the
    tiled gate/up stage forms): that configuration is refused before any device is touched."""
    lib = _lib.lib()
    n = C.c_uint64()

    def refused(gate_type, down_type):
        cfg = _lib.MoeConfig(1, 1024, 512, 8, 2, gate_type, down_type, 0, _lib.ROUTE_GIVEN, 0, 0, 1,
                             1.0, 0.0, 0.0)
        rc = lib.vl_moe_workspace(C.byref(cfg), C.byref(n))
        return rc == 1 and b"invalid MoE configuration" in lib.vl_last_error()

    q4_k, q6_k, iq2_xxs, iq1_s, iq2_s, mxfp4, i32 = 12, 14, 16, 19, 22, 39, 26
    assert refused(q4_k, iq2_xxs)
    assert refused(i32, i32)
    for gate_type, down_type in ((q4_k, q6_k), (iq2_xxs, mxfp4), (iq2_s, q4_k), (iq1_s, q6_k)):
        assert not refused(gate_type, down_type)
