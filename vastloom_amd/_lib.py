"""Loader for the in-tree HIP library (libvastloom_hip.so) and its C ABI.

There is no CPU fallback: if the library is missing or a device call fails, the error is raised.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libvastloom_hip.so"

VL_OK, VL_DECLINED = 0, 100
STATUS_NAMES = {
    1: "invalid_argument", 2: "invalid_format", 3: "not_found", 4: "permission_denied",
    5: "io_error", 6: "integrity_error", 7: "unsafe_path", 8: "unsupported",
    9: "resource_exhausted", 10: "internal_error", 100: "declined",
}
STATUS_NONFINITE_INPUT, STATUS_NONFINITE_OUTPUT, STATUS_BAD_ROUTE, STATUS_INTERNAL = 1, 2, 4, 8

_lib: C.CDLL | None = None


class VlError(RuntimeError):
    def __init__(self, code: int, what: str, message: str):
        super().__init__(f"{what}: {STATUS_NAMES.get(code, code)}: {message}")
        self.code = code
        self.name = STATUS_NAMES.get(code, str(code))


_U32, _U64, _I32, _P = C.c_uint32, C.c_uint64, C.c_int, C.c_void_p

# name -> argument types (all return int status unless listed in _RESTYPES)
class GpuInfo(C.Structure):
    """vl_gpu_info (GpuInfo, include/vastloom/hardware/hardware_probe.hpp:27-35)."""
    _fields_ = [("backend", C.c_char * 16), ("name", C.c_char * 128), ("arch", C.c_char * 64),
                ("driver_version", C.c_char * 32), ("total_vram_bytes", C.c_uint64),
                ("free_vram_bytes", C.c_uint64), ("compute_units", C.c_uint32),
                ("has_temperature", C.c_uint32), ("has_power_limit", C.c_uint32),
                ("reserved", C.c_uint32)]


_SIGNATURES = {
    "vl_last_error": [],
    "vl_device_count": [C.POINTER(C.c_int)],
    "vl_gpu_probe": [C.c_int, C.POINTER(GpuInfo)],
    "vl_vram_hard_limit": [C.c_uint64, C.c_uint64, C.POINTER(C.c_uint64)],
    "vl_matrix_layout": [_U32, _U64, _U64, C.POINTER(_U64), C.POINTER(_U64)],
    "vl_pack_matrix": [_U32, _U64, _U64, _P, _P, _P],
    "vl_dequantize": [_U32, _U64, _U64, _P, _P, _P],
    "vl_matvec_workspace": [_U32, _U64, _U64, _U32, C.POINTER(_U64)],
    "vl_matvec": [_U32, _U64, _U64, _P, _P, _U32, _P, _P, _U64, _P],
    "vl_read_status": [_P, _P, C.POINTER(_U32)],
    "vl_moe_workspace": [_P, C.POINTER(_U64)],
    "vl_moe_layer": [_P, _P, _P, _U64, _P],
    "vl_moe_route": [_P, _P, _P, _U64, _P],
    "vl_moe_layer_noalloc": [_P, _P, _P],
    "vl_moe_noalloc_status": [_P, _P],
    "vl_moe_read_routes": [_P, _P, _P, _P, _P],
    "vl_timeline_create": [_U32, C.POINTER(C.c_void_p)],
    "vl_timeline_destroy": [_P],
    "vl_moe_layer_profiled": [_P, _P, _P, _U64, _P, _P, _U32],
    "vl_timeline_stage_ms": [_P, _U32, C.POINTER(C.c_float)],
    "vl_timeline_kernel_ms": [_P, _U32, C.POINTER(C.c_float)],
    "vl_timeline_set_kernel_brackets": [_P, C.c_int],
    "vl_resource_limits_default": [_P],
    "vl_governor_create": [_P, C.POINTER(C.c_void_p)],
    "vl_governor_destroy": [_P],
    "vl_governor_try_reserve": [_P, _U32, _U64, C.c_char_p, C.POINTER(_U64)],
    "vl_governor_release": [_P, _U64],
    "vl_governor_abandon": [_P, _U64],
    "vl_governor_update_pressure": [_P, _P, C.POINTER(_U32)],
    "vl_governor_snapshot_get": [_P, _P],
    "vl_governor_as_ops": [_P],
    "vl_buffer_alloc": [_P, _U32, _I32, _U64, _U64, C.c_char_p, C.POINTER(C.c_void_p)],
    "vl_buffer_ptr": [_P],
    "vl_buffer_bytes": [_P],
    "vl_buffer_free": [_P],
    "vl_accel_options_default": [_P],
    "vl_accel_create": [_P, _P, _P, C.POINTER(C.c_void_p)],
    "vl_accel_destroy": [_P],
    "vl_accel_matvec": [_P, _P, _P, _U64, _P, _U64],
    "vl_accel_prefetch": [_P, _P],
    "vl_accel_holds": [_P, _U64],
    "vl_accel_resident_matrix": [_P, _U64, C.POINTER(C.c_void_p)],
    "vl_accel_stats_get": [_P, _P],
}
_RESTYPE_NONE = {"vl_timeline_destroy", "vl_resource_limits_default", "vl_governor_destroy",
                 "vl_accel_options_default"}

STAGES = ("router", "gate_up", "down")


class MoeConfig(C.Structure):
    """vl_moe_config (include/vastloom_hip.h)."""
    _fields_ = [(n, C.c_uint32) for n in (
        "tokens", "width", "intermediate", "experts", "top_k", "gate_type", "down_type",
        "semantics", "routing", "score_fn", "has_shared", "renormalize")] + [
        ("route_scale", C.c_float), ("routed_limit", C.c_float), ("shared_limit", C.c_float)]


class ExpertWeights(C.Structure):
    """vl_expert_weights: tiled device pointers of one expert."""
    _fields_ = [("gate", C.c_void_p), ("up", C.c_void_p), ("down", C.c_void_p)]


class MoeInputs(C.Structure):
    """vl_moe_inputs: device pointers of one layer call."""
    _fields_ = [("experts", C.c_void_p), ("router", C.c_void_p), ("bias", C.c_void_p),
                ("table_ids", C.c_void_p), ("given_ids", C.c_void_p),
                ("given_weights", C.c_void_p), ("x", C.c_void_p), ("out", C.c_void_p)]


SEM_DEEPSEEK, SEM_QWEN, SEM_PLAIN = 0, 1, 2
ROUTE_LEARNED, ROUTE_TABLE, ROUTE_SOFTMAX, ROUTE_GIVEN = 0, 1, 2, 3
SCORE_SQRT_SOFTPLUS, SCORE_SIGMOID = 0, 1
KIND_RAM, KIND_VRAM, KIND_STAGING, KIND_SCRATCH = 0, 1, 2, 3
STATE_NORMAL, STATE_PRESSURE, STATE_CRITICAL, STATE_EMERGENCY = 0, 1, 2, 3


class ResourceLimits(C.Structure):
    """vl_resource_limits (ResourceLimits of the reference's Safety Governor)."""
    _fields_ = [(n, C.c_uint64) for n in (
        "host_memory_hard_limit", "ram_hard_limit", "vram_hard_limit", "staging_hard_limit",
        "scratch_hard_limit", "minimum_system_ram_available", "minimum_storage_available")] + [
        ("pressure_ratio", C.c_double), ("critical_ratio", C.c_double),
        ("recovery_samples", C.c_uint32)]


class RuntimePressure(C.Structure):
    _fields_ = [("system_ram_available", C.c_uint64), ("gpu_vram_available", C.c_uint64),
                ("storage_available", C.c_uint64)]


class GovernorSnapshot(C.Structure):
    _fields_ = [("state", C.c_uint32), ("recovery_counter", C.c_uint32),
                ("reserved", C.c_uint64 * 4)]


RESERVE_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint32, C.c_uint64, C.c_char_p,
                         C.POINTER(C.c_uint64))
RELEASE_FN = C.CFUNCTYPE(None, C.c_void_p, C.c_uint64)


class GovernorOps(C.Structure):
    """vl_governor_ops: a Governor as the allocating entry points see it."""
    _fields_ = [("ctx", C.c_void_p), ("try_reserve", RESERVE_FN), ("release", RELEASE_FN),
                ("abandon", RELEASE_FN)]


class PackedMatrix(C.Structure):
    """vl_packed_matrix (DeepseekV4PackedMatrix)."""
    _fields_ = [("ggml_type", C.c_uint32), ("recurring", C.c_uint32), ("rows", C.c_uint64),
                ("logical_columns", C.c_uint64), ("storage_columns", C.c_uint64),
                ("encoded", C.c_void_p), ("encoded_bytes", C.c_uint64),
                ("cache_identity", C.c_uint64)]


class AccelOptions(C.Structure):
    """vl_accel_options (CudaMatvecAcceleratorOptions)."""
    _fields_ = [("device_ordinal", C.c_int), ("experts_only", C.c_uint32),
                ("minimum_free_vram_after", C.c_uint64), ("maximum_resident_bytes", C.c_uint64),
                ("maximum_matrices", C.c_uint64), ("staging_bytes", C.c_uint64)]


ACCEL_TYPE_SLOTS = 8


class AccelStats(C.Structure):
    """vl_accel_stats (CudaMatvecAcceleratorStats)."""
    _fields_ = [(n, C.c_uint64) for n in (
        "offered", "accelerated", "declined", "evicted", "declined_recurring",
        "resident_matrices", "resident_bytes", "uploaded_bytes")] + [
        ("declined_type", C.c_uint32 * ACCEL_TYPE_SLOTS),
        ("declined_by_type", C.c_uint64 * ACCEL_TYPE_SLOTS),
        ("kernel_ms", C.c_double), ("upload_ms", C.c_double)]


FREE_MEMORY_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.POINTER(C.c_uint64))
ALLOCATE_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint32, C.c_int, C.c_uint64,
                          C.POINTER(C.c_void_p))
BACKEND_RELEASE_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint32, C.c_void_p)
UPLOAD_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint32, C.c_uint64, C.c_uint64, C.c_void_p,
                        C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64)
IO_BYTES_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint32, C.c_uint64, C.c_uint64,
                          C.POINTER(C.c_uint64))
MATVEC_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint32, C.c_uint64, C.c_uint64, C.c_void_p,
                        C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64)


class AccelBackend(C.Structure):
    """vl_accel_backend: device operations of an accelerator (test seam)."""
    _fields_ = [("ctx", C.c_void_p), ("free_memory", FREE_MEMORY_FN), ("allocate", ALLOCATE_FN),
                ("release", BACKEND_RELEASE_FN), ("upload", UPLOAD_FN),
                ("io_bytes", IO_BYTES_FN), ("matvec", MATVEC_FN)]


_RESTYPES = {"vl_last_error": C.c_char_p, "vl_governor_as_ops": GovernorOps,
             "vl_buffer_ptr": C.c_void_p, "vl_buffer_bytes": C.c_uint64}


def lib() -> C.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m vastloom_amd.build` "
                "(there is no CPU fallback)")
        handle = C.CDLL(str(LIB_PATH))
        for name, args in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = None if name in _RESTYPE_NONE else _RESTYPES.get(name, C.c_int)
        _lib = handle
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def check(code: int, what: str) -> int:
    """Raise VlError for a failure; return the code (0 or VL_DECLINED) otherwise."""
    if code not in (VL_OK, VL_DECLINED):
        msg = lib().vl_last_error()
        raise VlError(code, what, msg.decode() if msg else "")
    return code


def call(name: str, *args) -> int:
    return check(getattr(lib(), name)(*args), name)
