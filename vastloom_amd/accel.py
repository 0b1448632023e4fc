"""Python view of the Safety Governor, Governor-reserved buffers and the matvec accelerator with
device residency (include/vastloom_hip.h). Everything runs in libvastloom_hip.so.

Names follow the reference: ``Governor`` is ``safety::ResourceGovernor``
(src/safety/resource_governor.cpp), ``Accelerator`` is ``cuda::CudaMatvecAccelerator``
(src/cuda/cuda_matvec_accelerator.cpp) behind the ``DeepseekV4MatvecAccelerator`` seam
(include/vastloom/inference/deepseek_v4_reference.hpp:437-451), and ``PackedMatrix`` is
``DeepseekV4PackedMatrix`` (:104-141).
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import VL_DECLINED, VL_OK, VlError, call, check, lib

KIND_RAM, KIND_VRAM, KIND_STAGING, KIND_SCRATCH = (_lib.KIND_RAM, _lib.KIND_VRAM,
                                                   _lib.KIND_STAGING, _lib.KIND_SCRATCH)
STATE_NAMES = {0: "normal", 1: "pressure", 2: "critical", 3: "emergency"}


@dataclass(frozen=True)
class GpuInfo:
    """One visible GPU (``hardware::GpuInfo``, include/vastloom/hardware/hardware_probe.hpp:27-35),
    from the HIP runtime; temperature and power limit are not reported (None)."""
    backend: str
    name: str
    arch: str
    driver_version: str
    total_vram_bytes: int
    free_vram_bytes: int
    compute_units: int
    temperature_celsius: float | None = None
    power_limit_watts: float | None = None


def gpu_probe(device: int = 0) -> GpuInfo:
    """The GPU probe the runtime policy reads (src/hardware/hardware_probe.cpp:304-311 runs
    nvidia-smi there)."""
    info = _lib.GpuInfo()
    check(lib().vl_gpu_probe(device, C.byref(info)), "vl_gpu_probe")
    return GpuInfo(info.backend.decode(), info.name.decode(), info.arch.decode(),
                   info.driver_version.decode(), info.total_vram_bytes, info.free_vram_bytes,
                   info.compute_units)


def vram_hard_limit(total_vram_bytes: int, free_vram_bytes: int) -> int:
    """The runtime policy's VRAM hard limit of a probed GPU (src/safety/runtime_policy.cpp:137-141):
    min(80 % of total, free - 1 GiB) above 1 GiB free, else 0."""
    out = C.c_uint64()
    check(lib().vl_vram_hard_limit(total_vram_bytes, free_vram_bytes, C.byref(out)),
          "vl_vram_hard_limit")
    return out.value


def default_limits(**overrides) -> _lib.ResourceLimits:
    """ResourceLimits with the reference's defaults and every hard budget 0, then overrides."""
    limits = _lib.ResourceLimits()
    lib().vl_resource_limits_default(C.byref(limits))
    for k, v in overrides.items():
        setattr(limits, k, v)
    return limits


class Governor:
    """The native Safety Governor."""

    def __init__(self, limits: _lib.ResourceLimits | None = None, **overrides):
        limits = limits if limits is not None else default_limits(**overrides)
        handle = C.c_void_p()
        call("vl_governor_create", C.byref(limits), C.byref(handle))
        self._h = handle

    def try_reserve(self, kind: int, nbytes: int, tag: str = "python") -> int:
        """Reservation id; raises VlError when refused."""
        rid = C.c_uint64()
        call("vl_governor_try_reserve", self._h, kind, nbytes, tag.encode(), C.byref(rid))
        return rid.value

    def release(self, reservation: int) -> None:
        call("vl_governor_release", self._h, reservation)

    def abandon(self, reservation: int) -> None:
        call("vl_governor_abandon", self._h, reservation)

    def update_pressure(self, system_ram: int, gpu_vram: int, storage: int) -> str:
        p = _lib.RuntimePressure(system_ram, gpu_vram, storage)
        state = C.c_uint32()
        call("vl_governor_update_pressure", self._h, C.byref(p), C.byref(state))
        return STATE_NAMES[state.value]

    def snapshot(self) -> dict:
        s = _lib.GovernorSnapshot()
        call("vl_governor_snapshot_get", self._h, C.byref(s))
        return {"state": STATE_NAMES[s.state], "recovery_counter": s.recovery_counter,
                "reserved": list(s.reserved)}

    def ops(self) -> _lib.GovernorOps:
        return lib().vl_governor_as_ops(self._h)

    def close(self) -> None:
        if self._h:
            lib().vl_governor_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Buffer:
    """A Governor-reserved device (KIND_VRAM) or pinned host (KIND_STAGING) allocation."""

    def __init__(self, governor: Governor, kind: int, nbytes: int, *, device: int = 0,
                 min_free_after: int = 0, tag: str = "python-buffer"):
        self._ops = governor.ops()
        self._gov = governor  # keeps the Governor alive
        handle = C.c_void_p()
        call("vl_buffer_alloc", C.byref(self._ops), kind, device, nbytes, min_free_after,
             tag.encode(), C.byref(handle))
        self._h = handle

    @property
    def ptr(self) -> int:
        return lib().vl_buffer_ptr(self._h)

    @property
    def nbytes(self) -> int:
        return lib().vl_buffer_bytes(self._h)

    def free(self) -> None:
        if self._h:
            h, self._h = self._h, None
            call("vl_buffer_free", h)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


@dataclass
class PackedMatrix:
    """DeepseekV4PackedMatrix: host GGUF bytes with a cache identity."""
    ggml_type: int
    rows: int
    storage_columns: int
    encoded: np.ndarray
    cache_identity: int = 0
    recurring: bool = False
    logical_columns: int | None = None

    def c(self) -> _lib.PackedMatrix:
        enc = np.ascontiguousarray(self.encoded, dtype=np.uint8)
        self.encoded = enc  # the pointer below must stay valid
        return _lib.PackedMatrix(
            self.ggml_type, 1 if self.recurring else 0, self.rows,
            self.logical_columns if self.logical_columns is not None else self.storage_columns,
            self.storage_columns, enc.ctypes.data if enc.size else None, enc.size,
            self.cache_identity)


def default_options(**overrides) -> _lib.AccelOptions:
    o = _lib.AccelOptions()
    lib().vl_accel_options_default(C.byref(o))
    for k, v in overrides.items():
        setattr(o, k, v)
    return o


class Accelerator:
    """CudaMatvecAccelerator's contract on MI355X: residency by identity, decline = untouched."""

    def __init__(self, governor: Governor, options: _lib.AccelOptions | None = None,
                 backend: _lib.AccelBackend | None = None, **overrides):
        self._gov = governor
        self._ops = governor.ops()
        self._backend = backend  # keeps callbacks alive
        self.options = options if options is not None else default_options(**overrides)
        handle = C.c_void_p()
        call("vl_accel_create", C.byref(self.options), C.byref(self._ops),
             C.byref(backend) if backend is not None else None, C.byref(handle))
        self._h = handle

    def matvec(self, matrix: PackedMatrix, x: np.ndarray, y: np.ndarray) -> bool:
        """True when accelerated (y written); False when declined (y untouched)."""
        m = matrix.c()
        xv = np.ascontiguousarray(x, dtype=np.float32)
        if y.dtype != np.float32 or not y.flags.c_contiguous:
            raise ValueError("y must be a contiguous float32 array")
        rc = check(lib().vl_accel_matvec(self._h, C.byref(m), xv.ctypes.data, xv.size,
                                         y.ctypes.data, y.size), "vl_accel_matvec")
        return rc == VL_OK

    def prefetch(self, matrix: PackedMatrix) -> bool:
        m = matrix.c()
        return check(lib().vl_accel_prefetch(self._h, C.byref(m)), "vl_accel_prefetch") == VL_OK

    def holds(self, identity: int) -> bool:
        return bool(lib().vl_accel_holds(self._h, identity))

    def resident_matrix(self, identity: int) -> int:
        p = C.c_void_p()
        call("vl_accel_resident_matrix", self._h, identity, C.byref(p))
        return p.value

    def stats(self) -> dict:
        s = _lib.AccelStats()
        call("vl_accel_stats_get", self._h, C.byref(s))
        out = {f: getattr(s, f) for f, _ in _lib.AccelStats._fields_
               if f not in ("declined_type", "declined_by_type")}
        out["declined_by_type"] = {int(s.declined_type[i]): int(s.declined_by_type[i])
                                   for i in range(_lib.ACCEL_TYPE_SLOTS) if s.declined_by_type[i]}
        return out

    def close(self) -> None:
        if self._h:
            h, self._h = self._h, None
            call("vl_accel_destroy", h)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


__all__ = ["Governor", "Buffer", "PackedMatrix", "Accelerator", "default_limits",
           "default_options", "VlError", "VL_OK", "VL_DECLINED"]
