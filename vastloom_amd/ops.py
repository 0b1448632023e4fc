"""Python view of the device operators, over the C ABI (include/vastloom_hip.h).

torch supplies device memory and the stream; every computation runs in libvastloom_hip.so.
Names follow the reference's operator API: a resident ``DeviceMatrix`` is the device side of a
``DeepseekV4PackedMatrix`` (include/vastloom/inference/deepseek_v4_reference.hpp:104-141),
``matvec`` is the device counterpart of ``matvec_<type>_f32`` (ggml_quantization.hpp:119-215),
``dequantize`` of ``dequantize_<type>``.
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _lib
from ._lib import VlError, call, lib

F32, Q8_0, IQ2_XXS, IQ3_XXS, IQ1_S = 0, 8, 16, 18, 19
QUANT_TYPES = (Q8_0, IQ2_XXS, IQ3_XXS, IQ1_S)


def _stream(stream: torch.cuda.Stream | None = None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def device_count() -> int:
    n = C.c_int()
    call("vl_device_count", C.byref(n))
    return n.value


def matrix_layout(qtype: int, rows: int, cols: int) -> tuple[int, int]:
    g, d = C.c_uint64(), C.c_uint64()
    call("vl_matrix_layout", qtype, rows, cols, C.byref(g), C.byref(d))
    return g.value, d.value


def to_device_bytes(data, device="cuda") -> torch.Tensor:
    if isinstance(data, torch.Tensor):
        return data.to(device=device, dtype=torch.uint8).contiguous()
    arr = np.ascontiguousarray(data, dtype=np.uint8)
    return torch.from_numpy(arr).to(device)


class DeviceMatrix:
    """A quantized matrix resident in HBM in its tiled form."""

    def __init__(self, qtype: int, rows: int, cols: int, gguf, stream=None,
                 tiled: torch.Tensor | None = None):
        self.qtype, self.rows, self.cols = qtype, rows, cols
        self.gguf_bytes, self.device_bytes = matrix_layout(qtype, rows, cols)
        src = to_device_bytes(gguf)
        if src.numel() != self.gguf_bytes:
            raise VlError(2, "DeviceMatrix", f"{src.numel()} bytes given, {self.gguf_bytes} expected")
        if tiled is None:
            tiled = torch.empty(self.device_bytes, dtype=torch.uint8, device=src.device)
        elif tiled.numel() < self.device_bytes:
            raise VlError(1, "DeviceMatrix", "tiled buffer too small")
        self.tiled = tiled
        call("vl_pack_matrix", qtype, rows, cols, _ptr(src), _ptr(tiled), _stream(stream))
        self._staging = src  # kept until the pack has run on the stream

    def release_staging(self) -> None:
        self._staging = None

    def ptr(self) -> int:
        return _ptr(self.tiled)

    def dequantize(self, stream=None) -> torch.Tensor:
        out = torch.empty((self.rows, self.cols), dtype=torch.float32, device=self.tiled.device)
        call("vl_dequantize", self.qtype, self.rows, self.cols, self.ptr(), _ptr(out),
             _stream(stream))
        return out

    def matvec(self, x: torch.Tensor, stream=None, check: bool = True) -> torch.Tensor:
        """x: [tokens, cols] (or [cols]) float32 on the device; returns [tokens, rows]."""
        squeeze = x.dim() == 1
        x2 = x.reshape(-1, self.cols).contiguous()
        tokens = x2.shape[0]
        ws_bytes = C.c_uint64()
        call("vl_matvec_workspace", self.qtype, self.rows, self.cols, tokens, C.byref(ws_bytes))
        ws = torch.empty(ws_bytes.value, dtype=torch.uint8, device=x.device)
        y = torch.empty((tokens, self.rows), dtype=torch.float32, device=x.device)
        s = _stream(stream)
        call("vl_matvec", self.qtype, self.rows, self.cols, self.ptr(), _ptr(x2), tokens,
             _ptr(y), _ptr(ws), ws_bytes.value, s)
        if check:
            raise_on_status(ws, s, "matvec")
        return y[0] if squeeze else y


def read_status(workspace: torch.Tensor, stream: int) -> int:
    bits = C.c_uint32()
    call("vl_read_status", _ptr(workspace), stream, C.byref(bits))
    return bits.value


def raise_on_status(workspace: torch.Tensor, stream: int, what: str) -> None:
    """The reference refuses non-finite inputs (invalid_argument) and non-finite results
    (invalid_format); the kernels record both in the workspace status word."""
    bits = read_status(workspace, stream)
    if bits & _lib.STATUS_NONFINITE_INPUT:
        raise VlError(1, what, "input contains a non-finite value")
    if bits & _lib.STATUS_NONFINITE_OUTPUT:
        raise VlError(2, what, "produced a non-finite result")
    if bits & _lib.STATUS_BAD_ROUTE:
        raise VlError(2, what, "router selected an out-of-range expert")


__all__ = ["DeviceMatrix", "device_count", "matrix_layout", "lib", "VlError", "QUANT_TYPES"]
