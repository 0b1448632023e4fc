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
Q4_K, Q5_K, Q6_K, IQ2_S, BF16, MXFP4 = 12, 13, 14, 22, 30, 39
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
    if not arr.flags.writeable:  # e.g. a view of a read-only expert pack mapping
        arr = arr.copy()
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


class DeviceExpert:
    """Gate (w1), up (w3) and down (w2) of one expert, resident and tiled."""

    def __init__(self, gate_type: int, down_type: int, width: int, intermediate: int,
                 gate, up, down, stream=None):
        self.gate = DeviceMatrix(gate_type, intermediate, width, gate, stream)
        self.up = DeviceMatrix(gate_type, intermediate, width, up, stream)
        self.down = DeviceMatrix(down_type, width, intermediate, down, stream)

    def release_staging(self) -> None:
        for m in (self.gate, self.up, self.down):
            m.release_staging()

    def weights(self) -> _lib.ExpertWeights:
        return _lib.ExpertWeights(self.gate.ptr(), self.up.ptr(), self.down.ptr())


class MoeLayer:
    """One MoE layer on the device: router, routing, expert SwiGLU FFNs and combine.

    The device counterpart of moe_forward (deepseek semantics,
    src/inference/deepseek_v4_graph.cpp:1902-2274) and qwen38_moe_block (qwen semantics,
    src/inference/qwen3_8_flash_next_reference.cpp:1377-1421); one call per layer, no host
    synchronisation inside.
    """

    def __init__(self, experts: list[DeviceExpert], shared: DeviceExpert | None, *, width: int,
                 intermediate: int, top_k: int, gate_type: int, down_type: int,
                 semantics: int, routing: int, score_fn: int = _lib.SCORE_SIGMOID,
                 renormalize: bool = True, route_scale: float = 1.0, routed_limit: float = 0.0,
                 shared_limit: float = 0.0, router: torch.Tensor | None = None,
                 bias: torch.Tensor | None = None, device="cuda"):
        self.experts, self.shared = experts, shared
        self.width, self.intermediate, self.top_k = width, intermediate, top_k
        self.gate_type, self.down_type = gate_type, down_type
        self.semantics, self.routing, self.score_fn = semantics, routing, score_fn
        self.renormalize, self.route_scale = renormalize, route_scale
        self.routed_limit, self.shared_limit = routed_limit, shared_limit
        self.router = None if router is None else router.to(device, torch.float32).contiguous()
        self.bias = None if bias is None else bias.to(device, torch.float32).contiguous()
        table = [e.weights() for e in experts] + ([shared.weights()] if shared else [])
        raw = (_lib.ExpertWeights * len(table))(*table)
        host = torch.frombuffer(bytearray(raw), dtype=torch.uint8)
        self.expert_table = host.to(device)
        self._ws: dict[int, torch.Tensor] = {}

    def config(self, tokens: int) -> _lib.MoeConfig:
        return _lib.MoeConfig(tokens, self.width, self.intermediate, len(self.experts),
                              self.top_k, self.gate_type, self.down_type, self.semantics,
                              self.routing, self.score_fn, int(self.shared is not None),
                              int(self.renormalize), self.route_scale, self.routed_limit,
                              self.shared_limit)

    def workspace(self, tokens: int) -> torch.Tensor:
        if tokens not in self._ws:
            n = C.c_uint64()
            cfg = self.config(tokens)
            call("vl_moe_workspace", C.byref(cfg), C.byref(n))
            self._ws[tokens] = torch.empty(n.value, dtype=torch.uint8,
                                           device=self.expert_table.device)
        return self._ws[tokens]

    def forward(self, x: torch.Tensor, out: torch.Tensor | None = None, *,
                table_ids: torch.Tensor | None = None, given_ids: torch.Tensor | None = None,
                given_weights: torch.Tensor | None = None, stream=None,
                check: bool = True, timeline: "Timeline | None" = None,
                call_slot: int = 0) -> torch.Tensor:
        x2 = x.reshape(-1, self.width).contiguous()
        tokens = x2.shape[0]
        if out is None:
            out = torch.empty_like(x2)
        ws = self.workspace(tokens)
        cfg = self.config(tokens)
        p = lambda t: 0 if t is None else t.data_ptr()  # noqa: E731
        inputs = _lib.MoeInputs(self.expert_table.data_ptr(), p(self.router), p(self.bias),
                                p(table_ids), p(given_ids), p(given_weights), x2.data_ptr(),
                                out.data_ptr())
        s = _stream(stream)
        if timeline is None:
            call("vl_moe_layer", C.byref(cfg), C.byref(inputs), ws.data_ptr(), ws.numel(), s)
        else:
            call("vl_moe_layer_profiled", C.byref(cfg), C.byref(inputs), ws.data_ptr(),
                 ws.numel(), s, timeline.handle, call_slot)
        if check:
            raise_on_status(ws, s, "moe_layer")
        return out

    def route(self, x: torch.Tensor, *, table_ids: torch.Tensor | None = None,
              stream=None) -> tuple[np.ndarray, np.ndarray]:
        """Routes the tokens without running the experts (vl_moe_route) and returns the routes:
        expert ids and weights [tokens, top_k], synchronising the stream. Refused tokens raise."""
        x2 = x.reshape(-1, self.width).contiguous()
        tokens = x2.shape[0]
        ws = self.workspace(tokens)
        cfg = self.config(tokens)
        p = lambda t: 0 if t is None else t.data_ptr()  # noqa: E731
        inputs = _lib.MoeInputs(self.expert_table.data_ptr(), p(self.router), p(self.bias),
                                p(table_ids), 0, 0, x2.data_ptr(), 0)
        s = _stream(stream)
        call("vl_moe_route", C.byref(cfg), C.byref(inputs), ws.data_ptr(), ws.numel(), s)
        raise_on_status(ws, s, "moe_route")
        return self.routes(tokens, stream)

    def routes(self, tokens: int, stream=None) -> tuple[np.ndarray, np.ndarray]:
        ids = np.zeros((tokens, self.top_k), np.uint32)
        w = np.zeros((tokens, self.top_k), np.float32)
        cfg = self.config(tokens)
        call("vl_moe_read_routes", C.byref(cfg), self.workspace(tokens).data_ptr(),
             _stream(stream), ids.ctypes.data, w.ctypes.data)
        return ids, w


class Timeline:
    """HIP events around the stages of profiled layer calls (vl_timeline_*)."""

    def __init__(self, calls: int, kernel_brackets: bool = False):
        """kernel_brackets: record each stage's kernel execution (kernel_ms) instead of the
        marks between stages (stage_ms)."""
        h = C.c_void_p()
        call("vl_timeline_create", calls, C.byref(h))
        self.handle, self.calls = h, calls
        if kernel_brackets:
            call("vl_timeline_set_kernel_brackets", self.handle, 1)

    def stage_ms(self, slot: int) -> dict[str, float]:
        ms = (C.c_float * len(_lib.STAGES))()
        call("vl_timeline_stage_ms", self.handle, slot, ms)
        return dict(zip(_lib.STAGES, list(ms)))

    def kernel_ms(self, slot: int) -> dict[str, float]:
        """Each stage's kernel alone: events recorded by the launch around its execution."""
        ms = (C.c_float * len(_lib.STAGES))()
        call("vl_timeline_kernel_ms", self.handle, slot, ms)
        return dict(zip(_lib.STAGES, list(ms)))

    def close(self) -> None:
        if self.handle:
            lib().vl_timeline_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def expert_ffn(expert: DeviceExpert, x: torch.Tensor, *, semantics: int,
               route_weights: torch.Tensor | None = None, limit: float = 0.0,
               stream=None) -> torch.Tensor:
    """One expert's SwiGLU FFN for up to 8 tokens: execute_expert (deepseek,
    deepseek_v4_graph.cpp:1826-1894), qwen38_expert_mlp_q8 (qwen) or
    routed_expert_iq1_s_iq3_xxs_f32 (plain)."""
    layer = MoeLayer([expert], None, width=expert.gate.cols, intermediate=expert.gate.rows,
                     top_k=1, gate_type=expert.gate.qtype, down_type=expert.down.qtype,
                     semantics=semantics, routing=_lib.ROUTE_GIVEN, routed_limit=limit,
                     device=x.device)
    gw = None if route_weights is None else route_weights.to(x.device, torch.float32).reshape(-1, 1).contiguous()
    return layer.forward(x, given_weights=gw, stream=stream)


def read_status(workspace: torch.Tensor, stream: int) -> int:
    bits = C.c_uint32()
    call("vl_read_status", _ptr(workspace), stream, C.byref(bits))
    return bits.value


def status_error(bits: int, what: str) -> VlError | None:
    """The error a device status word stands for, or None. The reference refuses non-finite
    inputs (invalid_argument), non-finite results (invalid_format) and routes it cannot form
    (invalid_argument: an out-of-range expert, a non-finite logit or bias, weights that cannot be
    normalised); a bounded wait that timed out inside a kernel is an internal error."""
    if bits & _lib.STATUS_INTERNAL:
        return VlError(10, what, "a device-side wait timed out; the output is not valid")
    if bits & _lib.STATUS_NONFINITE_INPUT:
        return VlError(1, what, "input contains a non-finite value")
    if bits & _lib.STATUS_NONFINITE_OUTPUT:
        return VlError(2, what, "produced a non-finite result")
    if bits & _lib.STATUS_BAD_ROUTE:
        return VlError(1, what, "the routing cannot be formed (out-of-range expert, non-finite "
                                "logit or bias, or weights that cannot be normalised)")
    return None


def raise_on_status(workspace: torch.Tensor, stream: int, what: str) -> None:
    """Raises the error the kernels recorded in the workspace status word, if any."""
    err = status_error(read_status(workspace, stream), what)
    if err is not None:
        raise err


__all__ = ["DeviceMatrix", "device_count", "matrix_layout", "lib", "VlError", "QUANT_TYPES"]
