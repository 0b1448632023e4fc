"""ctypes bindings for the CPU oracle. TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py`` import this
module, as the checker. ``Oracle`` wraps ``_build/liboracle.so`` (the C restatement in
``vl_oracle.c``); ``Reference`` wraps ``_ref/libvlref.so`` (the reference's own CPU kernels, built
from its sources by ``make -C oracle ref`` where the reference tree is present).
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "_build" / "liboracle.so"
REF_SO = HERE / "_ref" / "libvlref.so"

F32, Q8_0, IQ2_XXS, IQ3_XXS, IQ1_S = 0, 8, 16, 18, 19
Q4_K, Q5_K, Q6_K, IQ2_S, BF16, MXFP4 = 12, 13, 14, 22, 30, 39
SCORE_SQRT_SOFTPLUS, SCORE_SIGMOID = 0, 1
DEFAULT_MAX_ELEMENTS = 64_000_000

ERROR_NAMES = {
    1: "invalid_argument", 2: "invalid_format", 3: "not_found", 4: "permission_denied",
    5: "io_error", 6: "integrity_error", 7: "unsafe_path", 8: "unsupported",
    9: "resource_exhausted", 10: "internal_error",
}


class OracleError(RuntimeError):
    def __init__(self, code: int, what: str):
        super().__init__(f"{what}: {ERROR_NAMES.get(code, code)}")
        self.code = code
        self.name = ERROR_NAMES.get(code, str(code))


def build() -> None:
    """Compile the C restatement (and the reference build when its tree is present)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)


def build_binding() -> None:
    """Compile the reference-side binding's test driver (oracle/_ref/accel_binding) against the
    built HIP library, when the reference tree is present."""
    subprocess.run(["make", "-s", "-C", str(HERE), "binding"], check=True)


def _ptr(a: np.ndarray | None, ctype=C.c_void_p):
    if a is None:
        return None
    return a.ctypes.data_as(ctype)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint8)


class _Matrix(C.Structure):
    _fields_ = [("type", C.c_uint32), ("data", C.c_void_p), ("bytes", C.c_size_t)]


def _matrices(items):
    """items: iterable of (type, uint8 array). Keeps the arrays alive with the struct array."""
    items = list(items)
    arr = (_Matrix * len(items))()
    keep = []
    for i, (t, data) in enumerate(items):
        data = _u8(data)
        keep.append(data)
        arr[i] = _Matrix(t, data.ctypes.data, data.nbytes)
    return arr, keep


class Oracle:
    """The C restatement of the reference path (vl_oracle.c)."""

    def __init__(self, path: Path = ORACLE_SO):
        if not path.exists():
            raise FileNotFoundError(f"{path} is not built; run `make -C oracle`")
        self.lib = C.CDLL(str(path))
        L = self.lib
        L.vlo_fp16_to_f32.restype = C.c_float
        L.vlo_fp16_to_f32.argtypes = [C.c_uint16]
        for name in ("vlo_sqrt_softplus", "vlo_sigmoid", "vlo_silu_f"):
            getattr(L, name).restype = C.c_float
            getattr(L, name).argtypes = [C.c_float]

    def _check(self, code: int, what: str) -> None:
        if code != 0:
            raise OracleError(code, what)

    # ---- decoders and matvecs ---------------------------------------------------------
    def codebooks_ok(self) -> bool:
        return bool(self.lib.vlo_codebooks_ok())

    def fp16_to_f32(self, bits: int) -> float:
        return self.lib.vlo_fp16_to_f32(bits)

    def storage_bytes(self, qtype: int, rows: int, cols: int,
                      max_elements: int = DEFAULT_MAX_ELEMENTS) -> int:
        out = C.c_size_t()
        self._check(self.lib.vlo_storage_bytes(qtype, C.c_size_t(rows), C.c_size_t(cols),
                                               C.c_size_t(max_elements), C.byref(out)),
                    "storage_bytes")
        return out.value

    def dequantize(self, qtype: int, encoded, elements: int,
                   max_elements: int = DEFAULT_MAX_ELEMENTS, out: np.ndarray | None = None):
        enc = _u8(encoded)
        if out is None:
            out = np.zeros(elements, np.float32)
        self._check(self.lib.vlo_dequantize(qtype, _ptr(enc), C.c_size_t(enc.nbytes), _ptr(out),
                                            C.c_size_t(elements), C.c_size_t(max_elements)),
                    "dequantize")
        return out

    def dequantize_row(self, qtype: int, encoded, rows: int, cols: int, row: int):
        enc = _u8(encoded)
        out = np.zeros(cols, np.float32)
        self._check(self.lib.vlo_dequantize_row(qtype, _ptr(enc), C.c_size_t(enc.nbytes),
                                                C.c_size_t(rows), C.c_size_t(cols),
                                                C.c_size_t(row), _ptr(out), C.c_size_t(cols)),
                    "dequantize_row")
        return out

    def matvec(self, qtype: int, encoded, rows: int, cols: int, x, threads: int = 1,
               max_elements: int = DEFAULT_MAX_ELEMENTS, out: np.ndarray | None = None):
        enc, xs = _u8(encoded), _f32(x)
        if out is None:
            out = np.zeros(rows, np.float32)
        self._check(self.lib.vlo_matvec(qtype, _ptr(enc), C.c_size_t(enc.nbytes),
                                        C.c_size_t(rows), C.c_size_t(cols), _ptr(xs),
                                        C.c_size_t(xs.size), _ptr(out), C.c_size_t(out.size),
                                        C.c_size_t(max_elements), C.c_uint(threads)),
                    "matvec")
        return out

    # ---- experts ------------------------------------------------------------------------
    def routed_expert_iq1s_iq3xxs(self, gate, up, down, width: int, expert_width: int, x):
        mats, keep = _matrices([(IQ1_S, gate), (IQ1_S, up), (IQ3_XXS, down)])
        xs = _f32(x)
        y = np.zeros(width, np.float32)
        self._check(self.lib.vlo_routed_expert_iq1s_iq3xxs(
            C.byref(mats[0]), C.byref(mats[1]), C.byref(mats[2]), C.c_size_t(width),
            C.c_size_t(expert_width), _ptr(xs), _ptr(y)), "routed_expert")
        return y

    def expert_deepseek(self, w1, w3, w2, width: int, intermediate: int, x, routing=None,
                        limit: float = 0.0, threads: int = 1):
        """w1/w3/w2: (type, bytes). x: [tokens, width]. routing: [tokens] or None."""
        mats, keep = _matrices([w1, w3, w2])
        xs = _f32(x).reshape(-1)
        tokens = xs.size // width
        r = None if routing is None else _f32(routing)
        y = np.zeros(tokens * width, np.float32)
        self._check(self.lib.vlo_expert_deepseek(
            C.byref(mats[0]), C.byref(mats[1]), C.byref(mats[2]), C.c_size_t(width),
            C.c_size_t(intermediate), _ptr(xs), C.c_size_t(tokens), _ptr(r), C.c_float(limit),
            _ptr(y), C.c_uint(threads)), "expert_deepseek")
        return y.reshape(tokens, width)

    def expert_qwen(self, gate, up, down, width: int, intermediate: int, x, threads: int = 1):
        mats, keep = _matrices([gate, up, down])
        xs = _f32(x)
        y = np.zeros(width, np.float32)
        self._check(self.lib.vlo_expert_qwen(
            C.byref(mats[0]), C.byref(mats[1]), C.byref(mats[2]), C.c_size_t(width),
            C.c_size_t(intermediate), _ptr(xs), _ptr(y), C.c_uint(threads)), "expert_qwen")
        return y

    # ---- routing ------------------------------------------------------------------------
    def sqrt_softplus(self, v: float) -> float:
        return self.lib.vlo_sqrt_softplus(v)

    def sigmoid(self, v: float) -> float:
        return self.lib.vlo_sigmoid(v)

    def silu_f(self, v: float) -> float:
        return self.lib.vlo_silu_f(v)

    def linear_f64(self, weight, x, out_width: int):
        w, xs = _f32(weight), _f32(x)
        in_width = w.size // out_width
        tokens = xs.size // in_width
        out = np.zeros(tokens * out_width, np.float32)
        self._check(self.lib.vlo_linear_f64(_ptr(w), _ptr(xs), C.c_size_t(tokens),
                                            C.c_size_t(in_width), C.c_size_t(out_width),
                                            _ptr(out)), "linear_f64")
        return out.reshape(tokens, out_width)

    def route_learned(self, logits, bias, top_k: int, route_scale: float = 1.0,
                      score_fn: int = SCORE_SQRT_SOFTPLUS):
        lg = _f32(logits)
        tokens, experts = lg.shape
        b = None if bias is None else _f32(bias)
        idx = np.zeros(tokens * top_k, np.uint32)
        w = np.zeros(tokens * top_k, np.float32)
        self._check(self.lib.vlo_route_learned(_ptr(lg), _ptr(b), C.c_size_t(tokens),
                                               C.c_size_t(experts), C.c_size_t(top_k),
                                               C.c_float(route_scale), C.c_int(score_fn),
                                               _ptr(idx), _ptr(w)), "route_learned")
        return idx.reshape(tokens, top_k), w.reshape(tokens, top_k)

    def route_hash(self, logits, token_ids, table, top_k: int, route_scale: float = 1.0,
                   score_fn: int = SCORE_SQRT_SOFTPLUS):
        lg = _f32(logits)
        tokens, experts = lg.shape
        tid = np.ascontiguousarray(token_ids, np.uint32)
        tab = np.ascontiguousarray(table, np.uint32)
        vocabulary = tab.size // top_k
        idx = np.zeros(tokens * top_k, np.uint32)
        w = np.zeros(tokens * top_k, np.float32)
        self._check(self.lib.vlo_route_hash(_ptr(lg), _ptr(tid), _ptr(tab), C.c_size_t(tokens),
                                            C.c_size_t(vocabulary), C.c_size_t(experts),
                                            C.c_size_t(top_k), C.c_float(route_scale),
                                            C.c_int(score_fn), _ptr(idx), _ptr(w)),
                    "route_hash")
        return idx.reshape(tokens, top_k), w.reshape(tokens, top_k)

    def route_softmax(self, logits, top_k: int, renormalize: bool = True):
        lg = _f32(logits)
        idx = np.zeros(top_k, np.uint32)
        w = np.zeros(top_k, np.float32)
        self._check(self.lib.vlo_route_softmax(_ptr(lg), C.c_size_t(lg.size), C.c_size_t(top_k),
                                               C.c_int(int(renormalize)), _ptr(idx), _ptr(w)),
                    "route_softmax")
        return idx, w

    # ---- layers -------------------------------------------------------------------------
    def moe_deepseek(self, x, indices, weights, experts, shared, width: int, intermediate: int,
                     routed_limit: float = 0.0, shared_limit: float = 0.0, threads: int = 1):
        """experts: list of (w1, w3, w2), each (type, bytes); shared: same triple or None."""
        xs = _f32(x).reshape(-1)
        tokens = xs.size // width
        idx = np.ascontiguousarray(indices, np.uint32).reshape(-1)
        w = _f32(weights).reshape(-1)
        top_k = idx.size // tokens
        mats, keep = _matrices([m for e in experts for m in e])
        sh = None
        if shared is not None:
            sh, keep2 = _matrices(shared)
            keep.append(keep2)
        out = np.zeros(tokens * width, np.float32)
        self._check(self.lib.vlo_moe_deepseek(
            _ptr(xs), C.c_size_t(tokens), C.c_size_t(width), C.c_size_t(intermediate),
            C.c_size_t(len(experts)), C.c_size_t(top_k), _ptr(idx), _ptr(w), mats,
            sh, C.c_float(routed_limit), C.c_float(shared_limit), _ptr(out),
            C.c_uint(threads)), "moe_deepseek")
        return out.reshape(tokens, width)

    def moe_qwen(self, x, indices, weights, experts, shared, width: int, intermediate: int,
                 threads: int = 1):
        xs = _f32(x)
        idx = np.ascontiguousarray(indices, np.uint32).reshape(-1)
        w = _f32(weights).reshape(-1)
        mats, keep = _matrices([m for e in experts for m in e])
        sh = None
        if shared is not None:
            sh, keep2 = _matrices(shared)
            keep.append(keep2)
        out = np.zeros(width, np.float32)
        self._check(self.lib.vlo_moe_qwen(
            _ptr(xs), C.c_size_t(width), C.c_size_t(intermediate), C.c_size_t(len(experts)),
            C.c_size_t(idx.size), _ptr(idx), _ptr(w), mats, sh, _ptr(out), C.c_uint(threads)),
            "moe_qwen")
        return out


class Reference:
    """The reference's own CPU kernels, compiled from its sources (oracle/_ref)."""

    def __init__(self, path: Path = REF_SO):
        if not path.exists():
            raise FileNotFoundError(f"{path} is not built; run `make -C oracle ref`")
        self.lib = C.CDLL(str(path))

    @staticmethod
    def available() -> bool:
        return REF_SO.exists()

    def _check(self, code: int, what: str) -> None:
        if code != 0:
            raise OracleError(code, what)

    def dequantize(self, qtype: int, encoded, elements: int,
                   max_elements: int = DEFAULT_MAX_ELEMENTS):
        enc = _u8(encoded)
        out = np.zeros(elements, np.float32)
        self._check(self.lib.vlr_dequantize(C.c_uint32(qtype), _ptr(enc), C.c_size_t(enc.nbytes),
                                            _ptr(out), C.c_size_t(elements),
                                            C.c_size_t(max_elements)), "ref dequantize")
        return out

    def matvec(self, qtype: int, encoded, rows: int, cols: int, x, threads: int = 1,
               max_elements: int = DEFAULT_MAX_ELEMENTS):
        enc, xs = _u8(encoded), _f32(x)
        out = np.zeros(rows, np.float32)
        self._check(self.lib.vlr_matvec(C.c_uint32(qtype), _ptr(enc), C.c_size_t(enc.nbytes),
                                        C.c_size_t(rows), C.c_size_t(cols), _ptr(xs), _ptr(out),
                                        C.c_size_t(max_elements), C.c_uint(threads)),
                    "ref matvec")
        return out

    def routed_expert_iq1s_iq3xxs(self, gate, up, down, width: int, expert_width: int, x):
        g, u, d, xs = _u8(gate), _u8(up), _u8(down), _f32(x)
        y = np.zeros(width, np.float32)
        self._check(self.lib.vlr_routed_expert_iq1s_iq3xxs(
            _ptr(g), _ptr(u), _ptr(d), C.c_size_t(width), C.c_size_t(expert_width), _ptr(xs),
            _ptr(y)), "ref routed_expert")
        return y

    def route_learned(self, logits, bias, top_k: int, route_scale: float = 1.0):
        lg, b = _f32(logits), _f32(bias)
        tokens, experts = lg.shape
        idx = np.zeros(tokens * top_k, np.uint32)
        w = np.zeros(tokens * top_k, np.float32)
        self._check(self.lib.vlr_route_learned(_ptr(lg), _ptr(b), C.c_size_t(tokens),
                                               C.c_size_t(experts), C.c_size_t(top_k),
                                               C.c_float(route_scale), _ptr(idx), _ptr(w)),
                    "ref route_learned")
        return idx.reshape(tokens, top_k), w.reshape(tokens, top_k)

    def route_hash(self, logits, token_ids, table, top_k: int, route_scale: float = 1.0):
        lg = _f32(logits)
        tokens, experts = lg.shape
        tid = np.ascontiguousarray(token_ids, np.uint32)
        tab = np.ascontiguousarray(table, np.uint32)
        idx = np.zeros(tokens * top_k, np.uint32)
        w = np.zeros(tokens * top_k, np.float32)
        self._check(self.lib.vlr_route_hash(_ptr(lg), _ptr(tid), _ptr(tab), C.c_size_t(tokens),
                                            C.c_size_t(tab.size // top_k), C.c_size_t(experts),
                                            C.c_size_t(top_k), C.c_float(route_scale),
                                            _ptr(idx), _ptr(w)), "ref route_hash")
        return idx.reshape(tokens, top_k), w.reshape(tokens, top_k)

    def expert_swiglu_f32(self, x, gate_w, down_w, up_w, routing, width: int, intermediate: int,
                          limit: float):
        xs = _f32(x).reshape(-1)
        tokens = xs.size // width
        g, d, u = _f32(gate_w), _f32(down_w), _f32(up_w)
        r = None if routing is None else _f32(routing)
        y = np.zeros(tokens * width, np.float32)
        self._check(self.lib.vlr_expert_swiglu_f32(_ptr(xs), _ptr(g), _ptr(d), _ptr(u), _ptr(r),
                                                   C.c_size_t(tokens), C.c_size_t(width),
                                                   C.c_size_t(intermediate), C.c_float(limit),
                                                   _ptr(y)), "ref expert_swiglu")
        return y.reshape(tokens, width)

    def qwen_route(self, hidden, router, experts: int, top_k: int, renormalize: bool = True):
        h, r = _f32(hidden), _f32(router)
        idx = np.zeros(top_k, np.uint32)
        w = np.zeros(top_k, np.float32)
        logits = np.zeros(experts, np.float32)
        self._check(self.lib.vlr_qwen_route(_ptr(h), _ptr(r), C.c_size_t(h.size),
                                            C.c_uint32(experts), C.c_uint32(top_k),
                                            C.c_int(int(renormalize)), _ptr(idx), _ptr(w),
                                            _ptr(logits)), "ref qwen_route")
        return idx, w, logits

    def qwen_expert_mlp_q8(self, gate, up, down, width: int, intermediate: int, x):
        g, u, d, xs = _u8(gate), _u8(up), _u8(down), _f32(x)
        y = np.zeros(width, np.float32)
        self._check(self.lib.vlr_qwen_expert_mlp_q8(_ptr(g), _ptr(u), _ptr(d),
                                                    C.c_uint32(width), C.c_uint32(intermediate),
                                                    _ptr(xs), _ptr(y)), "ref qwen_expert_mlp_q8")
        return y


def default_threads() -> int:
    """The reference's runtime policy: clamp(logical / 2, 1, 12) (src/safety/runtime_policy.cpp:145)."""
    logical = os.cpu_count() or 1
    return max(1, min(logical // 2, 12))
