"""A MoE layer over experts that live in host memory and become device-resident on demand.

The reference's layer loop routes a layer before its expert provider acquires the selected experts
(moe_forward's router-first batch, src/inference/deepseek_v4_graph.cpp:1971-2029); the experts'
device copies are the VRAM tier of their residency objects (begin_vram_copy / publish_vram_ready,
include/vastloom/model/residency.hpp:130-131), which the reference declares but never drives. Here
one call:

1. routes the tokens on the device (vl_moe_route) and reads the routes;
2. makes every selected expert (and the shared expert) resident through the matvec accelerator
   (vl_accel_prefetch): every device byte is reserved with the Governor first, a miss is staged
   through the accelerator's pinned slots and copied on its copy stream, then repacked; when the
   residency ceiling is reached the least recently used experts are evicted, and a prefetch hit
   refreshes an expert's recency, so an expert selected by this call is never the one evicted while
   the call's experts fit under the ceiling (checked, and every selected expert confirmed resident
   before the layer runs);
3. points the device expert table at the resident copies (vl_accel_resident_matrix) and runs the
   layer with those routes as given routes (VL_ROUTE_GIVEN): the same kernels, weights and routes
   as a layer whose experts were all resident, hence the same output.

Host experts come from arrays or from an expert pack (vastloom_amd.expert_pack), whose records are
read straight from the mapped payload into the pinned slots.
"""

from __future__ import annotations

import time
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .accel import Accelerator, Governor, PackedMatrix
from .ops import MoeLayer, matrix_layout



@dataclass
class HostExpert:
    """An expert's three matrices in host memory (GGUF bytes; any array or a pack view)."""
    gate_type: int
    down_type: int
    width: int
    intermediate: int
    gate: np.ndarray
    up: np.ndarray
    down: np.ndarray

    @classmethod
    def from_pack(cls, record) -> "HostExpert":
        gt, gr, gc, g = record.matrix("gate")
        _, _, _, u = record.matrix("up")
        dt, dr, dc, d = record.matrix("down")
        return cls(gt, dt, gc, gr, g, u, d)

    def matrices(self, identity_base: int) -> list[PackedMatrix]:
        H, F = self.width, self.intermediate
        return [PackedMatrix(self.gate_type, F, H, self.gate, cache_identity=identity_base + 1),
                PackedMatrix(self.gate_type, F, H, self.up, cache_identity=identity_base + 2),
                PackedMatrix(self.down_type, H, F, self.down, cache_identity=identity_base + 3)]


class ResidentMoeLayer:
    """moe_forward over host experts with Governor-reserved device residency (see the module
    docstring). `accel_options` are vl_accel_options fields; maximum_resident_bytes is the
    residency ceiling."""

    def __init__(self, governor: Governor, experts: list[HostExpert], shared: HostExpert | None, *,
                 width: int, intermediate: int, top_k: int, gate_type: int, down_type: int,
                 semantics: int, routing: int, score_fn: int = _lib.SCORE_SIGMOID,
                 renormalize: bool = True, route_scale: float = 1.0, routed_limit: float = 0.0,
                 shared_limit: float = 0.0, router: torch.Tensor | None = None,
                 bias: torch.Tensor | None = None, layer_id: int = 1, device="cuda",
                 **accel_options):
        if routing == _lib.ROUTE_GIVEN:
            raise ValueError("a resident layer routes its tokens itself")
        self.experts, self.shared = experts, shared
        self.accel = Accelerator(governor, **accel_options)
        E = len(experts)
        # Cache identities: layer, expert (the shared one is E) and projection; never 0.
        self._mats = [e.matrices(((layer_id << 24) | (i << 2)) << 8) for i, e in
                      enumerate(experts + ([shared] if shared else []))]
        common = dict(width=width, intermediate=intermediate, top_k=top_k, gate_type=gate_type,
                      down_type=down_type, semantics=semantics, score_fn=score_fn,
                      renormalize=renormalize, route_scale=route_scale, routed_limit=routed_limit,
                      shared_limit=shared_limit, router=router, bias=bias, device=device)
        # The routing layer reads no expert; the layer that runs takes given routes.
        self._router = _TableLayer(E, shared is not None, routing=routing, **common)
        self._layer = _TableLayer(E, shared is not None, routing=_lib.ROUTE_GIVEN, **common)
        self._table = np.zeros((E + (1 if shared else 0), 3), np.uint64)
        self.timings = {"route_ms": 0.0, "residency_ms": 0.0, "layer_ms": 0.0, "calls": 0}

    def _ensure(self, needed: list[int]) -> None:
        need_bytes = 0
        for e in needed:
            for m in self._mats[e]:
                need_bytes += matrix_layout(m.ggml_type, m.rows, m.storage_columns)[1]
        cap = self.accel.options.maximum_resident_bytes
        if need_bytes > cap:
            raise ValueError(f"one call's experts need {need_bytes} B of residency, above the "
                             f"{cap} B ceiling")
        for e in needed:
            for m in self._mats[e]:
                if not self.accel.prefetch(m):
                    raise RuntimeError(f"expert {e} was declined by the accelerator "
                                       "(Governor budget or free device memory)")
        for e in needed:
            for j, m in enumerate(self._mats[e]):
                if not self.accel.holds(m.cache_identity):
                    raise RuntimeError(f"expert {e} was evicted by this call's own uploads")
                self._table[e, j] = self.accel.resident_matrix(m.cache_identity)

    def forward(self, x: torch.Tensor, out: torch.Tensor | None = None, *,
                table_ids: torch.Tensor | None = None) -> torch.Tensor:
        t0 = time.perf_counter()
        ids, w = self._router.route(x, table_ids=table_ids)  # synchronises the stream
        t1 = time.perf_counter()
        needed = sorted(set(int(i) for i in ids.reshape(-1)))
        if self.shared is not None:
            needed.append(len(self.experts))
        self._ensure(needed)
        self._layer.set_table(self._table)
        t2 = time.perf_counter()
        dev = self._layer.expert_table.device
        gi = torch.from_numpy(np.ascontiguousarray(ids, np.uint32).view(np.int32)).to(dev)
        gw = torch.from_numpy(np.ascontiguousarray(w, np.float32)).to(dev)
        y = self._layer.forward(x, out, given_ids=gi, given_weights=gw)
        torch.cuda.synchronize()
        t3 = time.perf_counter()
        tm = self.timings
        tm["route_ms"] += 1e3 * (t1 - t0)
        tm["residency_ms"] += 1e3 * (t2 - t1)
        tm["layer_ms"] += 1e3 * (t3 - t2)
        tm["calls"] += 1
        return y

    def routes(self, tokens: int) -> tuple[np.ndarray, np.ndarray]:
        return self._layer.routes(tokens)

    def stats(self) -> dict:
        s = self.accel.stats()
        s.update(self.timings)
        if s["upload_ms"] > 0:
            s["h2d_gbs"] = s["uploaded_bytes"] / (s["upload_ms"] * 1e-3) / 1e9
        return s

    def close(self) -> None:
        self.accel.close()


class _TableLayer(MoeLayer):
    """A MoeLayer whose device expert table is written from device addresses (resident copies)."""

    def __init__(self, experts: int, has_shared: bool, **kw):
        class _Stub:
            def weights(self):
                return _lib.ExpertWeights(0, 0, 0)
        stubs = [_Stub() for _ in range(experts)]
        super().__init__(stubs, _Stub() if has_shared else None, **kw)

    def set_table(self, table: np.ndarray) -> None:
        host = torch.from_numpy(np.ascontiguousarray(table, np.uint64).view(np.uint8).reshape(-1))
        self.expert_table.copy_(host)
