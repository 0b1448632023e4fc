#!/usr/bin/env python3
"""Benchmark: quantized expert FFN effective HBM GB/s (and % of peak) and µs per MoE layer, 1 GPU.

A step is one MoE layer over one token: router (float32 [256 x 7168], float64 accumulation),
sigmoid top-8 routing, eight IQ2_XXS routed experts plus the shared expert (7168 -> 2048 ->
7168 SwiGLU each), and the ascending-id combine; all weights resident in HBM before timing.
The value is the layer's quantized weight bytes (9 experts x 11,354,112 B) divided by the
measured time per layer. Tokens rotate through a pool so that routing (and therefore the
experts touched) changes every step, and layer instances rotate so that no weights stay in
cache between their uses.

    python bench.py [--steps K] [--warmup W] [--workload iq2_moe] [--no-cpu-baseline]
    python bench.py --copy-calibration BYTES     plain device copies of BYTES (counter scale)
    python bench.py --matvec q4_k [--matvec-shape 2048x7168] [--matvec-tokens 1]
                                                 device matvec of one storage type alone

ms_per_step is the mean over the K bracketed steps; step_us gives the median and spread of
per-step times from a second pass with an event between steps. roofline.traffic (HBM bytes per
launch of the gate/up kernel) is read from the committed rocprofv3 counter summary
profiles/<kernel>.<workload>.traffic.txt when it exists. The CPU baseline runs the reference's own
kernels on the host in three modes (one thread, the reference runtime policy's thread count, every
usable core), each the median of --cpu-samples tokens.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
PROFILES = ROOT / "profiles"


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=400)
    p.add_argument("--warmup", type=int, default=40)
    p.add_argument("--workload", default="iq2_moe",
                   choices=["q8_expert", "q8_moe", "iq2_moe", "mixed_moe", "grouped_moe",
                            "kquant_moe"])
    p.add_argument("--layers", type=int, default=None,
                   help="layer instances rotated between steps (defeats caching of weights); "
                        "default 6, or 2 for the grouped workload")
    p.add_argument("--token-pool", type=int, default=64)
    p.add_argument("--profile-steps", type=int, default=100)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-samples", type=int, default=10,
                   help="tokens timed per CPU-baseline mode (the median is reported)")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                   help="only run 20 device-to-device copies of BYTES (no layer)")
    p.add_argument("--residency-mib", type=int, default=0, metavar="MIB",
                   help="only run the layer with its experts in host memory and at most MIB of "
                        "them resident (misses streamed through pinned staging); prints its own line")
    p.add_argument("--matvec", default="", metavar="TYPE",
                   help="only time the device matvec of one storage type (q4_k, q5_k, q6_k, mxfp4, "
                        "bf16, f32, q8_0, iq2_xxs, iq3_xxs, iq1_s); prints its own line")
    p.add_argument("--matvec-shape", default="2048x7168", metavar="ROWSxCOLS")
    p.add_argument("--matvec-tokens", type=int, default=1)
    return p.parse_args()


def copy_calibration(nbytes: int) -> int:
    """Plain device copies of known size, for scaling the FETCH_SIZE / WRITE_SIZE counters."""
    import torch

    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(20):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes, "copies": 20}))
    return 0


def measured_traffic(kernel: str, workload: str) -> tuple[int | None, str | None]:
    """HBM bytes per launch of `kernel` from the committed counter summary, if there is one."""
    import re

    path = PROFILES / f"{kernel}.{workload}.traffic.txt"
    if not path.exists():
        return None, None
    m = re.search(r"traffic_bytes_per_launch = (\d+)", path.read_text())
    return (int(m.group(1)), str(path.relative_to(ROOT))) if m else (None, None)


def wide_path(wl) -> bool:
    """Whether a grouped layer of this workload runs on the fp16 kernels (IQ2_XXS gate, up and
    down; widths of whole 256-column blocks)."""
    return (wl.tokens > 8 and wl.gate_type == 16 and wl.down_type == 16 and wl.width % 256 == 0
            and wl.intermediate % 256 == 0)


TILED_TYPES = (8, 16, 18, 19)  # Q8_0, IQ2_XXS, IQ3_XXS, IQ1_S


def gguf_layout(wl) -> bool:
    """Whether the layer has GGUF-layout matrices (it then runs on the grouped plan)."""
    return wl.gate_type not in TILED_TYPES or wl.down_type not in TILED_TYPES


def gateup_kernel(wl) -> str:
    """The gate/up kernel a layer of this workload runs (single-token layers of the learned,
    softmax and given routings take the single-token kernels, except IQ3_XXS; 2-8 tokens the
    token-slot stream kernels; more tokens, or GGUF-layout matrices, the grouped path: the fp16
    kernels for IQ2_XXS, the int8 ones for the other tiled types, k_gguf_moe_gateup for a
    GGUF-layout gate/up)."""
    if wl.gate_type not in TILED_TYPES:
        return "k_gguf_moe_gateup"
    if wl.tokens > 8 or gguf_layout(wl):
        return "k_wide_gateup" if wide_path(wl) else "k_moe_gateup_grouped"
    if wl.tokens == 1 and wl.routing != "zipf_table" and 18 not in (wl.gate_type, wl.down_type):
        return "k_tok_gateup"
    return "k_moe_gateup"


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def usable_cpus() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def token_pool(wl, count: int) -> np.ndarray:
    """The workload's own tokens first, then further seeded N(0, 1) tokens."""
    base = wl.x()
    rng = np.random.Generator(np.random.PCG64(np.random.SeedSequence([wl.seed, 2, 1])))
    extra = rng.standard_normal((max(0, count * wl.tokens - base.shape[0]), wl.width))
    pool = np.concatenate([base, extra.astype(np.float32)])
    return pool[: count * wl.tokens].reshape(count, wl.tokens, wl.width)


def build_layers(wl, instances: int):
    import torch

    from vastloom_amd import _lib, ops

    experts = [wl.expert(e) for e in range(wl.experts)]
    shared = wl.shared()
    sem = _lib.SEM_QWEN if wl.semantics == "qwen" else _lib.SEM_DEEPSEEK
    routing = {"softmax": _lib.ROUTE_SOFTMAX, "single": _lib.ROUTE_GIVEN,
               "zipf_table": _lib.ROUTE_TABLE}.get(wl.routing, _lib.ROUTE_LEARNED)
    router = torch.from_numpy(wl.router())
    layers = []
    for _ in range(instances):
        devs = [ops.DeviceExpert(wl.gate_type, wl.down_type, wl.width, wl.intermediate,
                                 e.gate, e.up, e.down) for e in experts]
        sh = (ops.DeviceExpert(wl.gate_type, wl.down_type, wl.width, wl.intermediate,
                               shared.gate, shared.up, shared.down) if shared else None)
        torch.cuda.synchronize()
        for d in devs + ([sh] if sh else []):
            d.release_staging()
        layers.append(ops.MoeLayer(devs, sh, width=wl.width, intermediate=wl.intermediate,
                                   top_k=wl.top_k, gate_type=wl.gate_type,
                                   down_type=wl.down_type, semantics=sem, routing=routing,
                                   score_fn=wl.score_fn, router=router))
    return experts, shared, layers


def cpu_baseline(wl, experts, shared, pool, samples: int, measured: float | None = None) -> dict:
    """The reference's own CPU kernels (oracle/_ref, built from its sources) on a bounded sample
    of the same workload: for each token, router logits and routing, then per selected expert the
    reference matvecs (row-split over the mode's threads; IQ1_S and IQ3_XXS stay serial, as in the
    reference), SwiGLU and combine. Three modes: one thread, the reference runtime policy's thread
    count (the reported value), every usable core; each the median of `samples` tokens."""
    from oracle.oracle import Oracle, Reference, default_threads

    orc = Oracle()
    kind = "reference" if Reference.available() else "port"
    ref = Reference() if kind == "reference" else None
    H, F = wl.width, wl.intermediate
    router = wl.router()
    table = wl.zipf_table() if wl.routing == "zipf_table" else None

    def token_time(xt, t, threads) -> float:
        def matvec(qtype, data, rows, cols, x):
            if ref is not None:
                return ref.matvec(qtype, data, rows, cols, x, threads=threads)
            return orc.matvec(qtype, data, rows, cols, x, threads=threads)

        def expert(e, x, w_route):
            g = matvec(e.gate_type, e.gate, F, H, x)
            u = matvec(e.gate_type, e.up, F, H, x)
            if wl.semantics == "qwen":
                h = (np.array([orc.silu_f(float(v)) for v in g], np.float32) * u).astype(np.float32)
            else:
                gv, uv = g.astype(np.float64), u.astype(np.float64)
                h = gv / (1.0 + np.exp(-gv)) * uv
                if w_route is not None:
                    h = h * np.float64(w_route)
                h = h.astype(np.float32)
            return matvec(e.down_type, e.down, H, F, h)

        t0 = time.perf_counter()
        if wl.routing == "single":
            expert(experts[0], xt, None)
        else:
            logits = orc.linear_f64(router, xt, wl.experts)
            if wl.routing == "softmax":
                ids, w = orc.route_softmax(logits[0], wl.top_k, True)
            elif table is not None:
                ids, w = orc.route_hash(logits, np.zeros(1, np.uint32), table[t:t + 1],
                                        wl.top_k, wl.route_scale, wl.score_fn)
                ids, w = ids[0], w[0]
            else:
                ids, w = orc.route_learned(logits, None, wl.top_k, 1.0, wl.score_fn)
                ids, w = ids[0], w[0]
            out = np.zeros(H, np.float32)
            for e, wr in sorted(zip(ids, w)):
                y = expert(experts[e], xt, wr if wl.semantics == "deepseek" else None)
                out += y * wr if wl.semantics == "qwen" else y
            if shared is not None:
                out += expert(shared, xt, None)
        return time.perf_counter() - t0

    layer_bytes = layer_weight_bytes(wl, measured)
    modes = {}
    for mode, threads in (("threads_1", 1), ("policy", default_threads()), ("all_cores", usable_cpus())):
        per_token = []
        for i in range(samples):
            batch, t = i // wl.tokens, i % wl.tokens
            per_token.append(token_time(pool[batch % len(pool)][t], t, threads))
        per_layer = np.array(per_token) * wl.tokens  # tokens are independent
        med = float(np.median(per_layer))
        modes[mode] = {"threads": threads, "us_per_layer_median": round(med * 1e6, 1),
                       "us_per_layer_min": round(float(per_layer.min()) * 1e6, 1),
                       "us_per_layer_max": round(float(per_layer.max()) * 1e6, 1),
                       "gbs_median": round(layer_bytes / med / 1e9, 4), "samples": samples}
    pol = modes["policy"]
    return {"value": pol["gbs_median"], "unit": "GB/s", "cores": pol["threads"], "kind": kind,
            "us_per_layer": pol["us_per_layer_median"], "modes": modes,
            "cpu_model": cpu_model(), "nproc": usable_cpus(),
            "sample": f"{samples} token(s) per mode of the {wl.name} workload ({wl.tokens} per layer; "
                      f"per-layer time = median per-token time x {wl.tokens}); value = the "
                      f"reference runtime policy's {pol['threads']} threads of {usable_cpus()} usable CPUs"}


def routed_experts(wl, measured: float | None = None) -> float:
    """Distinct routed experts one layer call reads (for learned multi-token routing, the mean
    over the token pool of what the device routed, passed in as `measured`)."""
    if wl.routing == "single":
        return 1
    if wl.tokens == 1:
        return wl.top_k
    if wl.routing == "zipf_table":
        return int(np.unique(wl.zipf_table()).size)
    if measured is None:
        raise ValueError("per-layer bytes depend on the activations for this multi-token workload")
    return measured


def layer_weight_bytes(wl, measured: float | None = None) -> int:
    return int(round((routed_experts(wl, measured) + (1 if wl.has_shared else 0)) * wl.expert_bytes()))


def device_routed_experts(layer, pool, table) -> float:
    """Mean number of distinct experts the device routes each pool entry's tokens to."""
    counts = []
    for b in range(len(pool)):
        layer.forward(pool[b], check=False, table_ids=table)
        ids, _ = layer.routes(pool.shape[1])
        counts.append(np.unique(ids).size)
    return float(np.mean(counts))


def residency_run(args) -> int:
    """The layer over experts held in host memory, made resident on demand under a residency
    ceiling of args.residency_mib MiB (Governor-reserved): per-layer time including routing,
    misses and their uploads, and the host-to-device rate of the uploads (staging copy, DMA and
    repacking), next to the 7.2 GB/s the reference's CUDA tier measured for its pinned copies
    (docs/reports/D2B_DEVICE_RESIDENCY_VALIDATION.md:49)."""
    import torch

    from vastloom_amd import _lib
    from vastloom_amd.accel import Governor, default_limits
    from vastloom_amd.residency import HostExpert, ResidentMoeLayer
    from vastloom_amd.workloads import workload

    wl = workload(args.workload)
    if wl.routing in ("single", "zipf_table"):
        raise SystemExit("the residency run needs a routed workload")
    H, F = wl.width, wl.intermediate
    def host_expert(ex):
        return HostExpert(wl.gate_type, wl.down_type, H, F, ex.gate, ex.up, ex.down)

    host = [host_expert(wl.expert(e)) for e in range(wl.experts)]
    shared = wl.shared()
    sh = host_expert(shared) if shared else None
    ceiling = args.residency_mib << 20
    gov = Governor(default_limits(vram_hard_limit=ceiling + (512 << 20), staging_hard_limit=1 << 30))
    sem = _lib.SEM_QWEN if wl.semantics == "qwen" else _lib.SEM_DEEPSEEK
    routing = _lib.ROUTE_SOFTMAX if wl.routing == "softmax" else _lib.ROUTE_LEARNED
    layer = ResidentMoeLayer(gov, host, sh, width=H, intermediate=F, top_k=wl.top_k,
                             gate_type=wl.gate_type, down_type=wl.down_type, semantics=sem,
                             routing=routing, score_fn=wl.score_fn,
                             router=torch.from_numpy(wl.router()),
                             maximum_resident_bytes=ceiling, staging_bytes=64 << 20)
    pool = torch.from_numpy(token_pool(wl, args.token_pool)).cuda()
    for i in range(args.warmup):
        layer.forward(pool[i % len(pool)])
    s0 = layer.stats()
    t0 = time.perf_counter()
    for i in range(args.steps):
        layer.forward(pool[(args.warmup + i) % len(pool)])
    elapsed = time.perf_counter() - t0
    s1 = layer.stats()
    up_bytes = s1["uploaded_bytes"] - s0["uploaded_bytes"]
    up_ms = s1["upload_ms"] - s0["upload_ms"]
    n_exp = routed_experts(wl) + (1 if wl.has_shared else 0)
    print(json.dumps({
        "metric": "MoE layer with experts streamed from host memory under a residency ceiling",
        "workload": wl.name, "ceiling_mib": args.residency_mib, "steps": args.steps,
        "us_per_layer": round(elapsed / args.steps * 1e6, 1),
        "route_us": round((s1["route_ms"] - s0["route_ms"]) / args.steps * 1e3, 1),
        "residency_us": round((s1["residency_ms"] - s0["residency_ms"]) / args.steps * 1e3, 1),
        "layer_us": round((s1["layer_ms"] - s0["layer_ms"]) / args.steps * 1e3, 1),
        "uploaded_bytes_per_layer": int(up_bytes / args.steps),
        "miss_rate": round(up_bytes / args.steps / (n_exp * wl.expert_bytes()), 3),
        "h2d_gbs": round(up_bytes / (up_ms * 1e-3) / 1e9, 2) if up_ms else None,
        "reference_h2d_gbs": 7.2,
        "evicted": s1["evicted"] - s0["evicted"], "resident_matrices": s1["resident_matrices"]}))
    layer.close()
    return 0


def matvec_run(args) -> int:
    """The device matvec of one storage type alone: y = W x for one matrix of ROWS x COLS.

    Matrix instances (copies of one random matrix at distinct addresses, more than 1 GiB in all)
    rotate so that no weights stay in the 256 MiB last-level cache between uses. A spin kernel
    holds the stream while all launches are queued, so the timed region is the launches back to
    back: per launch, the status clear and the matvec kernel. GB/s = matrix bytes / time.
    """
    import ctypes as C

    import torch

    from vastloom_amd import ops
    from vastloom_amd._lib import call
    from vastloom_amd.workloads import TYPE_NAMES, random_matrix

    by_name = {v: k for k, v in TYPE_NAMES.items()}
    qtype = by_name[args.matvec]
    rows, cols = (int(v) for v in args.matvec_shape.lower().split("x"))
    tokens = args.matvec_tokens
    enc = random_matrix(np.random.default_rng(12), qtype, rows, cols, 0.01)
    src = torch.from_numpy(enc).cuda()
    copies = max(2, min(512, (1 << 30) // enc.size + 1))
    mats = [ops.DeviceMatrix(qtype, rows, cols, src) for _ in range(copies)]
    x = torch.randn((tokens, cols), dtype=torch.float32, device="cuda")
    ws_bytes = C.c_uint64()
    call("vl_matvec_workspace", qtype, rows, cols, tokens, C.byref(ws_bytes))
    ws = [torch.zeros(ws_bytes.value, dtype=torch.uint8, device="cuda") for _ in range(2)]
    y = torch.empty((tokens, rows), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream

    def launch(i):
        call("vl_matvec", qtype, rows, cols, mats[i % copies].ptr(), x.data_ptr(), tokens,
             y.data_ptr(), ws[i & 1].data_ptr(), ws_bytes.value, sp)

    for i in range(args.warmup):
        launch(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(50_000_000)  # holds the stream while the launches below are queued
    start.record(stream)
    for i in range(args.steps):
        launch(i)
    end.record(stream)
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1e3 / args.steps
    bits = ops.read_status(ws[0], sp) | ops.read_status(ws[1], sp)
    if bits:
        raise RuntimeError(f"matvec raised status bits {bits:#x}")
    gbs = enc.size / (us * 1e-6) / 1e9
    print(json.dumps({
        "metric": "matvec_hbm_gbs", "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "us_per_launch": round(us, 3),
        "higher_is_better": True, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"matvec {args.matvec} {rows}x{cols} tokens={tokens}",
                   "matrix_bytes": int(enc.size), "instances": copies},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "note": "per launch including the status-clear kernel"}}))
    return 0


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported on this path "
              "(no multi-GPU sharding or collectives are built)", file=sys.stderr)
        return 2
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)
    if args.residency_mib:
        return residency_run(args)
    if args.matvec:
        return matvec_run(args)
    import torch

    from vastloom_amd import ops
    from vastloom_amd.workloads import workload

    wl = workload(args.workload)
    if args.layers is None:
        args.layers = 6 if wl.tokens == 1 else 2
    if wl.tokens > 1:
        args.token_pool = min(args.token_pool, 4)
    t_build = time.perf_counter()
    experts, shared, layers = build_layers(wl, args.layers)
    pool_host = token_pool(wl, args.token_pool)
    pool = torch.from_numpy(pool_host).cuda()
    table = (torch.from_numpy(np.ascontiguousarray(wl.zipf_table(), np.uint32)).cuda()
             if wl.routing == "zipf_table" else None)
    outs = [torch.empty((wl.tokens, wl.width), dtype=torch.float32, device="cuda")
            for _ in range(2)]
    print(f"# built {args.layers} layer instance(s) of {wl.name} in "
          f"{time.perf_counter() - t_build:.1f}s", file=sys.stderr, flush=True)

    def step(i, **kw):
        layer = layers[i % len(layers)]
        return layer.forward(pool[i % len(pool)], outs[i % 2], check=False, table_ids=table, **kw)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(args.steps):
        step(i)
    end.record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    ms_per_step = total_ms / args.steps
    # Per-step times: a second pass with an event recorded between consecutive steps.
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    evs[0].record()
    for i in range(args.steps):
        step(i)
        evs[i + 1].record()
    torch.cuda.synchronize()
    per_step = np.array([evs[i].elapsed_time(evs[i + 1]) * 1000.0 for i in range(args.steps)])
    step_us = {"median": round(float(np.median(per_step)), 2),
               "p10": round(float(np.percentile(per_step, 10)), 2),
               "p90": round(float(np.percentile(per_step, 90)), 2),
               "min": round(float(per_step.min()), 2), "max": round(float(per_step.max()), 2)}
    stream = torch.cuda.current_stream().cuda_stream
    for layer in layers:
        for ws in layer._ws.values():
            bits = ops.read_status(ws, stream)
            if bits:
                raise RuntimeError(f"layer reported status bits {bits:#x}")

    # Per-stage durations from HIP events on the same stream, in a separate profiled pass; then
    # each stage's kernel alone, from events the launch records around its execution, in another.
    tl = ops.Timeline(args.profile_steps)
    for i in range(args.profile_steps):
        step(i, timeline=tl, call_slot=i)
    torch.cuda.synchronize()
    stages = [tl.stage_ms(i) for i in range(args.profile_steps)]
    tl.close()
    tk = ops.Timeline(args.profile_steps, kernel_brackets=True)
    for i in range(args.profile_steps):
        step(i, timeline=tk, call_slot=i)
    torch.cuda.synchronize()
    kernels = [tk.kernel_ms(i) for i in range(args.profile_steps)]
    tk.close()
    stage_us = {k: round(1000.0 * float(np.mean([s[k] for s in stages])), 2) for k in stages[0]}
    kernel_us = {k: round(1000.0 * float(np.mean([s[k] for s in kernels])), 2) for k in kernels[0]}

    measured = None
    if wl.tokens > 1 and wl.routing not in ("zipf_table", "single"):
        measured = device_routed_experts(layers[0], pool, table)
    layer_bytes = layer_weight_bytes(wl, measured)
    gbs = layer_bytes / (ms_per_step * 1e-3) / 1e9
    # Dominant kernel: the gate/up pass, which reads two matrices of every selected expert.
    n_exp = routed_experts(wl, measured) + (1 if wl.has_shared else 0)
    H, F = wl.width, wl.intermediate
    from vastloom_amd.workloads import storage_bytes
    gateup_bytes = n_exp * 2 * storage_bytes(wl.gate_type, F, H)
    # The kernels' own durations (events around their execution), as a kernel trace reports them.
    gateup_gbs = gateup_bytes / (kernel_us["gate_up"] * 1e-6) / 1e9
    down_gbs = n_exp * storage_bytes(wl.down_type, H, F) / (kernel_us["down"] * 1e-6) / 1e9
    gu_kernel = gateup_kernel(wl)
    traffic, traffic_src = measured_traffic(gu_kernel, wl.name)

    result = {
        "metric": "quant expert FFN effective HBM GB/s (% of peak) + us per MoE layer, 1 GPU",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "us_per_layer": round(ms_per_step * 1000.0, 2),
        "step_us": step_us,
        "pct_of_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"{TYPE(wl.gate_type).lower()}/{TYPE(wl.down_type).lower()} weights, "
                 + ("f16xf16->f32 MFMA (exact fp16 weights, hi/lo fp16 activations)" if wide_path(wl)
                    else "f32 FMA on the decoded codes, block scales factored out"
                    if wl.gate_type not in TILED_TYPES
                    else "i8xi8->i32 MFMA, f32 accumulate"),
        "data": f"synthetic (seeded PCG64; uniform random {TYPE(wl.gate_type)}/{TYPE(wl.down_type)} "
                f"payload bytes, |N(0,1)|*{wl.scale_factor} fp16 scales, N(0,0.02) router, N(0,1) tokens)",
        "config": {"workload": f"{wl.name}: {wl.model} {wl.kind}, width {wl.width}, expert "
                               f"width {wl.intermediate}, {wl.experts} routed experts top-"
                               f"{wl.top_k} + {int(wl.has_shared)} shared, {wl.tokens} token(s), "
                               f"{ROUTER_NAME[wl.routing]} router, {TYPE(wl.gate_type)} gate/up, "
                               f"{TYPE(wl.down_type)} down",
                   "tokens": wl.tokens, "selected_experts": n_exp,
                   "tokens_per_s": round(wl.tokens / (ms_per_step * 1e-3), 1),
                   "quantized_bytes_per_layer": layer_bytes,
                   "router_bytes_per_layer": wl.router_bytes(),
                   "layer_instances": args.layers, "token_pool": args.token_pool},
        "stages_us": stage_us,
        "kernels_us": kernel_us,
        "roofline": {"bound": "hbm", "kernel": gu_kernel,
                     "achieved": round(gateup_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gateup_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "bytes_per_launch": gateup_bytes,
                     "kernel_avg_us": kernel_us["gate_up"],
                     "down_kernel_achieved": round(down_gbs, 1)},
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(wl, experts, shared, pool_host, args.cpu_samples,
                                              measured)
    print(json.dumps(result))
    return 0


ROUTER_NAME = {"learned": "sigmoid", "softmax": "softmax", "single": "no",
               "zipf_table": "Zipf(1.1) table"}


def TYPE(t: int) -> str:
    from vastloom_amd.workloads import TYPE_NAMES

    return TYPE_NAMES[t].upper()


if __name__ == "__main__":
    sys.exit(main())
