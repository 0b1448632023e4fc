"""Summaries of rocprofv3 output for the stream kernels (text, a few KB).

    python -m vastloom_amd.profiling trace DIR            per-kernel durations (--kernel-trace --stats)
    python -m vastloom_amd.profiling pmc DIR [DIR ...]    per-kernel mean counter values (--pmc)
    python -m vastloom_amd.profiling traffic --fetch DIR --write DIR --calib-fetch DIR
                                             --calib-write DIR --calib-bytes N --kernel REGEX
    python -m vastloom_amd.profiling counters --trace DIR --kernel REGEX DIR [DIR ...]
                                             counter means per dispatch of the kernels matching
                                             REGEX, with the wave-state split and int8 MFMA rate

rocprofv3 is run with ``--output-format csv``; DIR is its ``-d`` directory. ``traffic`` turns the
FETCH_SIZE and WRITE_SIZE counters (KiB per dispatch) of one kernel into HBM bytes per launch,
each scaled by what the same counter reads for a plain copy of known size (the copy reads and
writes ``--calib-bytes`` bytes per dispatch).
"""

from __future__ import annotations

import argparse
import csv
import re
import statistics
import sys
from collections import defaultdict
from pathlib import Path


def _csvs(d: str, suffix: str) -> list[Path]:
    out = sorted(Path(d).rglob(f"*{suffix}"))
    if not out:
        raise FileNotFoundError(f"no *{suffix} under {d}")
    return out


def _short(name: str) -> str:
    """A kernel's name without its parameter list, return type or anonymous-namespace part."""
    name = name.replace("(anonymous namespace)::", "")
    name = re.sub(r"^void ", "", name)
    return re.sub(r"\(.*", "", name).strip()


def kernel_stats(d: str) -> list[dict]:
    """Rows of rocprofv3's kernel_stats.csv: name, calls, average/min/max duration (us)."""
    rows = []
    for f in _csvs(d, "kernel_stats.csv"):
        for r in csv.DictReader(open(f)):
            rows.append({"name": _short(r["Name"]), "calls": int(r["Calls"]),
                         "avg_us": float(r["AverageNs"]) / 1e3, "min_us": float(r["MinNs"]) / 1e3,
                         "max_us": float(r["MaxNs"]) / 1e3, "pct": float(r["Percentage"])})
    return sorted(rows, key=lambda r: -r["pct"])


def pmc_means(dirs: list[str], kernel: str | None = None) -> dict[str, dict[str, float]]:
    """Mean counter value per dispatch, per kernel and counter."""
    rx = re.compile(kernel) if kernel else None
    vals: dict[str, dict[str, list[float]]] = defaultdict(lambda: defaultdict(list))
    for d in dirs:
        for f in _csvs(d, "counter_collection.csv"):
            for r in csv.DictReader(open(f)):
                k = _short(r["Kernel_Name"])
                if rx and not rx.search(k):
                    continue
                vals[k][r["Counter_Name"]].append(float(r["Counter_Value"]))
    return {k: {c: statistics.mean(v) for c, v in cs.items()} for k, cs in vals.items()}


def _largest(means: dict[str, dict[str, float]], counter: str, kernel: str | None) -> tuple[str, float]:
    cands = [(k, cs[counter]) for k, cs in means.items() if counter in cs
             and (kernel is None or re.search(kernel, k))]
    if not cands:
        raise KeyError(f"no {counter} for kernel {kernel!r}")
    return max(cands, key=lambda kv: kv[1])


def traffic(fetch: str, write: str, calib_fetch: str, calib_write: str, calib_bytes: int,
            kernel: str) -> dict:
    kf, f_kib = _largest(pmc_means([fetch]), "FETCH_SIZE", kernel)
    kw, w_kib = _largest(pmc_means([write]), "WRITE_SIZE", kernel)
    cf, cf_kib = _largest(pmc_means([calib_fetch]), "FETCH_SIZE", None)
    cw, cw_kib = _largest(pmc_means([calib_write]), "WRITE_SIZE", None)
    f_scale = calib_bytes / (cf_kib * 1024.0)
    w_scale = calib_bytes / (cw_kib * 1024.0)
    return {"kernel": kf, "fetch_kib": f_kib, "write_kib": w_kib, "calib_kernel": cf,
            "calib_fetch_kib": cf_kib, "calib_write_kib": cw_kib, "calib_bytes": calib_bytes,
            "fetch_scale": f_scale, "write_scale": w_scale,
            "fetch_bytes": f_kib * 1024.0 * f_scale, "write_bytes": w_kib * 1024.0 * w_scale,
            "traffic_bytes": f_kib * 1024.0 * f_scale + w_kib * 1024.0 * w_scale}


def counters(dirs: list[str], kernel: str, trace: str | None = None) -> list[str]:
    """Mean counter values per dispatch of each kernel matching `kernel`, and what follows from them:
    the share of wave cycles spent waiting on an instruction's operands (SQ_WAIT_INST_ANY, mostly
    s_waitcnt) and issuing (SQ_ACTIVE_INST_ANY); int8 and f16 MFMA operations
    (SQ_INSTS_VALU_MFMA_MOPS_I8 / _F16 count units of 512) and, with the kernel's average duration
    from a trace, their rate against the dense peak."""
    means = pmc_means(dirs, kernel)
    durations = {r["name"]: r["avg_us"] for r in kernel_stats(trace)} if trace else {}
    out = []
    for k, cs in sorted(means.items()):
        out.append(k)
        for c, v in sorted(cs.items()):
            out.append(f"    {c:34s} {v:18.2f}")
        wc = cs.get("SQ_WAVE_CYCLES")
        if wc:
            if "SQ_WAIT_INST_ANY" in cs:
                out.append(f"    {'-> waiting on operands':34s} {100.0 * cs['SQ_WAIT_INST_ANY'] / wc:17.1f}% of wave cycles")
            if "SQ_ACTIVE_INST_ANY" in cs:
                out.append(f"    {'-> issuing':34s} {100.0 * cs['SQ_ACTIVE_INST_ANY'] / wc:17.1f}% of wave cycles")
            if "SQ_WAIT_INST_LDS" in cs:
                out.append(f"    {'-> waiting on LDS':34s} {100.0 * cs['SQ_WAIT_INST_LDS'] / wc:17.1f}% of wave cycles")
        for counter, label, peak in (("SQ_INSTS_VALU_MFMA_MOPS_I8", "int8", "dense int8 peak 5000 TOPS"),
                                     ("SQ_INSTS_VALU_MFMA_MOPS_F16", "f16", "dense f16 peak 2500 TFLOP/s")):
            if counter not in cs:
                continue
            ops = cs[counter] * 512.0
            line = f"    {'-> ' + label + ' MFMA ops per dispatch':34s} {ops:18.4e}"
            us = next((d for n, d in durations.items() if n == k), None)
            if us:
                line += f"   at {us:.2f} us: {ops / (us * 1e-6) / 1e12:.1f} T/s ({peak})"
            out.append(line)
    return out


def main(argv: list[str] | None = None) -> int:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = p.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("dir")
    m = sub.add_parser("pmc")
    m.add_argument("dirs", nargs="+")
    m.add_argument("--kernel")
    tr = sub.add_parser("traffic")
    for a in ("fetch", "write", "calib-fetch", "calib-write"):
        tr.add_argument(f"--{a}", required=True)
    tr.add_argument("--calib-bytes", type=int, required=True)
    tr.add_argument("--kernel", required=True)
    cn = sub.add_parser("counters")
    cn.add_argument("dirs", nargs="+")
    cn.add_argument("--kernel", required=True)
    cn.add_argument("--trace")
    a = p.parse_args(argv)
    if a.cmd == "trace":
        print(f"{'kernel':72s} {'calls':>6s} {'avg_us':>9s} {'min_us':>9s} {'max_us':>9s} {'pct':>6s}")
        for r in kernel_stats(a.dir):
            print(f"{r['name'][:72]:72s} {r['calls']:6d} {r['avg_us']:9.2f} {r['min_us']:9.2f} "
                  f"{r['max_us']:9.2f} {r['pct']:6.2f}")
    elif a.cmd == "counters":
        print("\n".join(counters(a.dirs, a.kernel, a.trace)))
    elif a.cmd == "pmc":
        for k, cs in pmc_means(a.dirs, a.kernel).items():
            print(k)
            for c, v in sorted(cs.items()):
                print(f"    {c:30s} {v:16.1f}")
    else:
        r = traffic(a.fetch, a.write, a.calib_fetch, a.calib_write, a.calib_bytes, a.kernel)
        print(f"kernel                 {r['kernel']}")
        print(f"FETCH_SIZE             {r['fetch_kib']:.1f} KiB/dispatch x {r['fetch_scale']:.3f}"
              f" = {r['fetch_bytes']:.0f} B")
        print(f"WRITE_SIZE             {r['write_kib']:.1f} KiB/dispatch x {r['write_scale']:.3f}"
              f" = {r['write_bytes']:.0f} B")
        print(f"calibration kernel     {r['calib_kernel']} ({r['calib_bytes']} B read and written:"
              f" FETCH_SIZE {r['calib_fetch_kib']:.1f} KiB, WRITE_SIZE {r['calib_write_kib']:.1f} KiB)")
        print(f"traffic_bytes_per_launch = {r['traffic_bytes']:.0f}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
