"""The record hand-off of the stream kernels, checked in the compiled gfx950 code.

A wave that hands a job's partial sums to another wave stores its record with agent-scope
atomic stores, waits until they have completed (s_waitcnt vmcnt(0)), then bumps the job's
counter with a relaxed agent-scope atomic add (vl_stream.h arrive, vl_moe_token.hip). The wave
that sees the last count reads the records with agent-scope atomic loads only after the add has
returned. The acquire-release form of the counter is correct under the memory model without
this reasoning, but on MI355X each one writes back and invalidates the XCD's L2 (buffer_wbl2,
buffer_inv): measured, iq2_moe went from 50.9 to 61.8 us per layer and mixed_moe from 272 to
1,117 us. So the protocol rests on the ordering of the instructions themselves, and this test
reads it from the compiler's output for every returning counter add (global_atomic_add ... sc0):
no global store may be outstanding at the add (none issued since the last vmcnt(0) wait), and
no global load may be issued between the add and the wait for its result.
"""

from __future__ import annotations

import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

from vastloom_amd import build as B

SOURCES = ["vl_kernels.hip", "vl_moe.hip", "vl_moe_token.hip"]


def ordering_violations(asm: str) -> tuple[int, list[tuple[str, int, str, str]]]:
    """(returning counter adds seen, violations) of a linear scan over one assembly file."""
    bad, adds = [], 0
    pending_store = awaiting = False
    fn = None
    for i, line in enumerate(asm.splitlines()):
        t = line.strip()
        if re.match(r"^[_A-Za-z][\w.$]*:", t) and not t.startswith(".L"):
            fn, pending_store, awaiting = t[:-1], False, False
            continue
        if not t or t.startswith((";", ".")):
            continue
        op = t.split()[0]
        if op == "s_waitcnt" and "vmcnt(0)" in t:
            pending_store = awaiting = False
            continue
        returning = " sc0" in t
        if op.startswith(("global_store", "buffer_store", "flat_store")) or (
                op.startswith("global_atomic") and not returning):
            pending_store = True
        if op.startswith("global_atomic_add") and returning:
            adds += 1
            if pending_store:
                bad.append((fn, i + 1, "store outstanding at the counter add", t))
            awaiting = True
            continue
        if awaiting and op.startswith(("global_load", "buffer_load", "flat_load")):
            bad.append((fn, i + 1, "load issued before the counter's result", t))
    return adds, bad


def test_checker_finds_planted_mistakes():
    ok = """k:
    global_store_dword v[0:1], v2, off sc1
    s_waitcnt vmcnt(0) expcnt(0) lgkmcnt(0)
    global_atomic_add v3, v[4:5], v6, off sc0
    s_waitcnt vmcnt(0)
    global_load_dword v7, v[8:9], off sc1
"""
    assert ordering_violations(ok) == (1, [])
    store_late = ok.replace("    s_waitcnt vmcnt(0) expcnt(0) lgkmcnt(0)\n", "", 1)
    assert [b[2] for b in ordering_violations(store_late)[1]] == ["store outstanding at the counter add"]
    load_early = ok.replace("    s_waitcnt vmcnt(0)\n    global_load", "    global_load", 1)
    assert [b[2] for b in ordering_violations(load_early)[1]] == ["load issued before the counter's result"]


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="needs hipcc")
def test_handoff_ordering_in_compiled_kernels(tmp_path):
    def compile_asm(src: str) -> Path:
        out = tmp_path / (Path(src).stem + ".s")
        cmd = [B.hipcc(), *[f for f in B.FLAGS if f != "-fPIC"], "-S", "--cuda-device-only",
               str(B.CSRC / src), "-o", str(out)]
        subprocess.run(cmd, check=True, capture_output=True, text=True)
        return out

    with ThreadPoolExecutor(len(SOURCES)) as pool:
        outs = list(pool.map(compile_asm, SOURCES))
    total = 0
    for src, out in zip(SOURCES, outs):
        adds, bad = ordering_violations(out.read_text())
        assert not bad, (src, bad[:5])
        total += adds
    assert total > 0, "no hand-off counters found: the scan no longer matches the code"
