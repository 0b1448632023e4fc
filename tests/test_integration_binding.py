"""The reference-side binding (integration/hip_matvec_accelerator.hpp) compiled against the
reference's own headers, Governor, packed-matrix payload and CPU matvec, and driven through the
graph's accelerator seam (DeepseekV4MatvecAccelerator::matvec,
include/vastloom/inference/deepseek_v4_reference.hpp:437-451) by tests/integration/accel_binding.cpp.

The driver is built from the reference sources in this container (make -C oracle binding) into
oracle/_ref/accel_binding, which travels with the tree; where neither the reference tree nor a
built driver is present the tests are skipped.
"""

from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
DRIVER = ROOT / "oracle" / "_ref" / "accel_binding"


def _driver() -> Path:
    if not DRIVER.exists() and Path("/root/reference/src/inference").is_dir():
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "binding"], check=True)
    if not DRIVER.exists():
        pytest.skip("the binding driver is not built and the reference tree is absent")
    return DRIVER


def _run(mode: str) -> str:
    proc = subprocess.run([str(_driver()), mode], capture_output=True, text=True, timeout=120)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert f"{mode}: 0 failure(s)" in proc.stdout
    return proc.stdout


def test_binding_through_fake_device():
    """Ok(true) bit-identical to the reference's CPU matvec, Ok(false) with the output untouched,
    errors, and every byte accounted for by the reference's ResourceGovernor."""
    out = _run("fake")
    for case in ("fake output bit-identical to the reference", "no identity declined, output untouched",
                 "non-finite input is an error, output untouched", "destroy returns every reservation",
                 "failed upload is an error, nothing resident or charged"):
        assert f"ok {case}" in out


@pytest.mark.gpu
def test_binding_through_hip_device():
    """The same seam on the MI355X: IQ2_XXS outputs within 1e-5 * |w_row| * |x| of the reference,
    declines and Governor accounting as on the fake device."""
    out = _run("hip")
    assert "ok device output within 1e-5 |w_row| |x| of the reference" in out
