"""The matvec accelerator on the MI355X, through the C ABI: uploads in row ranges through pinned
staging on the copy stream, packing on the compute stream, resident decode bit-exact against the
oracle, matvec within 1e-5 * |w_row| * |x|, residency reuse, and Governor accounting of every
device and pinned byte (src/cuda/cuda_matvec_accelerator.cpp:102-314)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.oracle import (BF16, F32, IQ1_S, IQ2_S, IQ2_XXS, IQ3_XXS, MXFP4, Q4_K, Q5_K, Q6_K,
                           Q8_0)
from vastloom_amd import _lib
from vastloom_amd.accel import (KIND_STAGING, KIND_VRAM, Accelerator, Buffer, Governor,
                                PackedMatrix, VlError, default_limits)
from vastloom_amd.workloads import random_matrix

pytestmark = pytest.mark.gpu

MiB, GiB = 1 << 20, 1 << 30
TOL = 1e-5


@pytest.fixture(scope="module")
def gov():
    assert torch.cuda.is_available(), "GPU tests need a visible HIP device"
    return Governor(default_limits(vram_hard_limit=8 * GiB, staging_hard_limit=512 * MiB))


def within(y, w, x):
    bound = TOL * np.linalg.norm(w.astype(np.float64), axis=1) * np.linalg.norm(x.astype(np.float64))
    return np.all(np.abs(y.astype(np.float64) - w.astype(np.float64) @ x.astype(np.float64)) <= bound + 1e-30)


CASES = [(Q8_0, 100, 512), (IQ2_XXS, 100, 1024), (IQ3_XXS, 33, 512), (IQ1_S, 31, 768),
         (IQ2_XXS, 2048, 7168),
         # GGUF-layout types: resident as their GGUF bytes, uploaded in row ranges as the others.
         (Q4_K, 2048, 7168), (Q5_K, 100, 1024), (Q6_K, 77, 2048), (MXFP4, 45, 2880),
         (IQ2_S, 65, 2048), (BF16, 33, 100), (F32, 64, 512)]


@pytest.mark.parametrize("qtype,rows,cols", CASES)
def test_upload_decode_and_matvec(gov, oracle, qtype, rows, cols):
    print(f"[accel] type {qtype} {rows}x{cols}", flush=True)
    rng = np.random.Generator(np.random.PCG64([qtype, rows, cols]))
    enc = random_matrix(rng, qtype, rows, cols, 0.01)
    x = rng.standard_normal(cols).astype(np.float32)
    # Slots of 256 KiB: the 2048-row matrix goes up in 32 ranges through both slots.
    acc = Accelerator(gov, staging_bytes=512 * 1024, minimum_free_vram_after=0)
    try:
        m = PackedMatrix(qtype, rows, cols, enc, cache_identity=1000 + qtype)
        y = np.zeros(rows, np.float32)
        assert acc.matvec(m, x, y)
        w = oracle.dequantize(qtype, enc, rows * cols).reshape(rows, cols)
        assert within(y, w, x)
        want = oracle.matvec(qtype, enc, rows, cols, x)
        assert np.max(np.abs(y - want)) <= np.max(TOL * np.linalg.norm(w, axis=1) * np.linalg.norm(x))
        # The resident tiled form decodes to the reference's weights exactly.
        out = torch.empty(rows * cols, dtype=torch.float32, device="cuda")
        _lib.call("vl_dequantize", qtype, rows, cols, acc.resident_matrix(m.cache_identity),
                  out.data_ptr(), torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), w.reshape(-1).view(np.uint32))
        # Second use: no upload.
        y2 = np.zeros(rows, np.float32)
        assert acc.matvec(m, x, y2)
        assert np.array_equal(y, y2)
        s = acc.stats()
        assert s["uploaded_bytes"] == enc.size and s["accelerated"] == 2
    finally:
        acc.close()
    assert gov.snapshot()["reserved"][KIND_VRAM] == 0
    assert gov.snapshot()["reserved"][KIND_STAGING] == 0


def test_eviction_and_reupload_on_device(gov, oracle):
    rng = np.random.Generator(np.random.PCG64(9))
    mats = [random_matrix(rng, IQ2_XXS, 64, 1024, 0.01) for _ in range(3)]
    x = rng.standard_normal(1024).astype(np.float32)
    per = 64 * 4 * 66  # tiled bytes of one 64 x 1024 IQ2_XXS matrix
    acc = Accelerator(gov, staging_bytes=256 * 1024, minimum_free_vram_after=0,
                      maximum_resident_bytes=2 * per)
    try:
        for rounds in range(2):
            for i, enc in enumerate(mats):
                y = np.zeros(64, np.float32)
                assert acc.matvec(PackedMatrix(IQ2_XXS, 64, 1024, enc, cache_identity=i + 1), x, y)
                assert within(y, oracle.dequantize(IQ2_XXS, enc, 64 * 1024).reshape(64, 1024), x)
        s = acc.stats()
        assert s["resident_matrices"] == 2 and s["evicted"] == 4
    finally:
        acc.close()


def test_non_finite_input_is_refused(gov):
    rng = np.random.Generator(np.random.PCG64(3))
    enc = random_matrix(rng, Q8_0, 32, 256, 0.01)
    acc = Accelerator(gov, staging_bytes=64 * 1024, minimum_free_vram_after=0)
    try:
        x = np.ones(256, np.float32)
        x[7] = np.inf
        y = np.full(32, 5.0, np.float32)
        with pytest.raises(VlError) as e:
            acc.matvec(PackedMatrix(Q8_0, 32, 256, enc, cache_identity=5), x, y)
        assert e.value.name == "invalid_argument"
        assert np.all(y == 5.0)
    finally:
        acc.close()


def test_governed_buffers(gov):
    before = gov.snapshot()["reserved"]
    dev = Buffer(gov, KIND_VRAM, 4 * MiB)
    pin = Buffer(gov, KIND_STAGING, 1 * MiB)
    assert dev.ptr and pin.ptr and dev.nbytes == 4 * MiB
    t = torch.zeros(1, device="cuda")  # the device is usable alongside
    snap = gov.snapshot()["reserved"]
    assert snap[KIND_VRAM] == before[KIND_VRAM] + 4 * MiB
    assert snap[KIND_STAGING] == before[KIND_STAGING] + 1 * MiB
    dev.free()
    pin.free()
    assert gov.snapshot()["reserved"] == before
    with pytest.raises(VlError) as e:   # the free-memory floor refuses
        Buffer(gov, KIND_VRAM, 1 * MiB, min_free_after=1 << 50)
    assert e.value.name == "resource_exhausted"
    assert gov.snapshot()["reserved"] == before
    del t


def test_gpu_probe_reports_the_device_and_a_policy_limit():
    """The GPU probe (GpuInfo from the HIP runtime) and the runtime policy's VRAM limit from it."""
    from vastloom_amd.accel import gpu_probe, vram_hard_limit
    info = gpu_probe(0)
    print(f"[gpu probe] {info}", flush=True)
    assert info.backend == "hip" and info.name and info.arch.startswith("gfx")
    assert int(info.driver_version) > 0
    assert info.compute_units > 0
    assert 0 < info.free_vram_bytes <= info.total_vram_bytes
    assert info.temperature_celsius is None and info.power_limit_watts is None
    limit = vram_hard_limit(info.total_vram_bytes, info.free_vram_bytes)
    assert 0 < limit <= min(info.total_vram_bytes * 4 // 5, info.free_vram_bytes - GiB)
    with pytest.raises(VlError):
        gpu_probe(1 << 20)
