"""The matvec accelerator's host logic through a fake device backend (the test seam of
vl_accel_create, like the reference's CudaDriver::from_backend_for_testing): declines, residency
by identity, eviction order, Governor accounting and failure handling. Runs without a GPU; the
fake backend multiplies with the oracle, so accelerated outputs are checked too.

Follows the reference's own accelerator test (tests/test_cuda_driver.cpp:713-790) and the
ensure_resident/matvec contract of src/cuda/cuda_matvec_accelerator.cpp:102-314."""

from __future__ import annotations

import ctypes as C
from collections import Counter

import numpy as np
import pytest

from oracle.oracle import IQ2_XXS, Q8_0
from vastloom_amd import _lib
from vastloom_amd.accel import (KIND_STAGING, KIND_VRAM, Accelerator, Governor, PackedMatrix,
                                VlError, default_limits)
from vastloom_amd.workloads import random_matrix

MiB = 1 << 20
STAGING = 8192
Q8_1x32_TILED = 32 * 34  # one Q8_0 row padded to a 32-row tile


class FakeBackend:
    """Host memory stands in for the device; matvec runs the oracle."""

    def __init__(self, oracle, free_bytes: int = 1 << 40):
        self.oracle = oracle
        self.free_bytes = free_bytes
        self.mem: dict[int, C.Array] = {}
        self.uploaded: dict[int, tuple[int, int, int, bytes]] = {}
        self.calls = Counter()
        self.fail_release = False
        self.fail_upload = False
        self.fail_allocate = False
        self.c = _lib.AccelBackend(
            None, _lib.FREE_MEMORY_FN(self._free_memory), _lib.ALLOCATE_FN(self._allocate),
            _lib.BACKEND_RELEASE_FN(self._release), _lib.UPLOAD_FN(self._upload),
            _lib.IO_BYTES_FN(self._io_bytes), _lib.MATVEC_FN(self._matvec))

    def _free_memory(self, ctx, device, out):
        out[0] = self.free_bytes
        return 0

    def _allocate(self, ctx, kind, device, nbytes, out):
        self.calls["allocate"] += 1
        if self.fail_allocate:
            return 9
        buf = (C.c_uint8 * nbytes)()
        addr = C.addressof(buf)
        self.mem[addr] = buf
        if kind == KIND_VRAM:
            self.free_bytes -= nbytes
        out[0] = addr
        return 0

    def _release(self, ctx, kind, ptr):
        self.calls["release"] += 1
        if self.fail_release:
            return 10
        buf = self.mem.pop(ptr, None)
        if buf is not None and kind == KIND_VRAM:
            self.free_bytes += len(buf)
        self.uploaded.pop(ptr, None)
        return 0

    def _upload(self, ctx, qtype, rows, cols, gguf, tiled, staging, scratch, staging_bytes):
        self.calls["upload"] += 1
        if self.fail_upload:
            return 5
        be, bb = {Q8_0: (32, 34), IQ2_XXS: (256, 66)}[qtype]
        self.uploaded[tiled] = (qtype, rows, cols, C.string_at(gguf, rows * (cols // be) * bb))
        return 0

    def _io_bytes(self, ctx, qtype, rows, cols, out):
        out[0] = 4 * (rows + cols) + 256
        return 0

    def _matvec(self, ctx, qtype, rows, cols, tiled, x, y, io, io_bytes):
        self.calls["matvec"] += 1
        try:
            t, r, c, data = self.uploaded[tiled]
            xv = np.ctypeslib.as_array(C.cast(x, C.POINTER(C.c_float)), shape=(c,)).copy()
            out = self.oracle.matvec(t, np.frombuffer(data, np.uint8), r, c, xv)
            C.memmove(y, out.astype(np.float32).ctypes.data, 4 * r)
            return 0
        except Exception:
            return 10


@pytest.fixture
def fake(oracle):
    return FakeBackend(oracle)


def governor(vram=64 * MiB, staging=16 * MiB):
    return Governor(default_limits(vram_hard_limit=vram, staging_hard_limit=staging))


def make(g, fake, **opt):
    opt.setdefault("staging_bytes", STAGING)
    opt.setdefault("minimum_free_vram_after", 0)
    return Accelerator(g, backend=fake.c, **opt)


def q8(identity=0, recurring=False, qtype=Q8_0, rows=1, cols=32):
    return PackedMatrix(qtype, rows, cols, np.zeros(rows * cols // 32 * 34, np.uint8),
                        cache_identity=identity, recurring=recurring)


def test_reference_placement_refusals(fake):
    g = governor()
    x, y = np.full(32, 0.25, np.float32), np.zeros(1, np.float32)
    acc = make(g, fake, experts_only=1, maximum_resident_bytes=8 * MiB)
    assert not acc.matvec(q8(11, recurring=True), x, y)
    s = acc.stats()
    assert (s["offered"], s["declined_recurring"], s["declined"], s["accelerated"]) == (1, 1, 1, 0)

    acc = make(g, fake, maximum_resident_bytes=8 * MiB)
    assert not acc.matvec(q8(0), x, y)                       # no identity: do not cache
    assert acc.stats()["declined"] == 1

    acc = make(g, fake, maximum_resident_bytes=8 * MiB)
    unsupported = PackedMatrix(999, 1, 32, np.zeros(0, np.uint8), cache_identity=12)
    assert not acc.matvec(unsupported, x, y)
    assert acc.stats()["declined"] == 1 and acc.stats()["declined_by_type"] == {999: 1}

    acc = make(g, fake, maximum_resident_bytes=1)
    assert not acc.matvec(q8(13), x, y)
    assert acc.stats()["declined"] == 1 and acc.stats()["resident_matrices"] == 0
    assert np.all(y == 0)                                    # declines leave output untouched


def test_span_and_payload_mismatches_decline(fake):
    acc = make(governor(), fake)
    y = np.zeros(1, np.float32)
    assert not acc.matvec(q8(1), np.zeros(31, np.float32), y)          # input != storage cols
    assert not acc.matvec(q8(1), np.zeros(32, np.float32), np.zeros(2, np.float32))
    short = PackedMatrix(Q8_0, 1, 32, np.zeros(33, np.uint8), cache_identity=2)
    assert not acc.matvec(short, np.zeros(32, np.float32), y)          # payload size mismatch
    ragged = PackedMatrix(Q8_0, 1, 48, np.zeros(51, np.uint8), cache_identity=3)
    assert not acc.matvec(ragged, np.zeros(48, np.float32), y)         # not whole blocks
    assert acc.stats()["declined"] == 4 and fake.calls["upload"] == 0


def test_accelerated_output_and_residency_reuse(fake, oracle):
    rng = np.random.Generator(np.random.PCG64(5))
    enc = random_matrix(rng, IQ2_XXS, 40, 512, 0.01)
    m = PackedMatrix(IQ2_XXS, 40, 512, enc, cache_identity=77)
    x = rng.standard_normal(512).astype(np.float32)
    acc = make(governor(), fake)
    for _ in range(3):
        y = np.zeros(40, np.float32)
        assert acc.matvec(m, x, y)
        assert np.array_equal(y, oracle.matvec(IQ2_XXS, enc, 40, 512, x))
    s = acc.stats()
    assert fake.calls["upload"] == 1 and s["uploaded_bytes"] == enc.size
    assert (s["offered"], s["accelerated"], s["resident_matrices"]) == (3, 3, 1)
    assert acc.holds(77) and not acc.holds(78) and not acc.holds(0)


def test_eviction_prefers_non_recurring_then_least_recent(fake):
    acc = make(governor(), fake, maximum_resident_bytes=3 * Q8_1x32_TILED)
    x, y = np.zeros(32, np.float32), np.zeros(1, np.float32)
    assert acc.matvec(q8(1, recurring=True), x, y)
    assert acc.matvec(q8(2), x, y)
    assert acc.matvec(q8(3), x, y)
    assert acc.matvec(q8(2), x, y)           # 2 is now more recent than 3
    assert acc.matvec(q8(4), x, y)           # evicts 3: not recurring, least recent
    assert [acc.holds(i) for i in (1, 2, 3, 4)] == [True, True, False, True]
    assert acc.matvec(q8(5, recurring=True), x, y)   # evicts 2 (the only non-recurring left but 4)
    assert acc.holds(1) and acc.holds(5) and acc.stats()["evicted"] == 2


def test_eviction_among_recurring_takes_least_recent(fake):
    acc = make(governor(), fake, maximum_resident_bytes=2 * Q8_1x32_TILED)
    x, y = np.zeros(32, np.float32), np.zeros(1, np.float32)
    assert acc.matvec(q8(1, recurring=True), x, y)
    assert acc.matvec(q8(2, recurring=True), x, y)
    assert acc.matvec(q8(1, recurring=True), x, y)    # 1 is now more recent than 2
    assert acc.matvec(q8(3, recurring=True), x, y)    # only recurring matrices: evicts 2
    assert [acc.holds(i) for i in (1, 2, 3)] == [True, False, True]
    assert acc.matvec(q8(4), x, y)                    # a non-recurring newcomer evicts 1
    assert [acc.holds(i) for i in (1, 3, 4)] == [False, True, True]
    assert acc.stats()["evicted"] == 2 and acc.stats()["resident_matrices"] == 2


def test_matrix_count_ceiling(fake):
    acc = make(governor(), fake, maximum_matrices=2)
    x, y = np.zeros(32, np.float32), np.zeros(1, np.float32)
    for i in (1, 2, 3):
        assert acc.matvec(q8(i), x, y)
    assert acc.stats()["resident_matrices"] == 2 and not acc.holds(1)


def test_governor_refusal_declines_and_accounts(fake):
    # Room for the scratch slots and one resident matrix, not two.
    g = governor(vram=STAGING + Q8_1x32_TILED + 4 * 33 + 256 + 100)
    acc = make(g, fake)
    x, y = np.zeros(32, np.float32), np.zeros(1, np.float32)
    assert acc.matvec(q8(1), x, y)
    assert not acc.matvec(q8(2), x, y)
    assert acc.stats()["declined"] == 1 and not acc.holds(2)
    acc.close()
    assert g.snapshot()["reserved"] == [0, 0, 0, 0]


def test_free_memory_floor_declines(fake):
    fake.free_bytes = STAGING + 3000         # the scratch slots leave 3000 B free
    acc = make(governor(), fake, minimum_free_vram_after=2048)
    x, y = np.zeros(32, np.float32), np.zeros(1, np.float32)
    assert not acc.matvec(q8(1), x, y)       # 1088 B would leave less than the 2 KiB floor


def test_allocation_failure_declines(fake):
    acc = make(governor(), fake)
    fake.fail_allocate = True
    assert not acc.matvec(q8(1), np.zeros(32, np.float32), np.zeros(1, np.float32))


def test_upload_failure_is_an_error_and_releases(fake):
    g = governor()
    acc = make(g, fake)
    before = g.snapshot()["reserved"][KIND_VRAM]
    fake.fail_upload = True
    with pytest.raises(VlError):
        acc.matvec(q8(1), np.zeros(32, np.float32), np.zeros(1, np.float32))
    assert not acc.holds(1) and g.snapshot()["reserved"][KIND_VRAM] == before


def test_release_failure_keeps_bytes_charged(fake):
    g = governor()
    acc = make(g, fake, maximum_resident_bytes=Q8_1x32_TILED)
    x, y = np.zeros(32, np.float32), np.zeros(1, np.float32)
    assert acc.matvec(q8(1), x, y)
    charged = g.snapshot()["reserved"][KIND_VRAM]
    fake.fail_release = True
    with pytest.raises(VlError):
        acc.matvec(q8(2), x, y)              # evicting 1 fails to free its memory
    assert not acc.holds(1)
    assert g.snapshot()["reserved"][KIND_VRAM] == charged   # abandoned, still charged


def test_staging_is_reserved_and_returned(fake):
    g = governor()
    acc = make(g, fake, staging_bytes=64 * 1024)
    snap = g.snapshot()["reserved"]
    assert snap[KIND_STAGING] == 64 * 1024 and snap[KIND_VRAM] == 64 * 1024
    acc.close()
    assert g.snapshot()["reserved"] == [0, 0, 0, 0]


def test_staging_refused_by_governor_fails_create(fake):
    with pytest.raises(VlError) as e:
        make(governor(staging=1024), fake)
    assert e.value.name == "resource_exhausted"
