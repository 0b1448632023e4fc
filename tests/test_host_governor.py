"""The native Safety Governor against the reference's own Governor test
(tests/test_main.cpp:8659-8727) and the try_reserve rules of
src/safety/resource_governor.cpp:64-105. Pure host code: runs without a GPU."""

from __future__ import annotations

import pytest

from vastloom_amd.accel import (KIND_RAM, KIND_SCRATCH, KIND_STAGING, KIND_VRAM, Buffer,
                                Governor, VlError, default_limits)

MiB, GiB = 1 << 20, 1 << 30


def limits(**kw):
    return default_limits(**kw)


def refused(fn, *args, code="resource_exhausted"):
    with pytest.raises(VlError) as e:
        fn(*args)
    assert e.value.name == code, str(e.value)


def test_reference_budget_release_and_pressure_sequence():
    g = Governor(limits(ram_hard_limit=8 * GiB, vram_hard_limit=4 * GiB,
                        staging_hard_limit=1 * GiB, scratch_hard_limit=2 * GiB,
                        minimum_system_ram_available=2 * GiB,
                        minimum_storage_available=20 * GiB, recovery_samples=2))
    first = g.try_reserve(KIND_RAM, 6 * GiB, "first")
    refused(g.try_reserve, KIND_RAM, 3 * GiB, "oversubscribe")
    g.release(first)
    g.try_reserve(KIND_RAM, 3 * GiB, "after-release")
    assert g.update_pressure(400 * MiB, 2 * GiB, 100 * GiB) == "emergency"
    refused(g.try_reserve, KIND_RAM, 1, "in-emergency")
    g.update_pressure(8 * GiB, 2 * GiB, 100 * GiB)
    assert g.update_pressure(8 * GiB, 2 * GiB, 100 * GiB) == "critical"


def test_reference_aggregate_host_budget():
    g = Governor(limits(host_memory_hard_limit=10 * MiB, ram_hard_limit=8 * MiB,
                        vram_hard_limit=8 * MiB, staging_hard_limit=4 * MiB,
                        scratch_hard_limit=4 * MiB, minimum_system_ram_available=1 * MiB,
                        minimum_storage_available=1 * MiB))
    g.try_reserve(KIND_RAM, 8 * MiB, "aggregate-ram")
    refused(g.try_reserve, KIND_STAGING, 3 * MiB, "aggregate-overflow")
    staging = g.try_reserve(KIND_STAGING, 2 * MiB, "aggregate-staging")
    refused(g.try_reserve, KIND_SCRATCH, 1, "aggregate-full")
    g.try_reserve(KIND_VRAM, 8 * MiB, "separate-vram-tier")
    snap = g.snapshot()
    assert snap["reserved"][KIND_RAM] == 8 * MiB and snap["reserved"][KIND_STAGING] == 2 * MiB
    g.release(staging)
    g.try_reserve(KIND_SCRATCH, 1 * MiB, "aggregate-scratch")


def test_reference_aggregate_pressure_state():
    g = Governor(limits(host_memory_hard_limit=10 * MiB, ram_hard_limit=10 * MiB,
                        vram_hard_limit=8 * MiB, staging_hard_limit=10 * MiB,
                        scratch_hard_limit=10 * MiB, minimum_system_ram_available=1 * MiB,
                        minimum_storage_available=1 * MiB))
    g.try_reserve(KIND_RAM, 8 * MiB, "pressure-ram")
    g.try_reserve(KIND_STAGING, 1 * MiB, "pressure-staging")
    assert g.update_pressure(10 * GiB, 10 * GiB, 10 * GiB) == "pressure"


def test_try_reserve_rules():
    g = Governor(limits(vram_hard_limit=100))
    refused(g.try_reserve, KIND_VRAM, 0, "zero", code="invalid_argument")
    refused(g.try_reserve, KIND_RAM, 1, "zero-budget")          # limit 0 refuses
    refused(g.try_reserve, KIND_VRAM, 101, "over")
    a = g.try_reserve(KIND_VRAM, 60, "a")
    refused(g.try_reserve, KIND_VRAM, 41, "b")
    b = g.try_reserve(KIND_VRAM, 40, "b")
    assert g.snapshot()["reserved"][KIND_VRAM] == 100
    g.release(a)
    g.release(b)
    assert g.snapshot()["reserved"][KIND_VRAM] == 0
    refused(g.release, b, code="not_found")


def test_abandon_keeps_bytes_charged():
    g = Governor(limits(vram_hard_limit=100))
    a = g.try_reserve(KIND_VRAM, 70, "leaked")
    g.abandon(a)
    assert g.snapshot()["reserved"][KIND_VRAM] == 70
    refused(g.try_reserve, KIND_VRAM, 31, "after-abandon")
    refused(g.release, a, code="not_found")


def test_recovery_steps_down_one_state_per_samples():
    g = Governor(limits(ram_hard_limit=1 * GiB, minimum_system_ram_available=2 * GiB,
                        minimum_storage_available=1 * GiB, recovery_samples=2))
    assert g.update_pressure(1 * GiB, 0, 10 * GiB) == "critical"
    assert g.update_pressure(64 * GiB, 0, 10 * GiB) == "critical"
    assert g.update_pressure(64 * GiB, 0, 10 * GiB) == "pressure"
    assert g.update_pressure(64 * GiB, 0, 10 * GiB) == "pressure"
    assert g.update_pressure(64 * GiB, 0, 10 * GiB) == "normal"
    g.try_reserve(KIND_RAM, 1, "recovered")


def test_buffer_refusals_before_any_device_call():
    g = Governor(limits(vram_hard_limit=1 * MiB, staging_hard_limit=1 * MiB))
    refused(Buffer, g, KIND_VRAM, 2 * MiB)                          # the Governor refuses
    refused(Buffer, g, KIND_VRAM, 0, code="invalid_argument")
    refused(Buffer, g, KIND_RAM, 1024, code="invalid_argument")   # not a device/pinned kind
    with pytest.raises(VlError):
        Buffer(g, KIND_VRAM, 1024, tag="")
    assert g.snapshot()["reserved"] == [0, 0, 0, 0]


def test_vram_hard_limit_follows_the_runtime_policy():
    """min(80 % of total, free - 1 GiB) above 1 GiB free, else 0
    (src/safety/runtime_policy.cpp:137-141; percentage() at src/core/bytes.cpp:99-107). The
    expected values use exact rationals (the double 0.80 as a fraction); each case's product lies
    far from an integer, so the reference's long double rounding cannot change its truncation."""
    from fractions import Fraction

    from vastloom_amd.accel import vram_hard_limit

    def expected(total, free):
        if free <= GiB:
            return 0
        return min(int(Fraction(total) * Fraction(0.80)), free - GiB)

    cases = [(288 * GiB, 287 * GiB), (288 * GiB, 10 * GiB), (288 * GiB, GiB + 1), (288 * GiB, GiB),
             (288 * GiB, 0), (80_000_000_000, 79_000_000_000), (24 * GiB, 23 * GiB + 7),
             (17, 2 * GiB), ((1 << 64) - 1, (1 << 64) - 1)]
    for total, free in cases:
        assert vram_hard_limit(total, free) == expected(total, free), (total, free)
    assert vram_hard_limit(288 * GiB, 287 * GiB) == 247_390_116_249  # floor(0.8 * 288 GiB)
    assert vram_hard_limit(288 * GiB, 10 * GiB) == 9 * GiB
    assert vram_hard_limit(288 * GiB, GiB) == 0
