"""Every kernel the library ships compiles without register spills.

A spill puts per-lane scratch (private memory) traffic inside the hot loops;
the compiler reports it as ScratchSize in its kernel-resource-usage remarks.
This compiles each source of ferret_amd/build.py for gfx950 (device code only,
into a scratch directory) and fails on any kernel with scratch use, naming it.
CPU-only: hipcc cross-compiles without a GPU.
"""
import shutil

import pytest

from ferret_amd import build

pytestmark = pytest.mark.skipif(shutil.which("hipcc") is None and not __import__("os").path.exists(
    "/opt/rocm/bin/hipcc"), reason="hipcc not installed")


@pytest.fixture(scope="module")
def usage():
    return build.resource_usage()


def test_every_source_reports_its_kernels(usage):
    # the remarks were parsed: dozens of kernel instances, each with its fields
    assert len(usage) >= 50
    for name, f in usage.items():
        assert {"vgpr", "sgpr", "scratch", "vgpr_spill", "sgpr_spill", "occupancy"} <= set(f), name


def test_no_kernel_spills(usage):
    spilling = {name: (f["scratch"], f["vgpr_spill"], f["sgpr_spill"]) for name, f in usage.items()
                if f["scratch"] > 0 or f["vgpr_spill"] > 0 or f["sgpr_spill"] > 0}
    assert not spilling, f"kernels with spills (scratch B/lane, VGPRs, SGPRs): {spilling}"


def test_hot_kernels_keep_their_occupancy(usage):
    # the large-M square kernel holds two waves per SIMD (8 waves per work-group)
    sq = [f for name, f in usage.items() if "fp8_square_kernel" in name]
    assert len(sq) == 2
    assert all(f["occupancy"] >= 2 for f in sq)
